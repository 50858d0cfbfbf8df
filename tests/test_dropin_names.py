"""The drop-in boundary on the host: every name the reference's unchanged
modules import from the files this package replaces exists here, and the
replacement files only import each other (plus torch/numpy), so they can be
copied over the reference's table_moe/ tree as an overlay (cache_engine/,
skip/, ops/, utils/modality.py and utils/importance.py, _native.py, _lib/).

The import list is transcribed from the reference:
  models/qwen3_vl_moe/cached_layers.py:5-13, hybrid_attention.py:11,
  builder.py:18-19, expert_wrapper.py:5, custom_layers.py:4-5;
  models/deepseek_vl2/deepseek_layers.py:4-11 and :326, deepseek_attention.py:28,
  builder.py:18-19; offload/expert_wrapper.py:4;
  cache_engine/test_search.py:6-8 (which also patches search.HAS_TRITON);
  skip/test_pruning.py:9; utils/__init__.py:1 (ModalityContext).
"""

import ast
import importlib
from pathlib import Path

import pytest

PKG = Path(__file__).resolve().parents[1] / "tablemoe-sc26_amd" / "table_moe"

# module (relative to table_moe) -> names imported from it by the reference's own files
HOOK_IMPORTS = {
    "ops": ["qwen_topk_softmax", "maybe_run_fp16_fused_expert"],
    "cache_engine": ["CacheConfig", "HybridStorageManager", "VectorSearchEngine", "HAS_TRITON",
                     "get_active_cache_config", "set_active_cache_config", "update_active_cache_config"],
    "cache_engine.config": ["CacheConfig", "set_active_cache_config"],
    "cache_engine.search": ["VectorSearchEngine", "HAS_TRITON"],
    "cache_engine.manager": ["HybridStorageManager"],
    "skip": ["build_decode_keep_mask", "build_fixed_keep_mask", "build_prefill_keep_mask",
             "renormalize_surviving_weights"],
    "utils.modality": ["ModalityContext"],
}

# the files the overlay copies into the reference's table_moe/ (relative paths)
OVERLAY = ["_native.py", "cache_engine/__init__.py", "cache_engine/config.py", "cache_engine/manager.py",
           "cache_engine/search.py", "cache_engine/table_file.py", "cache_engine/global_table.py",
           "skip/__init__.py", "skip/pruning.py", "ops/__init__.py", "ops/qwen_topk_softmax.py",
           "ops/fp16_fused_expert.py", "ops/grouped_expert.py", "utils/modality.py", "utils/importance.py"]

# modules of the reference tree the overlay may rely on (kept as they are)
KEPT = {"table_moe.utils"}


@pytest.mark.parametrize("module,names", sorted(HOOK_IMPORTS.items()))
def test_hook_imports_resolve(module, names):
    mod = importlib.import_module(f"table_moe.{module}")
    for name in names:
        assert hasattr(mod, name), f"table_moe.{module} lacks {name}"


def test_manager_and_engine_surface():
    """Methods and attributes the hooks call (cached_layers.py, deepseek_layers.py)."""
    from table_moe.cache_engine import HybridStorageManager, VectorSearchEngine

    for meth in ("search_prefill_offline", "search_prefill_offline_dot", "search_decode_offline",
                 "search_decode_offline_dot", "search_decode_hybrid", "search_decode_offline_bs1_into",
                 "search_decode_hybrid_bs1_into"):
        assert callable(getattr(VectorSearchEngine, meth)), meth
    for meth in ("gather_values", "gather_values_decode_bs1", "update_online_cache", "update_online_cache_bs1"):
        assert callable(getattr(HybridStorageManager, meth)), meth


def _module_of(path: Path) -> str:
    rel = path.relative_to(PKG.parent).with_suffix("")
    parts = list(rel.parts)
    if parts[-1] == "__init__":
        parts = parts[:-1]
    return ".".join(parts)


def test_overlay_files_import_only_each_other():
    """Every intra-package import of an overlay file resolves to another
    overlay file or to a module the reference tree keeps."""
    overlay_mods = {_module_of(PKG / f) for f in OVERLAY}
    for f in OVERLAY:
        path = PKG / f
        assert path.exists(), f
        pkg_parts = _module_of(path).split(".")
        if not path.name == "__init__.py":
            pkg_parts = pkg_parts[:-1]
        tree = ast.parse(path.read_text())
        for node in ast.walk(tree):
            if isinstance(node, ast.ImportFrom) and node.level > 0:
                base = pkg_parts[: len(pkg_parts) - (node.level - 1)]
                target = ".".join(base + ([node.module] if node.module else []))
                candidates = [target] + [f"{target}.{a.name}" for a in node.names]
                assert any(c in overlay_mods or c in KEPT for c in candidates), (f, target,
                                                                               [a.name for a in node.names])
            elif isinstance(node, ast.ImportFrom) and node.module and node.module.startswith("table_moe"):
                assert node.module in overlay_mods or node.module in KEPT, (f, node.module)
