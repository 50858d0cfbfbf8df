"""Process-global cache configuration.

Same keys, defaults, accessors and override environment variables as the
reference's ``CacheConfig`` (table_moe/cache_engine/config.py:12-74), because
the unchanged layer hooks and builders read and write these names.
"""

from __future__ import annotations

import os
from pathlib import Path

import torch

_PKG_ROOT = Path(__file__).resolve().parents[2]
_OFFLINE_ROOT = _PKG_ROOT / "offline_table" / "ds_fp16"
_BENCHMARK = "MMBench_DEV_EN_V11"


def _defaults() -> dict:
    return {
        "PCA_DIR": os.getenv(
            "DS_CACHE_PCA_DIR", str(_OFFLINE_ROOT / "clustering_results" / f"{_BENCHMARK}_LayerPCA_256")
        ),
        "CACHE_DIR": os.getenv(
            "DS_CACHE_DIR", str(_OFFLINE_ROOT / "offline_table" / f"{_BENCHMARK}_LayerPCA_256")
        ),
        "COMPRESSED_DIM": 64,
        "FIXED_K": 256,
        "KEEP_K": 3,
        "PREFILL_KEEP_K": 3,
        "DECODE_KEEP_K": 3,
        "KEEP_RATE": 0.6,
        "MODALITY_MAP": {"vision": 0, "text": 1},
        "ONLINE_CACHE_SIZE": 64,
        "ONLINE_TOP_K": 6,
        "ONLINE_MIN_LAYER_IDX": 1,
        "ONLINE_MAX_LAYER_IDX": 47,
        "MODEL_DTYPE": torch.bfloat16,
        "OFFLINE_COSINE_THRESHOLD_VISION": 0.6,
        "OFFLINE_COSINE_THRESHOLD_TEXT": 0.7,
        "OFFLINE_DOT_THRESHOLD": 0.0,
        "OFFLINE_COSINE_EPS": 1e-6,
    }


_ACTIVE = _defaults()


def set_active_cache_config(config):
    """Replace the active configuration by defaults updated with ``config``."""
    global _ACTIVE
    merged = _defaults()
    if config is not None:
        merged.update(config)
    _ACTIVE = merged


def update_active_cache_config(**kwargs):
    _ACTIVE.update(kwargs)


def get_active_cache_config():
    return dict(_ACTIVE)


class _ConfigView(type):
    """Class-attribute access to the active configuration dict."""

    def __getattr__(cls, name):
        try:
            return _ACTIVE[name]
        except KeyError:
            raise AttributeError(name) from None

    def __setattr__(cls, name, value):
        if name in _ACTIVE:
            _ACTIVE[name] = value
        else:
            super().__setattr__(name, value)


class CacheConfig(metaclass=_ConfigView):
    pass
