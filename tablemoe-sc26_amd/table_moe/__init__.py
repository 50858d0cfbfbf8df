"""TableMoE table-search path on MI355X (gfx950).

Drop-in replacements for the reference's ``table_moe.cache_engine``,
``table_moe.skip`` and ``table_moe.ops.qwen_topk_softmax`` (same module paths,
class names, method names, argument meaning and error types), whose compute
runs in hand-written HIP kernels behind the C ABI of ``include/tablemoe.h``
(``table_moe/_lib/libtablemoe_hip.so``).  Plus ``cache_engine.global_table``
for the single-global-table configuration.

Import-light: submodules load torch; the native library is loaded on first use.
"""

__version__ = "0.1.0"
