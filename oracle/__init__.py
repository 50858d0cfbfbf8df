"""CPU oracle for the TableMoE table-search path (TEST INFRASTRUCTURE ONLY).

This package restates, in numpy, the reference algorithm of every function on
the table-search hot path.  It is the checker, never the product: only the
files under ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it.  The product path (``table_moe`` in
``tablemoe-sc26_amd/``) never imports, calls or falls back to it.

Parity pinning status of each function is listed in the module docstring of
``oracle.tm_oracle``.
"""

from . import tm_oracle  # noqa: F401
