"""CPU checks of the C ABI: the library loads, exports every entry point that
include/tablemoe.h declares with the same arity as the ctypes prototypes, and
validates arguments before touching a device (no compute call needs a GPU)."""

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from table_moe import _native as N

HEADER = Path(__file__).resolve().parents[1] / "include" / "tablemoe.h"


def _declarations():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int|int64_t|size_t|const char \*)\s*\*?\s*(tm_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.S):
        args = m.group(2).strip()
        n = 0 if args in ("", "void") else len([a for a in args.split(",") if a.strip()])
        decls[m.group(1)] = n
    return decls


@pytest.fixture(scope="module")
def lib():
    return N.load()


def test_header_declares_all_prototypes():
    decls = _declarations()
    assert len(decls) >= 20
    assert set(decls) == set(N.PROTOTYPES), set(decls) ^ set(N.PROTOTYPES)
    for name, nargs in decls.items():
        assert len(N.PROTOTYPES[name][1]) == nargs, name


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(N.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    for name in _declarations():
        assert name in exported, name
        assert getattr(lib, name) is not None


def test_library_links_one_hip_runtime():
    out = subprocess.run(["readelf", "-d", str(N.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    needed = re.findall(r"NEEDED.*\[(.*)\]", out)
    hip = [n for n in needed if "amdhip64" in n]
    assert hip == ["libamdhip64.so.7"], needed  # resolves to the runtime torch already loaded


def test_status_strings(lib):
    assert lib.tm_version() >= 100
    assert lib.tm_status_string(N.TM_OK) == b"TM_OK"
    assert lib.tm_status_string(N.TM_EWORKSPACE) == b"TM_EWORKSPACE"


def test_keep_count_matches_reference_rule(lib):
    from oracle import tm_oracle as O

    for n in (0, 1, 2, 5, 32, 255, 256, 4096, 10007):
        for r in (0.0, 0.1, 0.25, 0.5, 0.6, 0.75, 0.9, 1.0):
            assert lib.tm_keep_count(n, r) == O.keep_count(n, r), (n, r)


def test_argument_validation_without_device(lib):
    # empty inputs are no-ops
    assert lib.tm_keep_select(None, 0, 1, 0, None, None, 0, None) == N.TM_OK
    assert lib.tm_project(N.TM_DT_BF16, None, 0, 2048, 2048, None, C.c_void_p(16), C.c_void_p(16), None, None,
                          1, 2048, 128, 0, 1e-6, C.c_void_p(16), 128, None, None, 0, None) == N.TM_OK
    assert lib.tm_project_workspace_size(4096, 2048, 128) == 4 * 4096 * 128 * 4  # 4-way split of hidden
    # bad sizes / enums / dtypes are rejected before any launch
    assert lib.tm_search_global(N.TM_DT_BF16, None, 10, 128, None, None, 100, 128, None, 128, 9, 0, None, None,
                                None, 0, None) == N.TM_EINVAL_SHAPE
    assert b"top_k 9" in lib.tm_last_error()
    assert lib.tm_search_global(7, None, 10, 128, None, None, 100, 128, None, 128, 1, 0, None, None,
                                None, 0, None) == N.TM_EINVAL_DTYPE
    assert lib.tm_search_gated(7, C.c_void_p(16), 4, 64, C.c_void_p(16), 8, 256, 64, 0, 0, 64, C.c_void_p(16), 8,
                               8, 1, None, None, 0, 0, 0, 0.6, 0.7, 0, C.c_void_p(16), C.c_void_p(16), 8, 1,
                               None) == N.TM_EINVAL_DTYPE
    assert lib.tm_search_gated(N.TM_DT_BF16, C.c_void_p(16), 4, 64, C.c_void_p(16), 8, 256, 64, 0, 0, 64,
                               C.c_void_p(16), 8, 8, 1, None, None, 0, 0, 0, 0.6, 0.7, 5, C.c_void_p(16),
                               C.c_void_p(16), 8, 1, None) == N.TM_EINVAL_ARG
    assert lib.tm_renormalize(N.TM_DT_F32, C.c_void_p(16), 8, C.c_void_p(16), 8, 4, 8, 9, None, 0,
                              C.c_void_p(16), None) == N.TM_EINVAL_ARG
    assert lib.tm_online_update(N.TM_DT_BF16, C.c_void_p(16), 8, C.c_void_p(16), 8, C.c_void_p(16), 64, 8, None, 0,
                                65, 8, 8, 0, 64, C.c_void_p(16), C.c_void_p(16), C.c_void_p(16),
                                None) == N.TM_EINVAL_SHAPE
    # workspace checks
    need = lib.tm_search_global_workspace_size(4096, 8192, 128, 1)
    assert need > 0
    assert lib.tm_search_global(N.TM_DT_BF16, C.c_void_p(16), 4096, 128, None, C.c_void_p(16), 8192, 128,
                                C.c_void_p(16), 128, 1, 0, C.c_void_p(16), C.c_void_p(16), C.c_void_p(16),
                                need - 1, None) == N.TM_EWORKSPACE
    assert lib.tm_expert_keep_mask_workspace_size(4096, 128) > 0
    # packed projection layout: ceil(hidden/32)*32 rows of dim 2-byte elements
    assert lib.tm_project_packed_size(2048, 128, N.TM_DT_BF16) == 2048 * 128 * 2
    assert lib.tm_project_packed_size(1000, 64, N.TM_DT_F16) == 1024 * 64 * 2
    assert lib.tm_project_packed_size(2048, 48, N.TM_DT_BF16) == 0
    assert lib.tm_project_packed_size(2048, 128, N.TM_DT_F32) == 0
    assert lib.tm_project_pack(N.TM_DT_BF16, C.c_void_p(16), 2048, 128, 128, 1, C.c_void_p(16), 100,
                               None) == N.TM_EWORKSPACE
    assert lib.tm_project_pack(N.TM_DT_F32, C.c_void_p(16), 2048, 128, 128, 1, C.c_void_p(16), 1 << 20,
                               None) == N.TM_EINVAL_DTYPE
    # packed expert weights: role, shape, overlap and dtype are checked before any launch
    assert lib.tm_expert_pack_weights(N.TM_DT_BF16, C.c_void_p(16), 4, 2560, 1536, 2, C.c_void_p(1 << 40),
                                      None) == N.TM_EINVAL_ARG
    assert lib.tm_expert_pack_weights(N.TM_DT_BF16, C.c_void_p(16), 4, 2500, 1536, N.TM_PACK_DOWN,
                                      C.c_void_p(1 << 40), None) == N.TM_EINVAL_SHAPE
    assert lib.tm_expert_pack_weights(N.TM_DT_BF16, C.c_void_p(1 << 20), 4, 256, 128, N.TM_PACK_GATE_UP,
                                      C.c_void_p((1 << 20) + 4096), None) == N.TM_EINVAL_ARG
    assert b"overlaps" in lib.tm_last_error()
    assert lib.tm_expert_pack_weights(N.TM_DT_F32, C.c_void_p(16), 4, 256, 128, N.TM_PACK_GATE_UP,
                                      C.c_void_p(1 << 40), None) == N.TM_EINVAL_DTYPE
    assert lib.tm_grouped_swiglu_packed(N.TM_DT_BF16, None, 2560, 2560, 1536, 64, None, None, None, 0, None, None,
                                        None, None, None, None, 0, None) == N.TM_OK  # no rows: no-op
    # the packed path's intermediate is whole 256-row tiles of the tile list
    assert lib.tm_grouped_swiglu_packed_workspace_size(24576, 1536, 64, N.TM_DT_BF16) == (96 + 64) * 256 * 1536 * 2
    assert lib.tm_swiglu_workspace_size(24576, 1536, N.TM_DT_BF16) == 24576 * 1536 * 2
    # the multi-workgroup grouping: one count row per 64 tokens, 0 (the one-workgroup kernel) outside its shapes
    assert lib.tm_group_slots_workspace_size(4096, 6, 64) == 64 * 64 * 4
    assert lib.tm_group_slots_workspace_size(8192, 8, 256) == 128 * 256 * 4
    for n_, k_, e_ in ((0, 6, 64), (8193, 6, 64), (4096, 9, 64), (4096, 6, 257), (4096, 6, 0)):
        assert lib.tm_group_slots_workspace_size(n_, k_, e_) == 0
    q = C.c_void_p(256)
    assert lib.tm_group_slots_ws(q, 4096, 6, 6, q, 6, 1, 64, 6 * 2560, 2560, q, q, q, q, q, 4096,
                                 None) == N.TM_EWORKSPACE
    # grouped rows are written in 16-byte pieces: output strides off a multiple of 8 elements are rejected
    p = C.c_void_p(256)
    assert lib.tm_group_slots(p, 16, 6, 6, p, 6, 1, 64, 6 * 2564, 2564, p, p, p, p, None) == N.TM_EINVAL_SHAPE
    assert b"multiples of 8" in lib.tm_last_error()
    assert lib.tm_group_slots(p, 16, 6, 6, p, 6, 1, 64, 6 * 2560 + 4, 2560, p, p, p, p, None) == N.TM_EINVAL_SHAPE



def test_ranked_limit_without_device(lib):
    """The ranked combine rejects a token count beyond its bound before any
    HIP call (each token's workgroup reads all n distances)."""
    p = C.c_void_p(256)
    assert lib.tm_gather_combine_ranked(N.TM_DT_BF16, 16385, 2048, p, 8 * 2048, 2048, p, 8, 8, p, 8192, 2048, p, p,
                                        p, 2048, p, 2048, 100, p, None) == N.TM_EINVAL_SHAPE
    assert b"16384" in lib.tm_last_error()


def test_noalloc_limit_without_device(lib):
    """tm_table_forward_noalloc rejects a layer whose workspace exceeds its
    static scratch before any HIP call."""
    t = N.TableLayer(dtype=N.TM_DT_BF16, metric=N.TM_METRIC_L2, dim=128, hidden=2048, n_cent=8192, ld_c=128,
                     ld_v=2048, ps_h=0, ps_d=0)
    io = N.LayerIO(n_tokens=4096, n_nearest=8, router_top_k=8, n_experts=128, keep_rate=0.6)
    assert lib.tm_table_forward_workspace_size(C.byref(t), 4096, 8) > N.TM_NOALLOC_SCRATCH_BYTES
    assert lib.tm_table_forward_noalloc(C.byref(t), C.byref(io), None) == N.TM_EWORKSPACE
    assert b"TM_NOALLOC_SCRATCH_BYTES" in lib.tm_last_error()
    io.n_tokens = 0
    assert lib.tm_table_forward_noalloc(C.byref(t), C.byref(io), None) == N.TM_OK
    assert lib.tm_table_forward_noalloc(None, C.byref(io), None) == N.TM_EINVAL_ARG
