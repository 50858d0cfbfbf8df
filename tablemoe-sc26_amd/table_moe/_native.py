"""ctypes binding of libtablemoe_hip.so (the C ABI in include/tablemoe.h).

The library is loaded lazily on first use.  torch is imported first so the
library's libamdhip64.so.7 dependency resolves to the HIP runtime torch has
already loaded: torch streams and device pointers are then valid in our
kernels.  There is no fallback: a missing library or a non-HIP tensor raises.
"""

from __future__ import annotations

import ctypes as C
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libtablemoe_hip.so"

TM_OK, TM_EINVAL_SHAPE, TM_EINVAL_DTYPE, TM_EINVAL_ARG, TM_EHIP, TM_EWORKSPACE = range(6)
TM_DT_F32, TM_DT_F16, TM_DT_BF16 = 0, 1, 2
TM_CMP_GE, TM_CMP_GT = 0, 1
TM_METRIC_L2, TM_METRIC_DOT = 0, 1
TM_TARGET_ONE, TM_TARGET_ORIG_SUM, TM_TARGET_GIVEN = 0, 1, 2
TM_SCORE_MODEL, TM_SCORE_F32 = 0, 1
TM_LAYER_NO_COMBINE = 1
TM_PACK_GATE_UP, TM_PACK_DOWN = 0, 1
# tm_table_forward workspace: sync region size and the byte offset of the
# count of bounded waits that ran out (include/tablemoe.h)
TM_LAYER_SYNC_BYTES = 16384
TM_LAYER_SYNC_ERR_BYTE = 3584

_DTYPE_TAG = {torch.float32: TM_DT_F32, torch.float16: TM_DT_F16, torch.bfloat16: TM_DT_BF16}

i32, i64, f32, f64, vp, sz = C.c_int32, C.c_int64, C.c_float, C.c_double, C.c_void_p, C.c_size_t



class TableLayer(C.Structure):
    """Mirror of tm_table_layer (include/tablemoe.h)."""

    _fields_ = [("dtype", i32), ("metric", i32), ("dim", i32), ("hidden", i32), ("n_cent", i64), ("cents", vp),
                ("ld_c", i64), ("c_sqnorm", vp), ("values", vp), ("ld_v", i64), ("proj_vis", vp), ("bias_vis", vp),
                ("proj_txt", vp), ("bias_txt", vp), ("ps_h", i64), ("ps_d", i64)]


class LayerIO(C.Structure):
    """Mirror of tm_layer_io (include/tablemoe.h)."""

    _fields_ = [("n_tokens", i64), ("x", vp), ("ld_x", i64), ("is_vision", vp), ("router_logits", vp),
                ("ld_logits", i64), ("n_experts", i32), ("router_top_k", i32), ("n_nearest", i32),
                ("flags", i32), ("keep_rate", f64), ("slot_out", vp), ("so_b", i64), ("so_s", i64),
                ("residual", vp), ("ld_r", i64), ("out", vp), ("ld_o", i64), ("weights", vp), ("expert_ids", vp),
                ("q", vp), ("q_sqnorm", vp), ("dist", vp), ("idx", vp), ("keep", vp)]


# name -> (restype, argtypes); mirrors include/tablemoe.h
PROTOTYPES = {
    "tm_version": (C.c_int, []),
    "tm_status_string": (C.c_char_p, [C.c_int]),
    "tm_last_error": (C.c_char_p, []),
    "tm_topk_softmax": (C.c_int, [vp, i64, i32, i64, i32, i32, vp, vp, vp]),
    "tm_project_workspace_size": (sz, [i64, i32, i32]),
    "tm_project_packed_size": (sz, [i32, i32, i32]),
    "tm_project_pack": (C.c_int, [i32, vp, i32, i32, i64, i64, vp, sz, vp]),
    "tm_project": (C.c_int, [i32, vp, i64, i32, i64, vp, vp, vp, vp, vp, i64, i64, i32, i32, f32, vp, i64, vp, vp, sz,
                             vp]),
    "tm_search_gated": (C.c_int, [i32, vp, i64, i64, vp, i64, i64, i32, i64, i64, i64, vp, i32, i64, i64, vp, vp,
                                  i64, i64, i32, f32, f32, i32, vp, vp, i64, i64, vp]),
    "tm_search_hybrid_workspace_size": (sz, [i64, i32, i32]),
    "tm_search_hybrid": (C.c_int, [i32, vp, i64, i32, i64, vp, vp, vp, vp, vp, i64, i64, i32, vp, i64, i32, vp, i32,
                                   i64, vp, i64, i64, i64, i64, i64, vp, i32, i64, i64, i32, vp, vp, vp, vp, vp, i64,
                                   i64, vp, i64, vp, sz, vp]),
    "tm_fixed_keep_mask": (C.c_int, [i64, i32, i32, vp, vp]),
    "tm_expert_keep_mask_workspace_size": (sz, [i64, i32]),
    "tm_expert_keep_mask": (C.c_int, [vp, vp, vp, i64, i32, i32, f64, vp, vp, vp, sz, vp]),
    "tm_renormalize": (C.c_int, [i32, vp, i64, vp, i64, i64, i32, i32, vp, i64, vp, vp]),
    "tm_gather_rows": (C.c_int, [i32, vp, i64, i64, i32, i64, i64, i64, vp, vp, i32, vp, i64, vp, vp, i64, i64, vp]),
    "tm_slot_combine": (C.c_int, [i32, i64, i32, i32, vp, i64, vp, vp, i64, i64, vp, vp, vp, i64, vp, vp, i64, i64,
                                  i64, i64, i64, vp, vp, vp, vp, i64, i32, i64, i64, i32, vp, i64, vp, i64, vp]),
    "tm_online_update": (C.c_int, [i32, vp, i64, vp, i64, vp, i64, i64, vp, i64, i64, i32, i32, i64, i64, vp, vp,
                                   vp, vp]),
    "tm_centroid_sqnorms": (C.c_int, [i32, vp, i64, i32, i64, vp, vp]),
    "tm_search_global_workspace_size": (sz, [i64, i64, i32, i32]),
    "tm_search_global": (C.c_int, [i32, vp, i64, i64, vp, vp, i64, i64, vp, i32, i32, i32, vp, vp, vp, sz, vp]),
    "tm_keep_count": (i64, [i64, f64]),
    "tm_keep_select_workspace_size": (sz, [i64]),
    "tm_keep_select": (C.c_int, [vp, i64, i64, i64, vp, vp, sz, vp]),
    "tm_gather_combine": (C.c_int, [i32, i64, i32, vp, vp, i64, i64, vp, i64, i32, vp, i64, i64, vp, vp, i64, i32,
                                    vp, i64, vp, i64, vp]),
    "tm_gather_combine_ranked": (C.c_int, [i32, i64, i32, vp, i64, i64, vp, i64, i32, vp, i64, i64, vp, vp, vp, i64,
                                           vp, i64, i64, vp, vp]),
    "tm_decode_combine_update": (C.c_int, [i32, i32, i32, vp, vp, vp, i64, vp, vp, vp, vp, vp, i64, i64, i64, i64, i64,
                                           vp, vp, vp, vp, i64, i32, i64, i64, i32, vp, vp, vp, vp, vp, i64, vp]),
    "tm_importance_workspace_size": (sz, [i64, i32, i64]),
    "tm_last_query_importance": (C.c_int, [i32, vp, i64, i64, vp, i64, i64, i64, i64, i32, i32, i32, i64, f32, i32,
                                           vp, i64, i64, vp, i64, vp, sz, vp]),
    "tm_swiglu_workspace_size": (sz, [i64, i32, i32]),
    "tm_expert_swiglu": (C.c_int, [i32, vp, i64, i32, i64, vp, vp, vp, i32, vp, i64, vp, sz, vp]),
    "tm_expert_swiglu_add": (C.c_int, [i32, vp, i64, i32, i64, vp, vp, vp, i32, vp, i64, vp, i64, vp, sz, vp]),
    "tm_group_slots_tiles": (i64, [i64, i32]),
    "tm_group_slots": (C.c_int, [vp, i64, i32, i64, vp, i64, i64, i32, i64, i64, vp, vp, vp, vp, vp]),
    "tm_group_slots_workspace_size": (sz, [i64, i32, i32]),
    "tm_group_slots_ws": (C.c_int, [vp, i64, i32, i64, vp, i64, i64, i32, i64, i64, vp, vp, vp, vp, vp, sz, vp]),
    "tm_grouped_swiglu": (C.c_int, [i32, vp, i64, i32, i32, i32, vp, vp, vp, i64, vp, vp, vp, vp, vp, vp, sz, vp]),
    "tm_grouped_swiglu_packed": (C.c_int, [i32, vp, i64, i32, i32, i32, vp, vp, vp, i64, vp, vp, vp, vp, vp, vp, sz,
                                           vp]),
    "tm_expert_pack_weights": (C.c_int, [i32, vp, i32, i32, i32, i32, vp, vp]),
    "tm_grouped_swiglu_packed_workspace_size": (sz, [i64, i32, i32, i32]),
    "tm_expert_swiglu_packed": (C.c_int, [i32, vp, i64, i32, i64, vp, vp, vp, i32, vp, i64, vp, i64, vp, sz, vp]),
    "tm_struct_size": (sz, [i32]),
    "tm_table_forward_workspace_size": (sz, [C.POINTER(TableLayer), i64, i32]),
    "tm_table_forward": (C.c_int, [C.POINTER(TableLayer), C.POINTER(LayerIO), vp, sz, vp, vp]),
    "tm_table_forward_noalloc": (C.c_int, [C.POINTER(TableLayer), C.POINTER(LayerIO), vp]),
}

# tm_table_forward_noalloc's static scratch (TM_NOALLOC_SCRATCH_BYTES, include/tablemoe.h)
TM_NOALLOC_SCRATCH_BYTES = 16 << 20

_lock = threading.Lock()
_lib = None


class NativeLibraryMissing(RuntimeError):
    pass


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load (once) and return the library; raise if it is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise NativeLibraryMissing(
                f"{p} is not built; run `python tablemoe-sc26_amd/build_lib.py` (or __graft_entry__.build())"
            )
        lib = C.CDLL(str(p))
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        for which, struct in ((0, TableLayer), (1, LayerIO)):
            if lib.tm_struct_size(which) != C.sizeof(struct):
                raise RuntimeError(f"{struct.__name__} mirror ({C.sizeof(struct)} bytes) does not match the library "
                                   f"({lib.tm_struct_size(which)} bytes)")
        _lib = lib
        return lib


def lib() -> C.CDLL:
    return _lib if _lib is not None else load()


def check(status: int, what: str) -> None:
    if status == TM_OK:
        return
    L = lib()
    msg = (L.tm_last_error() or b"").decode(errors="replace")
    name = (L.tm_status_string(status) or b"?").decode()
    if status == TM_EHIP:
        raise RuntimeError(f"{what}: {name}: {msg}")
    raise ValueError(f"{what}: {name}: {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def dtype_tag(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_TAG[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


def require_hip(*tensors: torch.Tensor | None) -> torch.device:
    """All given tensors must live on the same HIP device; return it."""
    first = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                f"table_moe kernels run on a HIP device only; got a tensor on {t.device} "
                "(there is no CPU fallback)"
            )
        if first is None:
            first, idx = t, t.get_device()
        elif t.get_device() != idx:
            raise ValueError(f"tensors on different devices: {first.device} and {t.device}")
    if first is None:
        raise ValueError("no tensor given")
    return first.device


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


# the current stream's handle without building a torch.cuda.Stream object
# (a few microseconds per call on the eager decode path)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(device: torch.device) -> int:
    if _raw_stream is not None and device.index is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def mask_bytes(mask: torch.Tensor, device: torch.device) -> torch.Tensor:
    """A token mask as contiguous bytes on ``device``: the tensor itself when
    it already is a contiguous bool tensor there, else a bool copy."""
    if mask.dtype == torch.bool and mask.is_cuda and mask.is_contiguous() and mask.get_device() == device.index:
        return mask
    return mask.reshape(-1).to(device=device, dtype=torch.bool).contiguous()


def as_u8(mask: torch.Tensor) -> torch.Tensor:
    """A bool/uint8 mask viewed as bytes (no copy for torch.bool)."""
    if mask.dtype == torch.bool:
        return mask.view(torch.uint8) if mask.is_contiguous() or mask.dim() == 0 else mask.to(torch.uint8)
    if mask.dtype == torch.uint8:
        return mask
    return (mask != 0).to(torch.uint8)


def pack_projection(proj: torch.Tensor, bias: torch.Tensor) -> torch.Tensor | None:
    """The packed device layout of a [hidden, dim] projection (tm_project_pack),
    or None when the packed fast path does not apply (fp32, unsupported dim or
    hidden, unaligned bias); callers then keep a strided layout."""
    require_hip(proj, bias)
    hidden, dim = proj.shape
    tag = dtype_tag(proj.dtype)
    nbytes = lib().tm_project_packed_size(hidden, dim, tag)
    if nbytes == 0 or hidden % 8 != 0 or bias.data_ptr() % 16 != 0:
        return None
    out = torch.empty(nbytes, dtype=torch.uint8, device=proj.device)
    call("tm_project_pack", tag, ptr(proj), hidden, dim, proj.stride(0), proj.stride(1), ptr(out), nbytes,
         stream(proj.device))
    return out


def exported_symbols() -> list[str]:
    return [n for n in PROTOTYPES]
