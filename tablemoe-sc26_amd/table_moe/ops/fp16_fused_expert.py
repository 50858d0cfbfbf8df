"""The expert MLP of the recompute path on the matrix cores.

``maybe_run_fp16_fused_expert`` keeps the reference's entry point and
contract (table_moe/ops/fp16_fused_expert.py:223-257): ``owner`` has
``w1`` / ``w3`` / ``w2`` linear wrappers (gate, up, down) whose
``linear_module`` is a bias-free nn.Linear on the device; hidden states are a
contiguous 2-D tensor of at most ``TABLEMOE_FP16_FUSED_MAX_TOKENS`` rows
(default 1, as the reference); ``TABLEMOE_USE_FP16_FUSED_EXPERT=0`` disables
it.  When the call does not apply it returns None and the caller runs the
torch expert, as with the reference.  The result is
y = dtype(dtype(silu(dtype(x W1^T)) * (x W3^T)) W2^T) — the rounding points of
the reference's fused kernel (fp16_fused_moe_mlp.cu:107-274, SiLU-mul
epilogue fp16_epilogue_utils.h:51-125) — written into a buffer the owner keeps.
fp16 and bf16 both run (the reference's CUTLASS kernel is fp16 only);
hidden and intermediate sizes must be multiples of 128.  A missing native
library raises: there is no silent fallback.
"""

from __future__ import annotations

import os
import warnings

import torch

from .. import _native as N

_ENV_NAME = "TABLEMOE_USE_FP16_FUSED_EXPERT"
_MAX_TOKENS_ENV_NAME = "TABLEMOE_FP16_FUSED_MAX_TOKENS"
_WARNED = set()


def _env_enabled() -> bool:
    raw = os.getenv(_ENV_NAME)
    return raw is None or raw.strip().lower() not in {"0", "false", "off", "no"}


def _max_tokens() -> int:
    raw = os.getenv(_MAX_TOKENS_ENV_NAME)
    if raw is None:
        return 1
    try:
        value = int(raw)
    except ValueError:
        value = 0
    if value <= 0:
        if raw not in _WARNED:
            _WARNED.add(raw)
            warnings.warn(f"Invalid {_MAX_TOKENS_ENV_NAME}={raw!r}, falling back to 1.", RuntimeWarning, stacklevel=3)
        return 1
    return value


def _eligible_weight(linear_wrapper):
    linear_module = getattr(linear_wrapper, "linear_module", None)
    if linear_module is None or getattr(linear_module, "bias", None) is not None:
        return None
    w = linear_module.weight
    if w.device.type != "cuda" or w.dtype not in (torch.float16, torch.bfloat16) or not w.is_contiguous():
        return None
    return w


def expert_swiglu(hidden_states: torch.Tensor, w1: torch.Tensor, w3: torch.Tensor, w2: torch.Tensor,
                  out: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                  addend: torch.Tensor | None = None) -> torch.Tensor:
    """y = SwiGLU expert MLP of ``hidden_states`` [M, H] with nn.Linear weights
    w1, w3 [I, H] and w2 [H, I] (one tm_expert_swiglu call).  With ``addend``
    [M, H] (not overlapping ``out``): y = dtype(addend + MLP) in one rounding
    (tm_expert_swiglu_add), e.g. a DeepSeek layer's shared experts added to
    the residual stream."""
    dev = N.require_hip(hidden_states, w1, w3, w2)
    m, h = hidden_states.shape
    inter = w1.shape[0]
    if w1.shape != (inter, h) or w3.shape != (inter, h) or w2.shape != (h, inter):
        raise ValueError("expert_swiglu: w1/w3 must be [I, H] and w2 [H, I]")
    dt = hidden_states.dtype
    if out is None:
        out = torch.empty((m, h), dtype=dt, device=dev)
    nbytes = N.lib().tm_swiglu_workspace_size(m, inter, N.dtype_tag(dt))
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    if addend is None:
        N.call("tm_expert_swiglu", N.dtype_tag(dt), N.ptr(hidden_states), m, h, hidden_states.stride(0), N.ptr(w1),
               N.ptr(w3), N.ptr(w2), inter, N.ptr(out), out.stride(0), N.ptr(workspace), workspace.numel(),
               N.stream(dev))
    else:
        N.require_hip(addend)
        if addend.shape != (m, h) or addend.dtype != dt or addend.stride(-1) != 1:
            raise ValueError(f"expert_swiglu: addend must be [{m}, {h}] {dt} with unit stride along hidden")
        N.call("tm_expert_swiglu_add", N.dtype_tag(dt), N.ptr(hidden_states), m, h, hidden_states.stride(0),
               N.ptr(w1), N.ptr(w3), N.ptr(w2), inter, N.ptr(addend), addend.stride(0), N.ptr(out), out.stride(0),
               N.ptr(workspace), workspace.numel(), N.stream(dev))
    return out


def maybe_run_fp16_fused_expert(owner, hidden_states: torch.Tensor):
    if not _env_enabled():
        return None
    if hidden_states.device.type != "cuda" or hidden_states.dtype not in (torch.float16, torch.bfloat16):
        return None
    if hidden_states.ndim != 2 or not hidden_states.is_contiguous():
        return None
    if hidden_states.shape[0] <= 0 or hidden_states.shape[0] > _max_tokens():
        return None
    w1, w3, w2 = (_eligible_weight(getattr(owner, k, None)) for k in ("w1", "w3", "w2"))
    if w1 is None or w3 is None or w2 is None:
        return None
    if any(w.dtype != hidden_states.dtype for w in (w1, w3, w2)):
        return None
    h, inter = hidden_states.shape[1], w1.shape[0]
    if h % 128 or inter % 128 or w3.shape != w1.shape or w2.shape != (h, inter):
        return None
    out = getattr(owner, "_fp16_fused_output_buf", None)
    if out is None or out.shape != hidden_states.shape or out.dtype != hidden_states.dtype or out.device != hidden_states.device:
        out = torch.empty_like(hidden_states)
        owner._fp16_fused_output_buf = out
    ws = getattr(owner, "_fp16_fused_buf", None)
    need = N.lib().tm_swiglu_workspace_size(hidden_states.shape[0], inter, N.dtype_tag(hidden_states.dtype))
    if ws is None or ws.numel() < need or ws.device != hidden_states.device:
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=hidden_states.device)
        owner._fp16_fused_buf = ws
    return expert_swiglu(hidden_states, w1, w3, w2, out=out, workspace=ws)
