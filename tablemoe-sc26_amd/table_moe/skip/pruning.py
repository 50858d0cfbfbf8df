"""Keep masks and surviving-weight renormalisation on HIP kernels.

Same functions, signatures and results as the reference's
table_moe/skip/pruning.py:4-73.  ``build_prefill_keep_mask`` sums the expert
scores in a fixed order (the reference's ``scatter_add_`` order is not fixed)
and ranks equal scores by lower expert id (the reference's ``argsort`` leaves
that order open); it needs no host synchronisation.
"""

from __future__ import annotations

import torch

from .. import _native as N

_ws_cache: dict = {}


def build_fixed_keep_mask(selected_experts: torch.Tensor, keep_k: int | None) -> torch.Tensor:
    """out[b, s] = s < keep_k (reference pruning.py:4-15)."""
    mask = torch.empty(selected_experts.shape, dtype=torch.bool, device=selected_experts.device)
    if selected_experts.numel() == 0:
        return mask
    dev = N.require_hip(selected_experts)
    n, top_k = selected_experts.shape
    if keep_k is None:
        keep_k = top_k
    keep_k = max(0, min(int(keep_k), top_k))
    N.call("tm_fixed_keep_mask", n, top_k, keep_k, N.ptr(N.as_u8(mask)), N.stream(dev))
    return mask


def _workspace(device, nbytes):
    # one scratch buffer per (device, stream): calls enqueued on different
    # streams must not share it
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    ws = _ws_cache.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        _ws_cache[key] = ws
    return ws


def build_prefill_keep_mask(
    selected_experts: torch.Tensor,
    routing_weights: torch.Tensor,
    attn_scores: torch.Tensor | None,
    num_experts: int,
    keep_rate: float,
) -> torch.Tensor:
    """Keep the top max(1, int(n_active*keep_rate)) activated experts by
    importance (reference pruning.py:18-48)."""
    mask = torch.empty(selected_experts.shape, dtype=torch.bool, device=selected_experts.device)
    if selected_experts.numel() == 0:
        return mask
    dev = N.require_hip(selected_experts, routing_weights)
    n, top_k = selected_experts.shape
    sel = selected_experts.long().contiguous()
    w = routing_weights.float().contiguous()
    attn = None
    if attn_scores is not None and attn_scores.numel() == n:
        attn = attn_scores.reshape(-1).to(device=dev, dtype=torch.float32).contiguous()
    nbytes = N.lib().tm_expert_keep_mask_workspace_size(n, int(num_experts))
    ws = _workspace(dev, nbytes)
    N.call(
        "tm_expert_keep_mask", N.ptr(sel), N.ptr(w), N.ptr(attn), n, top_k, int(num_experts), float(keep_rate),
        N.ptr(N.as_u8(mask)), None, N.ptr(ws), ws.numel(), N.stream(dev),
    )
    return mask


def build_decode_keep_mask(selected_experts: torch.Tensor, keep_k: int | None) -> torch.Tensor:
    return build_fixed_keep_mask(selected_experts, keep_k)


def renormalize_surviving_weights(
    routing_weights: torch.Tensor,
    keep_mask: torch.Tensor,
    target_row_sum: torch.Tensor | None = None,
) -> torch.Tensor:
    """w~ = (w*m) / sum(w*m) * target, zero rows where nothing survives
    (reference pruning.py:55-73); arithmetic rounds to the weights' dtype."""
    out = torch.empty(routing_weights.shape, dtype=routing_weights.dtype, device=routing_weights.device)
    if routing_weights.numel() == 0:
        return out.zero_()
    dev = N.require_hip(routing_weights, keep_mask)
    w = routing_weights.reshape(-1, routing_weights.shape[-1])
    if w.stride(-1) != 1:
        w = w.contiguous()
    m = N.as_u8(keep_mask.reshape(-1, keep_mask.shape[-1]).to(dtype=torch.bool).contiguous())
    n, top_k = w.shape
    mode, tgt, ld_t = N.TM_TARGET_ONE, None, 0
    if target_row_sum is not None:
        mode = N.TM_TARGET_GIVEN
        tgt = target_row_sum.to(device=dev, dtype=routing_weights.dtype).reshape(n, -1)[:, :1].contiguous()
        ld_t = tgt.stride(0)
    N.call(
        "tm_renormalize", N.dtype_tag(w.dtype), N.ptr(w), w.stride(0), N.ptr(m), m.stride(0), n, top_k, mode,
        N.ptr(tgt), ld_t, N.ptr(out), N.stream(dev),
    )
    return out
