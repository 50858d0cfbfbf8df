"""Router softmax + top-k on a HIP kernel.

Same entry point and results as the reference's qwen_topk_softmax
(table_moe/ops/qwen_topk_softmax.py:122-154): fp32 softmax probabilities of
the top_k experts in descending order (ties to the lower expert id), int64 ids;
``normalize_topk`` divides by their sum (clamped to 1e-20).
"""

from __future__ import annotations

import torch

from .. import _native as N


def qwen_topk_softmax(router_logits: torch.Tensor, top_k: int, *, normalize_topk: bool = False):
    if router_logits.dim() != 2:
        raise ValueError(f"qwen_topk_softmax expects 2D logits, got {tuple(router_logits.shape)}")
    dev = N.require_hip(router_logits)
    logits = router_logits.to(dtype=torch.float32)
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    n, n_exp = logits.shape
    weights = torch.empty((n, top_k), dtype=torch.float32, device=dev)
    ids = torch.empty((n, top_k), dtype=torch.long, device=dev)
    N.call(
        "tm_topk_softmax", N.ptr(logits), n, n_exp, logits.stride(0), int(top_k), 1 if normalize_topk else 0,
        N.ptr(weights), N.ptr(ids), N.stream(dev),
    )
    return weights, ids
