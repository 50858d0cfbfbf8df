"""torch-CPU restatement of the reference's fallback op sequence (BASELINE AND
TEST INFRASTRUCTURE ONLY).

Only ``bench.py``'s ``cpu_baseline`` leg and ``tests/`` may import this module;
it is never part of the product path.  It is the CPU path the bench times
beside the GPU: the reference's torch fallback (``HAS_TRITON = False``), op
for op, on host tensors, with torch's own CPU kernels doing the arithmetic.

* ``layer_forward_g`` -- one mode-G layer (the BASELINE configs): router
  softmax + top-k (table_moe/ops/qwen_topk_softmax.py:117-119), per-modality
  ``addmm`` projection (table_moe/cache_engine/search.py:484,492), distances
  by ``addmm`` + ``min``/``topk`` over the table (the L2 form of the fallback's
  ``bmm``/``max``, search.py:594-596), keep-by-distance count
  (table_moe/skip/pruning.py:45), fancy-index gather of cached outputs
  (cache_engine/manager.py:212-213), surviving-weight renormalisation
  (skip/pruning.py:55-73) and the ``bmm`` combine
  (models/qwen3_vl_moe/cached_layers.py:465), plus the residual add.
* ``recompute_slots`` -- the per-expert loop of the cached wrapper
  (cached_layers.py:431-437): index the expert's tokens, run its SwiGLU MLP,
  scatter into ``collected[token, slot]``.
* ``prefill_search_r`` -- the reference's own prefill search fallback
  (search.py:476-498 projection + normalisation, :566-602 materialised
  ``keys[eids, m]``, ``bmm``, ``max``, threshold).

Pinned by ``tests/test_cpu_ref.py`` against the numpy oracle
(``oracle/tm_oracle.py``: layer_forward_g, swiglu_expert, search_gated).
"""

from __future__ import annotations

import torch


def layer_forward_g(x, is_vision, pca_vis, pca_txt, cents, values, logits, slot_out, residual, top_k_router: int,
                    n_nearest: int, keep_rate: float, shared=None):
    """One mode-G layer in the fallback's op order; returns a dict of the
    stage outputs (``out`` = residual + combine, or residual + shared +
    combine when ``shared`` [N, H] is given)."""
    probs = torch.softmax(logits, dim=1, dtype=torch.float32)
    w, ids = torch.topk(probs, top_k_router, dim=-1)
    n, d = x.shape[0], pca_vis[0].shape[1]
    q = torch.empty((n, d), dtype=x.dtype)
    vis = is_vision.bool()
    for mask, (proj, bias) in ((vis, pca_vis), (~vis, pca_txt)):
        if bool(mask.any()):
            q[mask] = torch.addmm(bias, x[mask], proj)
    c_sq = (cents * cents).sum(dim=1)
    dist_all = torch.addmm(c_sq.unsqueeze(0), q, cents.t(), alpha=-2.0) + (q * q).sum(dim=1, keepdim=True)
    if n_nearest == 1:
        dist, idx = dist_all.min(dim=1, keepdim=True)
    else:
        dist, idx = torch.topk(dist_all, n_nearest, dim=1, largest=False)
    dist = dist.clamp_min(0.0)
    n_keep = max(1, int(n * keep_rate))
    n_keep = min(n_keep, n)
    order = torch.sort(dist[:, 0], descending=True, stable=True).indices
    keep = torch.zeros(n, dtype=torch.bool)
    keep[order[:n_keep]] = True
    out = residual.clone() if shared is None else residual + shared
    kept = keep.nonzero().squeeze(1)
    wk = w[kept]
    wk = wk / wk.sum(dim=1, keepdim=True)
    out[kept] += torch.bmm(wk.unsqueeze(1).to(slot_out.dtype), slot_out[kept]).squeeze(1)
    reused = (~keep).nonzero().squeeze(1)
    if n_nearest == 1:
        out[reused] += values[idx[reused, 0]]
    else:
        beta = 1.0 / (dist[reused] + 1e-6)
        beta = beta / beta.sum(dim=1, keepdim=True)
        out[reused] += torch.bmm(beta.unsqueeze(1).to(values.dtype), values[idx[reused]]).squeeze(1)
    return {"weights": w, "ids": ids, "q": q, "dist": dist, "idx": idx, "keep": keep, "out": out}


def swiglu(x, w1, w3, w2):
    """SwiGLU expert MLP with nn.Linear weights (w1, w3 [I, H], w2 [H, I])."""
    return (torch.nn.functional.silu(x @ w1.t()) * (x @ w3.t())) @ w2.t()


def recompute_slots(x, ids, keep, w1, w3, w2, slot_out):
    """slot_out[b, s] = expert ids[b, s] on x[b] for every kept token, one
    expert at a time (the cached wrapper's loop)."""
    kb = keep.nonzero().squeeze(1)
    sel = ids[kb]
    for e in torch.unique(sel).tolist():
        rows, slots = (sel == e).nonzero(as_tuple=True)
        tok = kb[rows]
        slot_out[tok, slots] = swiglu(x[tok], w1[e], w3[e], w2[e])
    return slot_out


def prefill_search_r(x, is_vision, pca_vis, pca_txt, keys, sel, reuse, thr_vision: float, thr_text: float,
                     eps: float = 1e-6):
    """The reference fallback of search_prefill_offline: projection,
    normalisation, materialised per-pair tables, bmm, max, threshold (>=)."""
    n, d = x.shape[0], pca_vis[0].shape[1]
    vis = is_vision.bool()
    q = torch.empty((n, d), dtype=x.dtype)
    for mask, (proj, bias) in ((vis, pca_vis), (~vis, pca_txt)):
        if bool(mask.any()):
            q[mask] = torch.addmm(bias, x[mask], proj)
    norm = torch.linalg.vector_norm(q, dim=-1, keepdim=True)
    q = torch.where(norm > eps, q / norm.clamp_min(eps), torch.zeros_like(q))
    hit = torch.zeros(sel.shape, dtype=torch.bool)
    idx = torch.zeros(sel.shape, dtype=torch.long)
    b, s = reuse.nonzero(as_tuple=True)
    if b.numel():
        m = (~vis[b]).long()
        tables = keys[sel[b, s], m]                       # [n, K, d]
        scores = torch.bmm(tables, q[b].unsqueeze(2)).squeeze(2)
        best, arg = scores.max(dim=1)
        thr = torch.where(vis[b], torch.tensor(thr_vision), torch.tensor(thr_text)).to(best.dtype)
        h = best >= thr
        hit[b, s] = h
        idx[b, s] = torch.where(h, arg, torch.zeros_like(arg))
    return hit, idx
