"""numpy restatement of the TableMoE table-search path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module.  It is never part of the product path.

Two semantics are restated:

* mode R -- the reference's own semantics (``table_moe`` torch fallback path):
  per-(expert, modality) tables, max dot / cosine with thresholds, expert-level
  keep-by-importance, slot combine with surviving-weight renormalisation.
* mode G -- the BASELINE measurement configs: one global centroid table, L2
  distance, top-k nearest, token keep-by-largest-distance, gather of cached
  per-cluster outputs fused with the combine and the residual add.

Arithmetic contract.  Scores and distances are evaluated exactly (float64 over
bf16/fp16 operands, whose products are exact in float64); the device computes
them in fp32.  Indices must then agree bit-exactly except where the exact gap
between the device's pick and the oracle's pick is within ``GAP_RTOL``
relative (``gap_ok``).  Rounding to the model dtype happens at the same op
boundaries as the reference's torch ops (addmm -> dtype, vector_norm -> dtype,
division -> fp32 -> dtype).

Pinning of each function (what checks it besides its own formula):

=============================  =================================================
function                       pinned by
=============================  =================================================
round_to                       numpy float16 / float32 casts, bit patterns
topk_softmax                   closed form (softmax of known logits), brute force
modality_mask                  closed form (token ids 151655/151656)
build_fixed_keep_mask          reference KAT test_pruning.py:109-113
renormalize_surviving_weights  reference KAT test_pruning.py:115-120 and the
                               DeepSeek target-row-sum cases :214-217, :314-320
build_prefill_keep_mask        brute force over expert subsets (tiny), closed
                               form on hand-built cases
project_queries                torch.addmm / vector_norm on CPU (library
                               routine), identity-PCA special case
search_gated                   reference KATs test_search.py:48-89, brute force
search_hybrid                  hand-built cases (closed form), brute force
online_update                  brute-force ring-buffer simulation
slot_combine                   closed form (constant experts, as the
                               reference's wrapper KATs test_pruning.py:183-327)
global_search                  brute force sort of all distances, closed form
                               (centroid queries map to themselves)
keep_select                    brute force sort; invariants
gather_combine                 closed form on one-hot tables
swiglu_expert                  torch.nn.functional.silu + matmul (library
                               routines) and one-hot weights, where the output
                               is silu(x_a) * x_b through scalar math.exp; the
                               addend form by its two closed forms (zero
                               addend = the plain MLP, zero W2 = the addend)
grouped_swiglu                 per-expert swiglu_expert on the pairs of each
                               expert (brute-force regrouping)
last_query_importance          torch.softmax / matmul (library routines) in
                               the reference's op order; closed forms (equal
                               scores give 1/S; one dominant key takes ~1)
=============================  =================================================
"""

from __future__ import annotations

import numpy as np

GAP_RTOL = 1e-5
GAP_ATOL = 1e-6

F32, F16, BF16 = "f32", "f16", "bf16"
_MANT_BITS = {F16: 10, BF16: 7}
_MIN_EXP = {F16: -14, BF16: -126}
_MAX_FINITE = {F16: 65504.0, BF16: 3.3895313892515355e38}


# ---------------------------------------------------------------------------
# dtype helpers
# ---------------------------------------------------------------------------
def round_to(x, dt: str) -> np.ndarray:
    """Round exact (float64) values to dtype ``dt`` (round-half-even), returned as float64.

    One rounding from the float64 value straight to the target format, as a
    fused device epilogue does after fp32 accumulation.
    """
    x = np.asarray(x, dtype=np.float64)
    if dt == F32:
        return x.astype(np.float32).astype(np.float64)
    mant = _MANT_BITS[dt]
    out = np.zeros_like(x)
    nz = (x != 0) & np.isfinite(x)
    _, ex = np.frexp(x[nz])  # |x| in [2^(ex-1), 2^ex)
    ulp_exp = np.maximum(ex - 1, _MIN_EXP[dt]) - mant
    scale = np.ldexp(1.0, ulp_exp)
    r = np.rint(x[nz] / scale) * scale
    r = np.where(np.abs(r) > _MAX_FINITE[dt], np.copysign(np.inf, r), r)
    out[nz] = r
    out[~np.isfinite(x)] = x[~np.isfinite(x)]
    return out


def f32(x) -> np.ndarray:
    """Round to fp32 (as float64 values)."""
    return np.asarray(x, dtype=np.float64).astype(np.float32).astype(np.float64)


def bf16_bits(x) -> np.ndarray:
    """bf16 bit patterns (uint16) of values already representable in bf16."""
    v = np.asarray(x, dtype=np.float32)
    return (v.view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32).astype(np.float64)


# ---------------------------------------------------------------------------
# index comparison under the near-tie rule
# ---------------------------------------------------------------------------
def gap_ok(values_row, got, want, larger_is_better: bool) -> bool:
    """True when picking ``got`` instead of ``want`` is within the near-tie rule.

    ``values_row`` holds the exact scores (or distances) of one query.  The
    pick may differ only when the exact gap is <= GAP_RTOL * |best| + GAP_ATOL.
    """
    if got == want:
        return True
    vg = float(values_row[got])
    vw = float(values_row[want])
    gap = (vw - vg) if larger_is_better else (vg - vw)
    return gap <= GAP_RTOL * abs(vw) + GAP_ATOL


def threshold_ok(score, thr, got_hit, want_hit) -> bool:
    """A hit flag may differ from the exact comparison only at a near-tie with the threshold."""
    if bool(got_hit) == bool(want_hit):
        return True
    return abs(float(score) - float(thr)) <= GAP_RTOL * max(abs(float(thr)), abs(float(score))) + GAP_ATOL


# ---------------------------------------------------------------------------
# a1: router top-k softmax
# ---------------------------------------------------------------------------
def topk_softmax(logits, top_k: int, renormalize: bool = False):
    """Router softmax + top-k (table_moe/ops/qwen_topk_softmax.py:117-119, 151-152;
    CUDA kernel semantics qwen_topk_softmax_kernels.cu:175-393: fp32 softmax,
    k rounds of argmax with ties to the lower expert id).

    Returns (weights float64 [N,k], ids int64 [N,k], probs float64 [N,E]).
    """
    z = np.asarray(logits, dtype=np.float64)
    z = z - z.max(axis=1, keepdims=True)
    e = np.exp(z)
    p = e / e.sum(axis=1, keepdims=True)
    n, n_exp = p.shape
    cols = np.broadcast_to(np.arange(n_exp), p.shape)
    order = np.lexsort((cols, -p), axis=1)[:, :top_k]
    ids = order.astype(np.int64)
    w = np.take_along_axis(p, ids, axis=1)
    if renormalize:
        w = w / np.maximum(w.sum(axis=1, keepdims=True), 1e-20)
    return w, ids, p


# ---------------------------------------------------------------------------
# a2: modality mask
# ---------------------------------------------------------------------------
VISION_TOKEN_IDS = (151655, 151656)


def modality_mask(input_ids, seq_len=None):
    """is_vision = input_id in {151655, 151656} (table_moe/utils/modality.py:46-69)."""
    ids = np.asarray(input_ids)
    m = np.isin(ids, VISION_TOKEN_IDS)
    if seq_len is not None and m.shape[1] != seq_len:
        m = m[:, -1:] if seq_len == 1 else m[:, -seq_len:]
    return m


# ---------------------------------------------------------------------------
# a3: keep masks and surviving-weight renormalisation
# ---------------------------------------------------------------------------
def build_fixed_keep_mask(selected_experts, keep_k):
    """First ``keep_k`` slots kept (table_moe/skip/pruning.py:4-15)."""
    sel = np.asarray(selected_experts)
    mask = np.zeros(sel.shape, dtype=bool)
    if sel.size == 0:
        return mask
    if keep_k is None:
        keep_k = sel.shape[1]
    keep_k = max(0, min(int(keep_k), sel.shape[1]))
    mask[:, :keep_k] = True
    return mask


def keep_count(n: int, keep_rate: float) -> int:
    """max(1, int(n * keep_rate)) clamped to n (table_moe/skip/pruning.py:45-46)."""
    if n <= 0:
        return 0
    return min(max(1, int(n * float(keep_rate))), n)


def build_prefill_keep_mask(selected_experts, routing_weights, attn_scores, num_experts, keep_rate):
    """Expert-level keep by importance (table_moe/skip/pruning.py:18-48).

    score[e] = sum over (b,s) with sel=e of attn[b]*w[b,s] (or w/N without
    attention); the top max(1, int(n_active*keep_rate)) activated experts are
    kept.  Equal scores are ordered by lower expert id (the reference's
    ``argsort`` leaves that order unspecified).
    """
    sel = np.asarray(selected_experts, dtype=np.int64)
    w = np.asarray(routing_weights, dtype=np.float64)
    mask = np.zeros(sel.shape, dtype=bool)
    if sel.size == 0:
        return mask, np.zeros(num_experts)
    if attn_scores is not None and np.asarray(attn_scores).size == sel.shape[0]:
        comb = np.asarray(attn_scores, dtype=np.float64)[:, None] * w
    else:
        comb = w / max(sel.shape[0], 1)
    sums = np.zeros(num_experts, dtype=np.float64)
    np.add.at(sums, sel.reshape(-1), comb.reshape(-1))
    active = np.unique(sel)
    order = np.lexsort((active, -sums[active]))
    ranked = active[order]
    n_keep = keep_count(ranked.size, keep_rate)
    kept = ranked[:n_keep]
    return np.isin(sel, kept), sums


def renormalize_surviving_weights(routing_weights, keep_mask, target_row_sum=None, dt: str = F32):
    """w~ = w*mask / sum(w*mask) * target (table_moe/skip/pruning.py:55-73).

    Each torch op rounds to the weights' dtype ``dt``; rows whose kept sum is
    not > 0 are all zero.
    """
    w = np.asarray(routing_weights, dtype=np.float64)
    m = np.asarray(keep_mask, dtype=bool)
    pruned = np.where(m, w, 0.0)
    rowsum = round_to(pruned.sum(axis=-1, keepdims=True), dt)
    if target_row_sum is None:
        target = np.ones_like(rowsum)
    else:
        target = round_to(np.asarray(target_row_sum, dtype=np.float64).reshape(rowsum.shape), dt)
    out = np.zeros_like(w)
    valid = rowsum[:, 0] > 0
    q = round_to(pruned[valid] / rowsum[valid], dt)
    out[valid] = round_to(q * target[valid], dt)
    return out


# ---------------------------------------------------------------------------
# a4: projection into the PCA space
# ---------------------------------------------------------------------------
def project_queries(x, is_vision, pca_vis, pca_txt, normalize: bool, dt: str, eps: float = 1e-6):
    """q = addmm(bias_m, x, P_m) per modality, optional L2 normalisation
    (table_moe/cache_engine/search.py:476-498; _normalize_last_dim :12-21).

    x, P, bias hold dtype-``dt`` values.  addmm rounds once to ``dt``; the norm
    rounds to ``dt``; the division is fp32 then ``dt``; norms <= eps give 0.
    Returns q (float64 values representable in ``dt``).
    """
    x = np.asarray(x, dtype=np.float64)
    vis = np.asarray(is_vision, dtype=bool)
    if pca_txt is None:  # one shared projection (search.py:408-410)
        pca_txt = pca_vis
    d = pca_vis[0].shape[1]
    q = np.zeros((x.shape[0], d), dtype=np.float64)
    for mask, (proj, bias) in ((vis, pca_vis), (~vis, pca_txt)):
        if not mask.any():
            continue
        low = round_to(x[mask] @ np.asarray(proj, np.float64) + np.asarray(bias, np.float64), dt)
        if normalize:
            low = normalize_rows(low, dt, eps)
        q[mask] = low
    return q


def normalize_rows(v, dt: str, eps: float = 1e-6):
    """Row L2 normalisation with torch's per-op rounding (search.py:12-21)."""
    v = np.asarray(v, dtype=np.float64)
    norms = round_to(np.sqrt((v * v).sum(axis=-1, keepdims=True)), dt)
    eps_dt = round_to(np.array(eps), dt)
    denom = np.maximum(norms, eps_dt)
    out = round_to(f32(v / denom), dt)
    out = np.where(norms <= eps_dt, 0.0, out)
    return out


def normalize_keys(k, dt: str, eps: float = 1e-6):
    """Key normalisation at table load (table_moe/cache_engine/manager.py:24-31):
    fp32 norm, fp32 division, then round to the model dtype."""
    k32 = f32(np.asarray(k, dtype=np.float64))
    n = f32(np.sqrt((k32 * k32).sum(axis=-1, keepdims=True)))
    denom = np.maximum(n, f32(eps))
    out = round_to(f32(k32 / denom), dt)
    return np.where(n <= f32(eps), 0.0, out)


# ---------------------------------------------------------------------------
# a5-a7: gated per-(expert, modality) search
# ---------------------------------------------------------------------------
CMP_GE, CMP_GT = 0, 1


def search_gated(q_low, keys, sel, is_vision, reuse, thr_vision, thr_text, cmp, col_offset=0):
    """Gated max-dot search over the (expert, modality) table of each reused slot
    (table_moe/cache_engine/search.py:566-602 cosine, :661-697 dot; kernel
    semantics :35-93, :95-256).

    For each (b, s) with reuse[b,s] (and s >= col_offset): scores over the K
    centroids of keys[sel[b,s], m(b)], (max, first argmax), hit = max >=thr
    (CMP_GE) or > thr (CMP_GT).  Non-searched slots and misses give (False, 0)
    (torch-fallback output convention).  Returns (hit, idx, max, scores) where
    scores[b,s,:] are the exact scores (NaN where not searched).
    """
    q = np.asarray(q_low, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    sel = np.asarray(sel, dtype=np.int64)
    vis = np.asarray(is_vision, dtype=bool)
    n, k = sel.shape
    n_exp, _, n_cent, _ = keys.shape
    rs = np.ones((n, k), dtype=bool) if reuse is None else np.asarray(reuse, dtype=bool)
    hit = np.zeros((n, k), dtype=bool)
    idx = np.zeros((n, k), dtype=np.int64)
    mx = np.full((n, k), np.nan)
    scores = np.full((n, k, n_cent), np.nan)
    thr_v = float(np.float32(thr_vision))
    thr_t = float(np.float32(thr_text))
    for b in range(n):
        m = 0 if vis[b] else 1
        thr = thr_v if vis[b] else thr_t
        for s in range(col_offset, k):
            e = sel[b, s]
            if not rs[b, s] or e < 0 or e >= n_exp:
                continue
            sc = keys[e, m] @ q[b]
            scores[b, s] = sc
            j = int(np.argmax(sc))
            mx[b, s] = sc[j]
            h = sc[j] >= thr if cmp == CMP_GE else sc[j] > thr
            if h:
                hit[b, s] = True
                idx[b, s] = j
    return hit, idx, mx, scores


# ---------------------------------------------------------------------------
# a8: decode hybrid search (online window + offline)
# ---------------------------------------------------------------------------
def search_hybrid(x, is_vision, pca_vis, pca_txt, dt, keys, sel, keep_k, online_keys, online_ids, n_valid):
    """Decode hybrid search, torch-fallback semantics
    (table_moe/cache_engine/search.py:839-954 with _search_decode_online_into
    :778-806 and the offline fallback :566-602 at threshold 0.0, >=).

    Returns dict(on_hit, on_idx, off_hit, off_idx, on_slot, on_max, on_scores,
    off_max, off_scores, q_low).
    """
    x = np.asarray(x, dtype=np.float64)
    sel = np.asarray(sel, dtype=np.int64)
    n, k = sel.shape
    keep_k = max(0, min(int(keep_k), k))
    on_hit = np.zeros((n, k), dtype=bool)
    off_hit = np.zeros((n, k), dtype=bool)
    off_idx = np.zeros((n, k), dtype=np.int64)
    on_idx = np.full((n,), -1, dtype=np.int64)
    on_slot = np.zeros((n, k), dtype=np.int64)
    res = dict(on_hit=on_hit, on_idx=on_idx, off_hit=off_hit, off_idx=off_idx, on_slot=on_slot,
               on_max=None, on_scores=None, off_max=None, off_scores=None, q_low=None)
    if k - keep_k <= 0:
        return res
    reuse = np.zeros((n, k), dtype=bool)
    has_online = online_keys is not None and online_ids is not None and n_valid > 0
    if has_online:
        ok = np.asarray(online_keys, dtype=np.float64)[:n_valid]
        oid = np.asarray(online_ids, dtype=np.int64)[:n_valid]
        sc = x @ ok.T
        j = np.argmax(sc, axis=1)
        mx = sc[np.arange(n), j]
        valid = mx > 0
        on_idx[valid] = j[valid]
        cached = oid[j]  # [n, topk_online]
        tail = sel[:, keep_k:]
        matches = tail[:, :, None] == cached[:, None, :]
        slot_hits = matches.any(axis=-1) & valid[:, None]
        on_hit[:, keep_k:] = slot_hits
        first = np.argmax(matches, axis=-1)
        on_slot[:, keep_k:] = np.where(slot_hits, first, 0)
        reuse[:, keep_k:] = ~slot_hits
        res["on_max"], res["on_scores"] = mx, sc
    else:
        reuse[:, keep_k:] = True
    q = project_queries(x, is_vision, pca_vis, pca_txt, normalize=False, dt=dt)
    h, i, omx, osc = search_gated(q, keys, sel, is_vision, reuse, 0.0, 0.0, CMP_GE)
    off_hit[:] = h
    off_idx[:] = i
    res["off_max"], res["off_scores"], res["q_low"] = omx, osc, q
    return res


# ---------------------------------------------------------------------------
# a9/a10: table gather; a12: online ring buffer
# ---------------------------------------------------------------------------
def gather_values(values, eids, mids, cids):
    """values[e, m, c] rows (table_moe/cache_engine/manager.py:212-213)."""
    return np.asarray(values)[np.asarray(eids), np.asarray(mids), np.asarray(cids)]


def online_update(state, hidden, ids, outputs, valid_mask=None):
    """Ring-buffer update of the online window (manager.py:108-155).

    ``state`` is a dict with keys/ids/values arrays and ptr/full/size; a new
    dict is returned.
    """
    st = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in state.items()}
    size = st["size"]
    hidden = np.asarray(hidden)
    n = hidden.shape[0]
    if n == 0:
        return st
    ids = np.array(ids, copy=True)
    outputs = np.array(outputs, copy=True)
    if valid_mask is not None:
        inv = ~np.asarray(valid_mask, dtype=bool)
        ids[inv] = -1
        outputs[inv] = 0
    if n > size:
        hidden, ids, outputs = hidden[-size:], ids[-size:], outputs[-size:]
        n = size
    for i in range(n):
        r = (st["ptr"] + i) % size
        st["keys"][r] = hidden[i]
        st["ids"][r] = ids[i]
        st["values"][r] = outputs[i]
    end = st["ptr"] + n
    if end > size:
        st["full"] = True
    st["ptr"] = end % size
    if st["ptr"] == 0:
        st["full"] = True
    return st


# ---------------------------------------------------------------------------
# a11: slot combine (reference semantics)
# ---------------------------------------------------------------------------
def slot_combine(collected, routing_weights, survivor, dt: str, target_mode: str = "one", residual=None,
                 out_dt: str | None = None):
    """Combine of surviving slots.

    target_mode "one": Qwen path, w~ = renormalize(w, survivor).to(dtype),
    y = bmm(w~, collected) (fp32 accumulate, one rounding)
    (table_moe/models/qwen3_vl_moe/cached_layers.py:463-465).
    target_mode "orig_sum": DeepSeek path, w~ rescaled to sum(w), product and
    sum in the weights' fp32, then rounded
    (table_moe/models/deepseek_vl2/deepseek_layers.py:715-729).
    ``dt`` is the model dtype (the weights' rounding in the Qwen path); the
    output is rounded to ``out_dt`` (default ``dt``; F32 gives the value
    before the final rounding).
    """
    c = np.asarray(collected, dtype=np.float64)
    w = np.asarray(routing_weights, dtype=np.float64)
    if target_mode == "one":
        wt = round_to(renormalize_surviving_weights(w, survivor), dt)
        y = np.einsum("bs,bsh->bh", wt, c)
    else:
        wt = renormalize_surviving_weights(w, survivor, target_row_sum=w.sum(axis=-1, keepdims=True))
        y = np.einsum("bs,bsh->bh", wt, c)
    if residual is not None:
        y = y + np.asarray(residual, dtype=np.float64)
    return round_to(y, dt if out_dt is None else out_dt), wt


# ---------------------------------------------------------------------------
# mode G: global table search, keep-by-distance, gather + combine
# ---------------------------------------------------------------------------
def sq_distances(q, cents):
    """Exact squared L2 distances [N, C] (float64 over dtype operands)."""
    q = np.asarray(q, dtype=np.float64)
    c = np.asarray(cents, dtype=np.float64)
    d = (q * q).sum(1)[:, None] - 2.0 * (q @ c.T) + (c * c).sum(1)[None, :]
    return np.maximum(d, 0.0)


def global_search(q, cents, top_k: int, metric: str = "l2"):
    """Top-k nearest centroids; ascending distance (or descending dot), ties to
    the lower centroid index.  Returns (vals [N,k], idx [N,k], full [N,C])."""
    if metric == "l2":
        full = sq_distances(q, cents)
        key = full
    else:
        full = np.asarray(q, np.float64) @ np.asarray(cents, np.float64).T
        key = -full
    n, c = key.shape
    if top_k == 1:
        idx = np.argmin(key, axis=1)[:, None]  # first minimum
    else:
        k = min(top_k, c)
        kth = np.partition(key, k - 1, axis=1)[:, k - 1 : k]
        idx = np.empty((n, k), dtype=np.int64)
        for r in range(n):
            cand = np.nonzero(key[r] <= kth[r, 0])[0]  # every tie of the k-th value
            order = np.lexsort((cand, key[r, cand]))[:k]
            idx[r] = cand[order]
    idx = idx.astype(np.int64)
    return np.take_along_axis(full, idx, axis=1), idx, full


def keep_select(score, n_keep: int):
    """Keep the ``n_keep`` tokens with the largest score; equal scores keep the
    lower token index first (BASELINE keep_rate rule, floor as pruning.py:45)."""
    s = np.asarray(score, dtype=np.float64)
    n = s.shape[0]
    order = np.lexsort((np.arange(n), -s))
    keep = np.zeros(n, dtype=bool)
    keep[order[:n_keep]] = True
    return keep


def blend_weights(dist, eps: float = 1e-6):
    """beta_j proportional to 1/(d_j + eps), normalised over the k nearest."""
    inv = 1.0 / (np.asarray(dist, dtype=np.float64) + eps)
    return inv / inv.sum(axis=1, keepdims=True)


def gather_combine(keep, slot_out, weights, values, idx, dist, residual, dt: str = BF16):
    """out_i = R_i + (keep_i ? sum_s w~_is E_is : sum_j beta_ij V[idx_ij]),
    w~ = w / sum(w) (top-k softmax renormalised to 1), beta from blend_weights
    (top-1 gives beta = 1).  fp64 math, one rounding to ``dt``."""
    keep = np.asarray(keep, dtype=bool)
    w = np.asarray(weights, dtype=np.float64)
    wt = w / w.sum(axis=1, keepdims=True)
    e = np.asarray(slot_out, dtype=np.float64)
    v = np.asarray(values, dtype=np.float64)
    idx = np.asarray(idx, dtype=np.int64)
    beta = blend_weights(dist) if idx.shape[1] > 1 else np.ones(idx.shape)
    y_keep = np.einsum("bs,bsh->bh", wt[keep], e[keep])
    y_reuse = np.einsum("bj,bjh->bh", beta[~keep], v[idx[~keep]])
    y = np.zeros((keep.shape[0], v.shape[1]))
    y[keep] = y_keep
    y[~keep] = y_reuse
    return round_to(np.asarray(residual, dtype=np.float64) + y, dt)


def layer_forward_g(x, is_vision, pca_vis, pca_txt, cents, values, logits, slot_out, residual,
                    top_k_router: int, n_nearest: int, keep_rate: float, dt: str = BF16):
    """Mode-G single-layer path: router top-k -> projection -> nearest
    centroids -> keep-by-distance -> gather + combine + residual."""
    w, ids, _ = topk_softmax(logits, top_k_router)
    q = project_queries(x, is_vision, pca_vis, pca_txt, normalize=False, dt=dt)
    dist, idx, _ = global_search(q, cents, n_nearest)
    n_keep = keep_count(q.shape[0], keep_rate)
    keep = keep_select(dist[:, 0], n_keep)
    out = gather_combine(keep, slot_out, w, values, idx, dist, residual, dt)
    return dict(weights=w, ids=ids, q=q, dist=dist, idx=idx, keep=keep, out=out)


def layer_forward_g_fp32(x, is_vision, pca_vis, pca_txt, cents, values, logits, slot_out, residual,
                         top_k_router: int, n_nearest: int, keep_rate: float):
    """Same op sequence in float32 numpy (BLAS), used only as the timed CPU
    baseline: the reference fallback's order addmm -> bmm/min -> compare ->
    fancy-index gather -> renorm -> weighted sum (search.py:476-602,
    cached_layers.py:455-465), at the CPU's fp32 precision."""
    x = np.asarray(x, dtype=np.float32)
    z = np.asarray(logits, dtype=np.float32)
    z = z - z.max(axis=1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argpartition(-p, top_k_router - 1, axis=1)[:, :top_k_router]
    w = np.take_along_axis(p, ids, axis=1)
    vis = np.asarray(is_vision, dtype=bool)
    q = np.empty((x.shape[0], pca_vis[0].shape[1]), dtype=np.float32)
    for mask, (proj, bias) in ((vis, pca_vis), (~vis, pca_txt)):
        if mask.any():
            q[mask] = x[mask] @ proj + bias
    c = np.asarray(cents, dtype=np.float32)
    d = (q * q).sum(1)[:, None] - 2.0 * (q @ c.T) + (c * c).sum(1)[None, :]
    idx = np.argpartition(d, n_nearest - 1, axis=1)[:, :n_nearest]
    dist = np.take_along_axis(d, idx, axis=1)
    n_keep = keep_count(q.shape[0], keep_rate)
    keep = np.zeros(q.shape[0], dtype=bool)
    keep[np.argsort(-dist.min(axis=1), kind="stable")[:n_keep]] = True
    wt = w / w.sum(axis=1, keepdims=True)
    v = np.asarray(values, dtype=np.float32)
    out = np.asarray(residual, dtype=np.float32).copy()
    kept = np.nonzero(keep)[0]
    out[kept] += np.einsum("bs,bsh->bh", wt[kept], np.asarray(slot_out[kept], dtype=np.float32))
    reused = np.nonzero(~keep)[0]
    if n_nearest == 1:
        out[reused] += v[idx[reused, 0]]
    else:
        beta = 1.0 / (dist[reused] + 1e-6)
        beta /= beta.sum(axis=1, keepdims=True)
        out[reused] += np.einsum("bj,bjh->bh", beta, v[idx[reused]])
    return out


__all__ = [name for name in dir() if not name.startswith("_")]


# ---------------------------------------------------------------------------
# recompute path: the SwiGLU expert MLP
# ---------------------------------------------------------------------------
def silu(v):
    """x * sigmoid(x) = x / (1 + exp(-x)), float64."""
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def swiglu_expert(x, w1, w3, w2, dt: str = BF16, addend=None):
    """One expert's MLP with the rounding points of the reference's fused
    kernel (ops/csrc/fp16_fused_expert/fp16_fused_moe_mlp.cu:107-274 and the
    SiLU-mul epilogue fp16_epilogue_utils.h:51-125): g = dt(x W1^T),
    f = dt(silu(g) * (x W3^T)) with the up projection unrounded,
    y = dt(f W2^T).  Exact float64 sums of exact products.  With ``addend``
    (a DeepSeek layer's residual under its shared experts,
    deepseek_layers.py:743): y = dt(addend + f W2^T), one rounding."""
    x = np.asarray(x, dtype=np.float64)
    g = round_to(x @ np.asarray(w1, dtype=np.float64).T, dt)
    u = x @ np.asarray(w3, dtype=np.float64).T
    f = round_to(silu(g) * u, dt)
    y = f @ np.asarray(w2, dtype=np.float64).T
    if addend is not None:
        y = y + np.asarray(addend, dtype=np.float64)
    return round_to(y, dt), f


def grouped_swiglu(x, ids, mask, w1, w3, w2, dt: str = BF16):
    """slot outputs [N, k, H] of every (token, slot) pair with mask set (a
    per-token [N] mask applies to all k slots); other slots are NaN."""
    x = np.asarray(x, dtype=np.float64)
    ids = np.asarray(ids, dtype=np.int64)
    n, k = ids.shape
    m = np.asarray(mask, dtype=bool)
    if m.ndim == 1:
        m = np.repeat(m[:, None], k, axis=1)
    out = np.full((n, k, x.shape[1]), np.nan)
    for e in range(np.asarray(w1).shape[0]):
        b, s = np.nonzero(m & (ids == e))
        if len(b):
            out[b, s] = swiglu_expert(x[b], w1[e], w3[e], w2[e], dt)[0]
    return out


# ---------------------------------------------------------------------------
# importance for the expert keep rule: last-query attention probabilities
# ---------------------------------------------------------------------------
def last_query_importance(q, k, n_kv_heads: int, scale: float, score_dt: str, key_mask=None, out_len=None):
    """q [B, H, D], k [B, S, Hkv, D] -> [B, out_len] float64: per head, the
    softmax over keys of the last query's scores, averaged over heads, for
    the last ``out_len`` keys.  score_dt = the model dtype (scores rounded
    after the dot product and again after the scaling, as
    hybrid_attention.py:111-146 does) or F32 (deepseek_attention.py:206-249);
    masked keys (key_mask False) get probability 0."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    b, h, d = q.shape
    s = k.shape[1]
    groups = h // n_kv_heads
    kk = np.repeat(k, groups, axis=2)  # [B, S, H, D]: head h reads KV head h // groups
    dot = np.einsum("bhd,bshd->bhs", q, kk)
    if score_dt == F32:
        sc = f32(f32(dot) * np.float32(scale))
    else:
        sc = round_to(round_to(dot, score_dt) * np.float64(np.float32(scale)), score_dt)
    valid = np.ones((b, s), dtype=bool) if key_mask is None else np.asarray(key_mask, dtype=bool)
    sc = np.where(valid[:, None, :], sc, -np.inf)
    m = sc.max(axis=2, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    e = np.where(valid[:, None, :], np.exp(sc - m), 0.0)
    tot = e.sum(axis=2, keepdims=True)
    p = np.where(tot > 0, e / np.where(tot > 0, tot, 1.0), 0.0)
    out_len = s if out_len is None else out_len
    return p[:, :, s - out_len:].mean(axis=1)
