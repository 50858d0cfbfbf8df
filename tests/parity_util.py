"""Helpers shared by the GPU parity tests (comparison rules of the oracle)."""

import numpy as np
import torch

from oracle import tm_oracle as O

ODT = {torch.bfloat16: O.BF16, torch.float16: O.F16, torch.float32: O.F32}
MANT = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}


def np64(t: torch.Tensor) -> np.ndarray:
    """Exact float64 (or int64/bool) copy of a device tensor."""
    t = t.detach().cpu()
    if t.dtype in (torch.bfloat16, torch.float16, torch.float32, torch.float64):
        return t.double().numpy()
    return t.numpy()


def ulp(ref: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    a = np.abs(np.asarray(ref, dtype=np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    return np.where(a > 0, np.ldexp(1.0, (e - MANT[dtype]).astype(int)), np.ldexp(1.0, -133))


def assert_within_ulps(got, ref, dtype, n_ulp=1, min_exact=0.97):
    got, ref = np.asarray(got), np.asarray(ref)
    bad = np.abs(got - ref) > n_ulp * ulp(ref, dtype) + 1e-30
    assert not bad.any(), f"{bad.sum()} values beyond {n_ulp} ulp, e.g. got {got[bad][:4]} want {ref[bad][:4]}"
    frac = float(np.mean(got == ref)) if got.size else 1.0
    assert frac >= min_exact, f"only {frac:.4f} bit-exact"


def check_pick(values_row, got, want, larger_is_better, what=""):
    assert O.gap_ok(values_row, int(got), int(want), larger_is_better), (
        f"{what}: picked {got} ({values_row[got]}) instead of {want} ({values_row[want]})"
    )


def check_topk_rows(exact, got_idx, want_idx, larger_is_better, what=""):
    """Row-wise top-k lists: position j of the device list must be a near-tie of
    the exact j-th best; the device indices must be distinct."""
    n_mis = 0
    for r in range(got_idx.shape[0]):
        g, w = got_idx[r], want_idx[r]
        assert len(set(g.tolist())) == len(g), f"{what}: duplicate indices in row {r}: {g}"
        for j in range(len(g)):
            if g[j] != w[j]:
                n_mis += 1
                check_pick(exact[r], g[j], w[j], larger_is_better, f"{what} row {r} pos {j}")
    return n_mis


def assert_projection_close(got, ref, abssum, dtype, min_exact=0.95):
    """q from an fp32-accumulated contraction vs the exactly-rounded oracle:
    within 1 ulp of the reference plus the fp32 accumulation bound on the
    absolute sum of the terms (cancellation can leave tiny results whose ulp
    is below the accumulation error)."""
    got, ref = np.asarray(got), np.asarray(ref)
    tol = ulp(ref, dtype) + 2.0**-18 * np.asarray(abssum)
    bad = np.abs(got - ref) > tol
    assert not bad.any(), f"{bad.sum()} values off, e.g. got {got[bad][:4]} want {ref[bad][:4]}"
    frac = float(np.mean(got == ref)) if got.size else 1.0
    assert frac >= min_exact, f"only {frac:.4f} bit-exact"


def proj_abssum(x, is_vision, pv, pt, normalized_ref=None):
    """sum_h |x_h P_hj| per output (scaled by 1/||q|| for normalised outputs)."""
    x = np.abs(np.asarray(x, dtype=np.float64))
    vis = np.asarray(is_vision, dtype=bool)
    out = np.where(vis[:, None], x @ np.abs(pv), x @ np.abs(pt))
    return out


def assert_bf16_output(got, exact, abssum, dtype=torch.bfloat16, atol=1e-2, rtol=2e-3):
    """A combined output stored in a 16-bit type against the unrounded exact
    value: within one ulp of it (plus the fp32 accumulation bound over the
    absolute terms), and within (atol, rtol) wherever that tolerance exceeds
    the type's own half-ulp (|v| < 8 for bf16; beyond, one rounding alone can
    exceed 2e-3 relative)."""
    got, exact = np.asarray(got), np.asarray(exact)
    tol = ulp(exact, dtype) + 2.0**-20 * np.asarray(abssum)
    bad = np.abs(got - exact) > tol
    assert not bad.any(), f"{bad.sum()} values off, e.g. got {got[bad][:4]} want {exact[bad][:4]}"
    small = np.abs(exact) < 8.0
    np.testing.assert_allclose(got[small], exact[small], atol=atol, rtol=rtol)


def check_end_to_end_topk(q_dev, q_ora, cents, got_idx, what="", max_qdiff_frac=0.01):
    """Index parity from x, not only stage-wise: the oracle's search on its
    OWN queries (projected from x) against the device's top-k lists.  Every
    position that disagrees must be explained either by the near-tie rule on
    the oracle's exact distances (the device's pick within 1e-5 relative of
    the oracle's) or by the row's device query differing from the oracle's
    (the fp32-accumulated projection rounded a component the other way).
    The second kind is counted, printed and bounded by ``max_qdiff_frac`` of
    the positions.  Returns (oracle distances of the oracle's top-k, number
    explained by the gap rule, number explained by a different query)."""
    got_idx = np.asarray(got_idx)
    k = got_idx.shape[1]
    vals, want, exact = O.global_search(np.asarray(q_ora), cents, k)
    qdiff = np.any(np.asarray(q_dev) != np.asarray(q_ora), axis=1)
    n_gap = n_q = 0
    for r, j in zip(*np.nonzero(got_idx != want)):
        if O.gap_ok(exact[r], int(got_idx[r, j]), int(want[r, j]), False):
            n_gap += 1
        elif qdiff[r]:
            n_q += 1
        else:
            raise AssertionError(f"{what}: row {r} pos {j} picked {got_idx[r, j]} ({exact[r, got_idx[r, j]]}) "
                                 f"instead of {want[r, j]} ({exact[r, want[r, j]]}) with the oracle's own query")
    bound = max(1, int(max_qdiff_frac * got_idx.size))
    print(f"[e2e] {what}: {int(qdiff.sum())}/{len(qdiff)} query rows differ from the oracle's; "
          f"{int((got_idx != want).sum())} of {got_idx.size} indices differ from the oracle run from x: "
          f"{n_gap} near-ties, {n_q} in rows with another query (bound {bound})", flush=True)
    assert n_q <= bound, f"{what}: {n_q} index changes from query differences > {bound}"
    return vals, n_gap, n_q


def check_end_to_end_keep(dist_dev, dist_ora, keep_dev, n_keep, what="", max_frac=0.01):
    """Keep mask from x: the oracle's keep set on its own distances against
    the device's.  With delta = max |device distance - oracle distance| and T
    the oracle's n_keep-th largest distance, a token whose oracle distance is
    more than 2 delta from T is kept (or reused) by both (order statistics
    move by at most delta), so every disagreement must lie in that band; the
    count is printed and bounded by ``max_frac`` of the tokens."""
    d_dev = np.asarray(dist_dev, dtype=np.float64)
    d_ora = np.asarray(dist_ora, dtype=np.float64)
    keep_dev = np.asarray(keep_dev, dtype=bool)
    keep_ora = O.keep_select(d_ora, n_keep)
    delta = float(np.max(np.abs(d_dev - d_ora))) if d_dev.size else 0.0
    t = float(np.sort(d_ora)[::-1][n_keep - 1])
    bad = keep_ora != keep_dev
    band = np.abs(d_ora[bad] - t)
    print(f"[e2e] {what}: keep differs from the oracle run from x on {int(bad.sum())} of {len(bad)} tokens "
          f"(max distance change {delta:.3g}, threshold {t:.6g})", flush=True)
    assert np.all(band <= 2 * delta * (1 + 1e-9) + 1e-12 * abs(t)), f"{what}: keep change outside the 2-delta band"
    assert int(bad.sum()) <= max(2, int(max_frac * len(bad))), f"{what}: {int(bad.sum())} keep changes"
    return int(bad.sum())


def check_gated_end_to_end(q_dev, q_ora, keys, sel, vis, reuse, hit, idx, thr_v, thr_t, cmp, col_offset=0,
                           what="", max_qdiff_frac=0.01):
    """Mode-R (hit, idx) from x: O.search_gated on the oracle's own queries
    against the device's results (all arrays host-side, the rows already
    selected).  A hit flag may differ only within the near-threshold rule on
    the oracle's exact maximum, a hit index only within the near-tie rule on
    the oracle's exact scores, or in a row whose device query differs from
    the oracle's; the last kind is counted, printed and bounded."""
    want_hit, _, mx, scores = O.search_gated(np.asarray(q_ora), keys, sel, vis, reuse, thr_v, thr_t, cmp,
                                             col_offset=col_offset)
    qdiff = np.any(np.asarray(q_dev) != np.asarray(q_ora), axis=1)
    got_hit = np.asarray(hit).astype(bool)
    got_idx = np.asarray(idx)
    n_rule = n_q = n_slots = 0
    for i in range(got_hit.shape[0]):
        thr = float(np.float32(thr_v if vis[i] else thr_t))
        for s in range(got_hit.shape[1]):
            if np.isnan(mx[i, s]):
                continue
            n_slots += 1
            hit_ok = got_hit[i, s] == want_hit[i, s]
            idx_ok = not got_hit[i, s] or not want_hit[i, s] or got_idx[i, s] == int(np.argmax(scores[i, s]))
            if hit_ok and idx_ok:
                continue
            rule = O.threshold_ok(mx[i, s], thr, got_hit[i, s], want_hit[i, s]) and (
                not got_hit[i, s] or O.gap_ok(scores[i, s], int(got_idx[i, s]), int(np.argmax(scores[i, s])), True))
            if rule:
                n_rule += 1
            elif qdiff[i]:
                n_q += 1
            else:
                raise AssertionError(f"{what}: row {i} slot {s}: hit {got_hit[i, s]} idx {got_idx[i, s]} vs the "
                                     f"oracle's {want_hit[i, s]} / {int(np.argmax(scores[i, s]))} (max {mx[i, s]})")
    bound = max(1, int(max_qdiff_frac * max(n_slots, 1)))
    print(f"[e2e] {what}: {int(qdiff.sum())}/{len(qdiff)} query rows differ from the oracle's; of {n_slots} "
          f"searched slots {n_rule} differ within the threshold/tie rules, {n_q} in rows with another query "
          f"(bound {bound})", flush=True)
    assert n_q <= bound, f"{what}: {n_q} result changes from query differences > {bound}"
    return n_rule, n_q
