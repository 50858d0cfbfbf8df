"""How often the reference's torch fallback picks a different cluster, or a
different hit, than this build on the Qwen-shape mode-R prefill workload
(CPU, oracle arithmetic).

The fallback (table_moe/cache_engine/search.py:595-597 cosine, :689-691 dot)
computes scores with a bf16 ``torch.bmm`` -- fp32 accumulation, one rounding
to bf16 -- takes ``max`` (the first maximal index) of the ROUNDED scores and
compares the rounded maximum with a Python float threshold, which torch casts
to bf16 as well (0.7 becomes 0.69921875).  The Triton kernels the build
replaces, and the build itself, rank fp32 scores and compare them with the
fp32 threshold.  The test measures both rates, prints them, and checks that
every difference is a bf16-level effect: a changed pick lies within one bf16
rounding of the exact maximum, a changed hit has its exact maximum within
one bf16 rounding of the threshold."""

import numpy as np
import torch

from oracle import tm_oracle as O

E, K, D, H, TOPK = 128, 256, 64, 2048, 8


def _workload(seed=7):
    from synth import make_workload

    wl = make_workload(2, with_slot_out=False)
    n = wl.x.shape[0]
    g = torch.Generator().manual_seed(seed)
    raw = torch.randn(E, 2, K, D, generator=g)
    keys_n = (raw / raw.norm(dim=-1, keepdim=True).clamp_min(1e-6)).to(torch.bfloat16)
    keys_raw = raw.to(torch.bfloat16)
    pca = {}
    for mod in ("vision", "text"):
        p = torch.linalg.qr(torch.randn(H, D, generator=g))[0].to(torch.bfloat16)
        pca[mod] = (p, (torch.randn(D, generator=g) * 0.05).to(torch.bfloat16))
    _, sel, _ = O.topk_softmax(wl.logits.double().numpy(), TOPK)
    reuse = torch.rand(n, TOPK, generator=g).numpy() < 0.6
    # half the tokens lifted near a key of their first expert (as the GPU test of this search does)
    near = torch.rand(n, generator=g).numpy() < 0.5
    isv = wl.is_vision.numpy()
    j = torch.randint(0, K, (n,), generator=g).numpy()
    src = keys_n.double().numpy()[sel[:, 0], np.where(isv, 0, 1), j]
    pv, pt = pca["vision"][0].double().numpy(), pca["text"][0].double().numpy()
    lift = np.where(isv[:, None], src @ pv.T, src @ pt.T) * 4.0
    x = wl.x.double().numpy()
    x = np.where(near[:, None], x * 0.2 + lift, x)
    x = torch.from_numpy(x).to(torch.bfloat16).double().numpy()
    return x, isv, sel, reuse, keys_n.double().numpy(), keys_raw.double().numpy(), \
        {m: (p.double().numpy(), b.double().numpy()) for m, (p, b) in pca.items()}


def _compare(q, keys, sel, isv, reuse, thr_v, thr_t, ge):
    bf = lambda v: O.round_to(v, O.BF16)  # noqa: E731
    rows, cols = np.nonzero(reuse)
    mods = np.where(isv[rows], 0, 1)
    tabs = keys[sel[rows, cols], mods]  # [m, K, D]
    exact = np.einsum("mkd,md->mk", tabs, q[rows])
    thr = np.where(isv[rows], np.float32(thr_v), np.float32(thr_t)).astype(np.float64)
    thr_bf = bf(thr)
    # this build: fp32 scores (exact here), first maximum, fp32 threshold
    pick = exact.argmax(axis=1)
    mx = exact[np.arange(len(rows)), pick]
    hit = mx >= thr if ge else mx > thr
    # the fallback: bf16 scores (one rounding of the fp32 sum), first maximum, bf16 threshold
    rs = bf(exact.astype(np.float32).astype(np.float64))
    pick_r = rs.argmax(axis=1)
    mx_r = rs[np.arange(len(rows)), pick_r]
    hit_r = mx_r >= thr_bf if ge else mx_r > thr_bf
    both = hit & hit_r
    d_pick = both & (pick != pick_r)
    d_hit = hit != hit_r
    u = 2.0 ** -8  # bf16 unit roundoff
    # a changed pick: the fallback's choice is within one bf16 rounding of the exact maximum
    gap = mx[d_pick] - exact[np.arange(len(rows))[d_pick], pick_r[d_pick]]
    assert np.all(gap <= 2 * u * np.abs(mx[d_pick]) + 1e-12)
    # a changed hit: the exact maximum lies within one bf16 rounding of the threshold
    assert np.all(np.abs(mx[d_hit] - thr[d_hit]) <= 2 * u * np.maximum(np.abs(mx[d_hit]), np.abs(thr[d_hit])) + 1e-12)
    return len(rows), int(both.sum()), int(d_pick.sum()), int(d_hit.sum())


def test_fallback_bf16_scores_change_rate():
    x, isv, sel, reuse, keys_n, keys_raw, pca = _workload()
    q_cos = O.project_queries(x, isv, pca["vision"], pca["text"], True, O.BF16)
    q_dot = O.project_queries(x, isv, pca["vision"], pca["text"], False, O.BF16)
    for name, q, keys, tv, tt, ge in (("cosine (prefill offline)", q_cos, keys_n, 0.6, 0.7, True),
                                      ("dot (prefill offline dot)", q_dot, keys_raw, 0.0, 0.0, False)):
        n_s, n_both, n_pick, n_hit = _compare(q, keys, sel, isv, reuse, tv, tt, ge)
        print(f"[fallback rounding] {name}: {n_s} searched slots, {n_hit} hit flags differ "
              f"({n_hit / n_s:.2e}), {n_pick} of {n_both} common hits pick another cluster "
              f"({n_pick / max(n_both, 1):.2e})", flush=True)
        assert n_s > 15000 and n_both > 1000
        # bf16-level effects stay rare on this workload
        assert n_pick / n_both < 0.05 and n_hit / n_s < 0.05
