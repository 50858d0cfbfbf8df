"""Pins the CPU oracle (oracle/tm_oracle.py) before it is trusted as the checker.

Each check is independent of the oracle's own formula: the reference's known-
answer tests (table_moe/cache_engine/test_search.py:48-89,
table_moe/skip/test_pruning.py:109-327), library routines (numpy/torch casts,
torch CPU ops), closed forms and brute force on tiny inputs.
"""

import itertools

import numpy as np
import pytest
import torch

from oracle import tm_oracle as O


# ----------------------------------------------------------------- rounding
def test_round_to_matches_library_casts():
    rng = np.random.default_rng(0)
    x32 = (rng.standard_normal(50000) * np.exp(rng.standard_normal(50000) * 4)).astype(np.float32)
    want_bf16 = torch.from_numpy(x32).to(torch.bfloat16).double().numpy()
    np.testing.assert_array_equal(O.round_to(x32.astype(np.float64), O.BF16), want_bf16)
    want_f16 = x32.astype(np.float16).astype(np.float64)
    np.testing.assert_array_equal(O.round_to(x32.astype(np.float64), O.F16), want_f16)


def test_round_to_ties_to_even():
    # 1 + 2^-8 is halfway between bf16 1.0 and 1.0078125: even mantissa wins
    assert O.round_to(np.array([1.0 + 2**-8]), O.BF16)[0] == 1.0
    assert O.round_to(np.array([1.0 + 3 * 2**-8]), O.BF16)[0] == 1.0 + 2**-6
    assert O.round_to(np.array([1.0 + 2**-11]), O.F16)[0] == 1.0


# ------------------------------------------------------------ a1 top-k softmax
def test_topk_softmax_closed_form():
    logits = np.array([[8.0, 7.0, 6.0, 5.0, 4.0, 3.0, 2.0, 1.0], [1.0, 8.0, 7.0, 6.0, 5.0, 4.0, 3.0, 2.0]])
    w, ids, _ = O.topk_softmax(logits, 5)
    z = np.exp(np.arange(8, 0, -1.0))
    p = z / z.sum()
    np.testing.assert_allclose(w[0], p[:5], rtol=1e-12)
    np.testing.assert_array_equal(ids[0], [0, 1, 2, 3, 4])
    np.testing.assert_array_equal(ids[1], [1, 2, 3, 4, 5])
    wn, _, _ = O.topk_softmax(logits, 5, renormalize=True)
    np.testing.assert_allclose(wn.sum(1), 1.0, rtol=1e-12)


def test_topk_softmax_ties_go_to_lower_id():
    logits = np.array([[1.0, 3.0, 3.0, 0.0, 3.0]])
    _, ids, _ = O.topk_softmax(logits, 3)
    np.testing.assert_array_equal(ids[0], [1, 2, 4])


def test_topk_softmax_brute_force():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((64, 16))
    w, ids, p = O.topk_softmax(logits, 4)
    for r in range(64):
        order = sorted(range(16), key=lambda e: (-p[r, e], e))[:4]
        assert list(ids[r]) == order
        np.testing.assert_allclose(w[r], np.exp(logits[r][order]) / np.exp(logits[r]).sum(), rtol=1e-12)


# ------------------------------------------------------------ a2 modality
def test_modality_mask():
    ids = np.array([[1, 151655, 5, 151656, 151657]])
    np.testing.assert_array_equal(O.modality_mask(ids), [[False, True, False, True, False]])
    np.testing.assert_array_equal(O.modality_mask(ids, seq_len=1), [[False]])
    np.testing.assert_array_equal(O.modality_mask(ids, seq_len=3), [[False, True, False]])


# ------------------------------------------------------- a3 masks, renorm
def test_fixed_keep_mask_reference_kat():
    # table_moe/skip/test_pruning.py:109-113
    sel = np.array([[0, 1, 2, 3], [4, 5, 6, 7]])
    want = np.array([[True, True, False, False], [True, True, False, False]])
    np.testing.assert_array_equal(O.build_fixed_keep_mask(sel, 2), want)
    np.testing.assert_array_equal(O.build_fixed_keep_mask(sel, None), np.ones_like(want))
    np.testing.assert_array_equal(O.build_fixed_keep_mask(sel, 9), np.ones_like(want))


def test_renormalize_reference_kat():
    # table_moe/skip/test_pruning.py:115-120
    out = O.renormalize_surviving_weights([[0.4, 0.3, 0.2, 0.1]], [[True, True, False, False]])
    np.testing.assert_allclose(out, [[4 / 7, 3 / 7, 0, 0]], atol=1e-6)


def test_renormalize_target_row_sum_kat():
    # DeepSeek target-row-sum expectation, table_moe/skip/test_pruning.py:214-217, :314-320
    w = np.array([[0.5, 0.4, 0.3, 0.2, 0.1, 0.05], [0.6, 0.3, 0.2, 0.1, 0.05, 0.02]], dtype=np.float32)
    keep = O.build_fixed_keep_mask(np.tile(np.arange(6), (2, 1)), 5)
    out = O.renormalize_surviving_weights(w, keep, target_row_sum=w.sum(-1, keepdims=True))
    kept = w[:, :5].astype(np.float64)
    want = kept * (w.sum(-1, keepdims=True) / kept.sum(-1, keepdims=True))
    np.testing.assert_allclose(out[:, :5], want, atol=1e-6)
    assert np.all(out[:, 5] == 0)


def test_renormalize_zero_survivors_and_bf16_steps():
    out = O.renormalize_surviving_weights([[0.3, 0.7], [0.5, 0.5]], [[False, False], [True, False]])
    np.testing.assert_array_equal(out[0], [0, 0])
    np.testing.assert_array_equal(out[1], [1.0, 0])
    # bf16 arithmetic agrees with torch's bf16 ops on CPU step by step
    rng = np.random.default_rng(2)
    w = torch.from_numpy(rng.random((256, 8)).astype(np.float32)).to(torch.bfloat16)
    m = torch.from_numpy(rng.random((256, 8)) < 0.6)
    pruned = w * m.to(w.dtype)
    s = pruned.sum(-1, keepdim=True)
    want = torch.where(s > 0, pruned / s, torch.zeros_like(pruned)).double().numpy()
    got = O.renormalize_surviving_weights(w.double().numpy(), m.numpy(), dt=O.BF16)
    assert np.mean(got == want) > 0.99
    np.testing.assert_allclose(got, want, atol=2**-8)


def _prefill_keep_brute(sel, w, attn, n_exp, keep_rate):
    scores = {}
    n = len(sel)
    for b, row in enumerate(sel):
        for s, e in enumerate(row):
            c = (attn[b] * w[b][s]) if attn is not None else w[b][s] / n
            scores[e] = scores.get(e, 0.0) + c
    active = sorted(scores)
    ranked = sorted(active, key=lambda e: (-scores[e], e))
    n_keep = min(max(1, int(len(active) * keep_rate)), len(active))
    kept = set(ranked[:n_keep])
    return np.array([[e in kept for e in row] for row in sel])


def test_prefill_keep_mask_brute_force():
    rng = np.random.default_rng(3)
    for trial in range(40):
        n, k, e = int(rng.integers(1, 12)), int(rng.integers(1, 5)), int(rng.integers(2, 9))
        sel = np.stack([rng.choice(e, size=k, replace=False) if k <= e else rng.integers(0, e, k) for _ in range(n)])
        w = rng.random((n, k))
        attn = rng.random(n) if trial % 2 else None
        kr = float(rng.choice([0.1, 0.25, 0.5, 0.6, 0.75, 1.0]))
        got, _ = O.build_prefill_keep_mask(sel, w, attn, e, kr)
        np.testing.assert_array_equal(got, _prefill_keep_brute(sel.tolist(), w.tolist(),
                                                                None if attn is None else attn.tolist(), e, kr))


def test_prefill_keep_mask_closed_form():
    # experts 3 (score .9), 1 (.5), 7 (.2): keep_rate .6 -> int(3*.6)=1 expert kept
    sel = np.array([[3, 1], [7, 3]])
    w = np.array([[0.5, 0.5], [0.2, 0.4]])
    mask, sums = O.build_prefill_keep_mask(sel, w, np.ones(2), 8, 0.6)
    np.testing.assert_allclose(sums[[1, 3, 7]], [0.5, 0.9, 0.2])
    np.testing.assert_array_equal(mask, [[True, False], [False, True]])
    # equal scores: the lower expert id ranks first
    mask, _ = O.build_prefill_keep_mask(np.array([[5, 2]]), np.array([[0.5, 0.5]]), None, 8, 0.5)
    np.testing.assert_array_equal(mask, [[False, True]])


# ------------------------------------------------------------ a4 projection
def test_projection_identity_pca_closed_form():
    rng = np.random.default_rng(4)
    x = O.round_to(rng.standard_normal((16, 8)), O.BF16)
    P = np.zeros((8, 4))
    P[:4, :4] = np.eye(4)
    b = O.round_to(rng.standard_normal(4), O.BF16)
    q = O.project_queries(x, np.ones(16, bool), (P, b), (P, b), normalize=False, dt=O.BF16)
    np.testing.assert_array_equal(q, O.round_to(x[:, :4] + b, O.BF16))


def test_projection_matches_torch_cpu_ops():
    """addmm / vector_norm / div in bf16 on CPU (the reference's op sequence,
    search.py:484-486 and :12-21) agree with the restatement up to 1 ulp."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(64, 256, generator=g).to(torch.bfloat16)
    P = torch.linalg.qr(torch.randn(256, 32, generator=g))[0].to(torch.bfloat16)
    b = (torch.randn(32, generator=g) * 0.1).to(torch.bfloat16)
    low = torch.addmm(b, x, P)
    norms = torch.linalg.vector_norm(low, dim=-1, keepdim=True)
    want = (low / norms.clamp_min(1e-6)).double().numpy()
    got = O.project_queries(x.double().numpy(), np.ones(64, bool), (P.double().numpy(), b.double().numpy()),
                            None, normalize=True, dt=O.BF16)
    ulp = np.abs(want) * 2**-7 + 1e-30
    assert np.all(np.abs(got - want) <= ulp)
    assert np.mean(got == want) > 0.97
    raw = O.project_queries(x.double().numpy(), np.ones(64, bool), (P.double().numpy(), b.double().numpy()),
                            None, normalize=False, dt=O.BF16)
    assert np.mean(raw == low.double().numpy()) > 0.97


def test_normalize_zero_rows():
    q = O.normalize_rows(np.array([[0.0, 0.0], [3.0, 4.0]]), O.F32)
    np.testing.assert_allclose(q, [[0, 0], [0.6, 0.8]], rtol=1e-7)


# --------------------------------------------------------- a5-a7 gated search
def _dummy_tables():
    # DummyManager of table_moe/cache_engine/test_search.py:11-26 with the raw
    # keys set by :30-41
    raw = np.zeros((2, 2, 2, 2))
    raw[0, 0] = [[1.0, 0.0], [-1.0, 0.0]]
    raw[1, 0] = [[0.0, 0.0], [-1.0, 0.0]]
    return raw


@pytest.mark.parametrize("projection", ["prefill", "decode"])
def test_search_dot_reference_kat(projection):
    # test_search.py:48-67 (prefill dot) and :69-89 (decode dot, fallback)
    raw = _dummy_tables()
    x = np.array([[1.0, 0.0], [1.0, 0.0]])
    eye = (np.eye(2), np.zeros(2))
    q = O.project_queries(x, np.array([True, True]), eye, eye, normalize=False, dt=O.F32)
    hit, idx, _, _ = O.search_gated(q, raw, np.array([[0], [1]]), np.array([True, True]),
                                    np.array([[True], [True]]), 0.0, 0.0, O.CMP_GT)
    assert hit[0, 0] and idx[0, 0] == 0
    assert not hit[1, 0]


def test_search_gated_comparators_and_reuse():
    keys = np.zeros((1, 2, 3, 2))
    keys[0, 0] = [[0.6, 0.0], [0.2, 0.0], [0.6, 0.0]]  # max 0.6 twice: first index
    keys[0, 1] = [[0.1, 0.0], [0.7, 0.0], [0.0, 0.0]]
    q = np.array([[1.0, 0.0], [1.0, 0.0], [1.0, 0.0]])
    vis = np.array([True, False, True])
    sel = np.zeros((3, 2), dtype=np.int64)
    reuse = np.array([[True, True], [True, False], [False, False]])
    thr_v, thr_t = float(np.float32(0.6)), float(np.float32(0.7))
    keys[0, 0, 0, 0] = keys[0, 0, 2, 0] = thr_v
    keys[0, 1, 1, 0] = thr_t
    hit, idx, mx, _ = O.search_gated(q, keys, sel, vis, reuse, 0.6, 0.7, O.CMP_GE)
    np.testing.assert_array_equal(hit, [[True, True], [True, False], [False, False]])
    np.testing.assert_array_equal(idx, [[0, 0], [1, 0], [0, 0]])
    hit, _, _, _ = O.search_gated(q, keys, sel, vis, reuse, 0.6, 0.7, O.CMP_GT)
    assert not hit.any()


def test_search_gated_brute_force():
    rng = np.random.default_rng(6)
    keys = rng.standard_normal((5, 2, 7, 3))
    q = rng.standard_normal((9, 3))
    sel = rng.integers(0, 5, (9, 4))
    vis = rng.random(9) < 0.5
    reuse = rng.random((9, 4)) < 0.7
    hit, idx, mx, _ = O.search_gated(q, keys, sel, vis, reuse, 0.1, -0.2, O.CMP_GE)
    for b, s in itertools.product(range(9), range(4)):
        if not reuse[b, s]:
            assert not hit[b, s] and idx[b, s] == 0
            continue
        sc = [float(np.dot(q[b], keys[sel[b, s], 0 if vis[b] else 1, c])) for c in range(7)]
        best = max(sc)
        first = sc.index(best)
        want = best >= (float(np.float32(0.1)) if vis[b] else float(np.float32(-0.2)))
        assert hit[b, s] == want
        assert idx[b, s] == (first if want else 0)


# ------------------------------------------------------------- a8 hybrid
def test_search_hybrid_closed_form():
    # online window: 3 valid entries; token 0 best matches entry 2 (score 2 > 0)
    x = np.array([[1.0, 0.0], [-1.0, 0.0]])
    on_keys = np.array([[0.5, 0.0], [1.0, 0.0], [2.0, 0.0], [9.0, 0.0]])
    on_ids = np.array([[4, 5], [6, 7], [7, 3], [1, 1]])
    keys = np.zeros((8, 2, 2, 2))
    keys[:, :, 0] = [0.0, 1.0]
    keys[:, :, 1] = [1.0, 0.0]
    eye = (np.eye(2), np.zeros(2))
    sel = np.array([[0, 3, 7, 5], [1, 3, 7, 5]])
    r = O.search_hybrid(x, np.array([False, False]), eye, eye, O.F32, keys, sel, 1, on_keys, on_ids, 3)
    # token 0: j*=2 (ids 7,3): slot1 (3) hit at position 1, slot2 (7) at 0, slot3 (5) miss -> offline
    np.testing.assert_array_equal(r["on_idx"], [2, -1])
    np.testing.assert_array_equal(r["on_hit"][0], [False, True, True, False])
    np.testing.assert_array_equal(r["on_slot"][0], [0, 1, 0, 0])
    # offline for token 0 slot 3: q=[1,0]: centroid 1 scores 1 >= 0 -> hit idx 1
    np.testing.assert_array_equal(r["off_hit"][0], [False, False, False, True])
    np.testing.assert_array_equal(r["off_idx"][0], [0, 0, 0, 1])
    # token 1: all online scores < 0 -> no online hit; offline q=[-1,0]: scores (0,-1): max 0 >= 0 -> hit idx 0
    assert not r["on_hit"][1].any()
    np.testing.assert_array_equal(r["off_hit"][1], [False, True, True, True])
    np.testing.assert_array_equal(r["off_idx"][1], [0, 0, 0, 0])


def test_search_hybrid_without_window_and_keep_all():
    keys = np.zeros((2, 2, 1, 2))
    keys[:, :, 0] = [1.0, 0.0]
    eye = (np.eye(2), np.zeros(2))
    r = O.search_hybrid(np.array([[1.0, 0.0]]), np.array([True]), eye, eye, O.F32, keys, np.array([[0, 1]]), 0,
                        None, None, 0)
    np.testing.assert_array_equal(r["off_hit"], [[True, True]])
    r = O.search_hybrid(np.array([[1.0, 0.0]]), np.array([True]), eye, eye, O.F32, keys, np.array([[0, 1]]), 2,
                        None, None, 0)
    assert not r["off_hit"].any() and r["on_idx"][0] == -1


# ------------------------------------------------------ a12 online window
def test_online_update_brute_force():
    rng = np.random.default_rng(7)
    size, k, h = 5, 2, 3
    st = dict(keys=np.zeros((size, h)), ids=np.full((size, k), -1), values=np.zeros((size, k, h)), ptr=0,
              full=False, size=size)
    stream = []  # every row written, in order
    for _ in range(12):
        n = int(rng.integers(1, 8))
        hid = rng.standard_normal((n, h))
        ids = rng.integers(0, 9, (n, k))
        out = rng.standard_normal((n, k, h))
        valid = rng.random((n, k)) < 0.7
        st = O.online_update(st, hid, ids, out, valid)
        m = min(n, size)
        for i in range(n - m, n):
            stream.append((hid[i], np.where(valid[i], ids[i], -1), np.where(valid[i][:, None], out[i], 0)))
        assert st["ptr"] == len(stream) % size
        assert st["full"] == (len(stream) >= size)
    for r in range(size):
        last = max(g for g in range(len(stream)) if g % size == r)
        np.testing.assert_array_equal(st["keys"][r], stream[last][0])
        np.testing.assert_array_equal(st["ids"][r], stream[last][1])
        np.testing.assert_array_equal(st["values"][r], stream[last][2])


# --------------------------------------------------------- a11 slot combine
def test_slot_combine_constant_experts_closed_form():
    # as the wrapper KATs of test_pruning.py:183-250: expert i outputs (i+1)
    w = np.array([[0.5, 0.4, 0.3, 0.2, 0.1, 0.05]])
    collected = np.stack([np.full((1, 3), i + 1.0) for i in range(6)], axis=1)
    keep = O.build_fixed_keep_mask(np.arange(6)[None], 5)
    out, wt = O.slot_combine(collected, w, keep, O.F32, target_mode="orig_sum")
    kept = w[:, :5]
    ew = kept * (w.sum(-1, keepdims=True) / kept.sum(-1, keepdims=True))
    np.testing.assert_allclose(out, np.full((1, 3), (ew * np.arange(1, 6)).sum()), rtol=1e-6)
    out, _ = O.slot_combine(collected, w, keep, O.F32, target_mode="one")
    np.testing.assert_allclose(out, np.full((1, 3), (kept / kept.sum() * np.arange(1, 6)).sum()), rtol=1e-6)


# ------------------------------------------------------------ mode G
def test_global_search_brute_force_and_self_match():
    rng = np.random.default_rng(8)
    c = O.round_to(rng.standard_normal((300, 16)), O.BF16)
    q = O.round_to(rng.standard_normal((40, 16)), O.BF16)
    vals, idx, full = O.global_search(q, c, 4)
    for r in range(40):
        d = [float(((q[r] - c[j]) ** 2).sum()) for j in range(300)]
        order = sorted(range(300), key=lambda j: (d[j], j))[:4]
        assert list(idx[r]) == order
        np.testing.assert_allclose(vals[r], [d[j] for j in order], rtol=1e-9, atol=1e-9)
    v, i, _ = O.global_search(c[:50], c, 1)
    np.testing.assert_array_equal(i[:, 0], np.arange(50))
    np.testing.assert_allclose(v[:, 0], 0.0, atol=1e-9)
    vd, idd, _ = O.global_search(q, c, 2, metric="dot")
    for r in range(5):
        s = [float(np.dot(q[r], c[j])) for j in range(300)]
        assert list(idd[r]) == sorted(range(300), key=lambda j: (-s[j], j))[:2]


def test_keep_select_brute_force_and_ties():
    rng = np.random.default_rng(9)
    for _ in range(30):
        n = int(rng.integers(1, 60))
        s = rng.integers(0, 6, n).astype(np.float64)  # many ties
        k = int(rng.integers(0, n + 1))
        keep = O.keep_select(s, k)
        order = sorted(range(n), key=lambda i: (-s[i], i))[:k]
        np.testing.assert_array_equal(np.nonzero(keep)[0], sorted(order))
    assert O.keep_count(4096, 0.6) == 2457 and O.keep_count(1, 0.6) == 1 and O.keep_count(32, 0.6) == 19


def test_gather_combine_closed_form_one_hot():
    H = 6
    values = np.eye(H)                    # centroid c outputs e_c
    idx = np.array([[2, 4], [0, 1], [5, 3]])
    dist = np.array([[1.0, 3.0], [0.0, 1.0], [2.0, 2.0]])
    keep = np.array([False, True, False])
    slot_out = np.zeros((3, 2, H))
    slot_out[1, 0] = 1.0
    slot_out[1, 1, 0] = 4.0
    w = np.array([[0.1, 0.2], [0.3, 0.1], [1.0, 1.0]])
    out = O.gather_combine(keep, slot_out, w, values, idx, dist, np.zeros((3, H)), O.F32)
    b0 = np.array([1 / (1 + 1e-6), 1 / (3 + 1e-6)])
    b0 /= b0.sum()
    np.testing.assert_allclose(out[0], b0[0] * values[2] + b0[1] * values[4], rtol=1e-6)
    np.testing.assert_allclose(out[1], 0.75 * slot_out[1, 0] + 0.25 * slot_out[1, 1], rtol=1e-6)
    np.testing.assert_allclose(out[2], 0.5 * values[5] + 0.5 * values[3], rtol=1e-6)


def test_layer_fp32_baseline_agrees_with_oracle():
    from synth import make_workload

    wl = make_workload(1, n=64)
    args = [t.double().numpy() if isinstance(t, torch.Tensor) else t for t in
            (wl.x, wl.is_vision, (wl.proj_vis, wl.bias_vis), (wl.proj_txt, wl.bias_txt), wl.centroids,
             wl.values, wl.logits, wl.slot_out, wl.residual)]
    args[2] = tuple(t.double().numpy() for t in args[2])
    args[3] = tuple(t.double().numpy() for t in args[3])
    ref = O.layer_forward_g(*args, 8, 1, 0.6, dt=O.F32)
    fast = O.layer_forward_g_fp32(*args, 8, 1, 0.6)
    np.testing.assert_allclose(fast, ref["out"], rtol=1e-4, atol=1e-4)


# ------------------------------------------------------- recompute: SwiGLU MLP
def test_swiglu_expert_one_hot_closed_form():
    """One-hot weights route single coordinates: W1 picks x_a (gate), W3 picks
    x_b (up), W2 routes intermediate column j to output c.  The output is then
    dt(dt(silu(dt(x_a))) * x_b)) evaluated with scalar math.exp: pins which
    matrix is the gate, which the up projection, the orientation of each, and
    the rounding points (g rounded, up unrounded, f rounded, y rounded)."""
    import math

    rng = np.random.default_rng(7)
    H, I = 16, 8
    x = O.round_to(rng.normal(size=(5, H)) * 3, O.BF16)
    a = rng.integers(0, H, I)
    b = rng.integers(0, H, I)
    c = rng.permutation(H)[:I]
    w1 = np.zeros((I, H)); w1[np.arange(I), a] = 1.0
    w3 = np.zeros((I, H)); w3[np.arange(I), b] = 1.0
    w2 = np.zeros((H, I)); w2[c, np.arange(I)] = 1.0
    y, f = O.swiglu_expert(x, w1, w3, w2, O.BF16)
    for r in range(x.shape[0]):
        for j in range(I):
            g = float(O.round_to(x[r, a[j]], O.BF16))
            want_f = float(O.round_to(g / (1.0 + math.exp(-g)) * x[r, b[j]], O.BF16))
            assert f[r, j] == want_f
            assert y[r, c[j]] == want_f  # one term: the down projection only rounds it again
    others = np.setdiff1d(np.arange(H), c)
    assert np.all(y[:, others] == 0.0)


def test_swiglu_expert_addend_closed_forms():
    """The addend form (shared experts folded into the residual): a zero
    addend gives the plain MLP bit for bit; zero down weights give the addend
    rounded once; with one-hot weights, dt(addend + f) where f is the routed
    intermediate, so the addend enters before the single final rounding (the
    sum of two bf16 values generally needs that rounding)."""
    rng = np.random.default_rng(11)
    H, I, M = 16, 8, 6
    x = O.round_to(rng.normal(size=(M, H)), O.BF16)
    w1 = O.round_to(rng.normal(size=(I, H)) * 0.3, O.BF16)
    w3 = O.round_to(rng.normal(size=(I, H)) * 0.3, O.BF16)
    w2 = O.round_to(rng.normal(size=(H, I)) * 0.3, O.BF16)
    r = O.round_to(rng.normal(size=(M, H)) * 5, O.BF16)
    plain, _ = O.swiglu_expert(x, w1, w3, w2, O.BF16)
    zero, _ = O.swiglu_expert(x, w1, w3, w2, O.BF16, addend=np.zeros((M, H)))
    np.testing.assert_array_equal(plain, zero)
    only, _ = O.swiglu_expert(x, w1, w3, np.zeros((H, I)), O.BF16, addend=r)
    np.testing.assert_array_equal(only, r)
    c = rng.permutation(H)[:I]
    w2h = np.zeros((H, I)); w2h[c, np.arange(I)] = 1.0
    y, f = O.swiglu_expert(x, w1, w3, w2h, O.BF16, addend=r)
    np.testing.assert_array_equal(y[:, c], O.round_to(r[:, c] + f, O.BF16))
    assert not np.array_equal(y[:, c], r[:, c] + f)  # the exact sum is not a bf16 value everywhere


def test_swiglu_expert_matches_torch_silu_and_matmul():
    """Against torch's own silu and float64 matmul (library routines) with the
    same rounding points; and the up projection is NOT rounded before the
    product (rounding it, as the unfused torch expert does, changes results)."""
    import torch

    rng = np.random.default_rng(3)
    H, I, M = 64, 32, 9
    x = O.round_to(rng.normal(size=(M, H)), O.BF16)
    w1 = O.round_to(rng.normal(size=(I, H)) * 0.2, O.BF16)
    w3 = O.round_to(rng.normal(size=(I, H)) * 0.2, O.BF16)
    w2 = O.round_to(rng.normal(size=(H, I)) * 0.2, O.BF16)
    y, f = O.swiglu_expert(x, w1, w3, w2, O.BF16)
    tx, t1, t3, t2 = (torch.from_numpy(v) for v in (x, w1, w3, w2))
    g = torch.from_numpy(O.round_to((tx @ t1.T).numpy(), O.BF16))
    tf = O.round_to((torch.nn.functional.silu(g) * (tx @ t3.T)).numpy(), O.BF16)
    np.testing.assert_allclose(f, tf, rtol=0, atol=0)
    ty = O.round_to((torch.from_numpy(tf) @ t2.T).numpy(), O.BF16)
    np.testing.assert_array_equal(y, ty)
    f_rounded_up = O.round_to(O.silu(g.numpy()) * O.round_to((tx @ t3.T).numpy(), O.BF16), O.BF16)
    assert np.any(f_rounded_up != f)


def test_grouped_swiglu_regroups_pairs():
    rng = np.random.default_rng(5)
    E, H, I, N, K = 5, 16, 8, 11, 3
    x = rng.normal(size=(N, H))
    w1, w3 = rng.normal(size=(E, I, H)) * 0.3, rng.normal(size=(E, I, H)) * 0.3
    w2 = rng.normal(size=(E, H, I)) * 0.3
    ids = np.stack([rng.permutation(E)[:K] for _ in range(N)])
    mask = rng.random((N, K)) < 0.6
    out = O.grouped_swiglu(x, ids, mask, w1, w3, w2, O.F32)
    for bb in range(N):
        for s in range(K):
            if mask[bb, s]:
                want = O.swiglu_expert(x[bb:bb + 1], w1[ids[bb, s]], w3[ids[bb, s]], w2[ids[bb, s]], O.F32)[0][0]
                np.testing.assert_array_equal(out[bb, s], want)
            else:
                assert np.all(np.isnan(out[bb, s]))
    tok = O.grouped_swiglu(x, ids, mask[:, 0], w1, w3, w2, O.F32)  # per-token mask covers every slot
    assert np.isnan(tok).any(axis=2).sum() == (~mask[:, 0]).sum() * K


# ------------------------------------------- importance: last-query attention
def test_last_query_importance_matches_torch_softmax():
    """Against the reference's op sequence written with torch library calls
    (matmul of the model-dtype tensors, * scaling, softmax(dtype=float32),
    mean over heads; repeat_interleave for grouped KV heads), and the fp32
    variant with a key padding mask (masked_fill min, softmax, masked_fill 0,
    last query_length keys)."""
    import torch

    rng = np.random.default_rng(13)
    B, H, HKV, D, S = 2, 8, 2, 64, 40
    q = O.round_to(rng.normal(size=(B, H, D)), O.BF16)
    k = O.round_to(rng.normal(size=(B, S, HKV, D)), O.BF16)
    scale = D ** -0.5
    got = O.last_query_importance(q, k, HKV, scale, O.BF16)
    tq = torch.from_numpy(q).to(torch.bfloat16)[:, :, None, :]                   # [B, H, 1, D]
    tk = torch.from_numpy(k).to(torch.bfloat16).transpose(1, 2)                  # [B, HKV, S, D]
    tk = torch.repeat_interleave(tk, dim=1, repeats=H // HKV)
    score = torch.matmul(tq.float(), tk.float().transpose(2, 3)).to(torch.bfloat16) * scale  # bf16 rounding twice
    want = torch.softmax(score, dim=-1, dtype=torch.float32).mean(dim=1).squeeze(1).double().numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-9)

    mask = rng.random((B, S)) < 0.8
    got = O.last_query_importance(q, k, HKV, scale, O.F32, key_mask=mask, out_len=17)
    tqf = torch.from_numpy(q).float()
    tkf = torch.from_numpy(np.repeat(k, H // HKV, axis=2)).float()
    sc = torch.einsum("bhd,bkhd->bhk", tqf, tkf) * float(scale)
    km = torch.from_numpy(mask)
    sc = sc.masked_fill(~km[:, None, :], torch.finfo(sc.dtype).min)
    p = torch.softmax(sc, dim=-1, dtype=torch.float32).masked_fill(~km[:, None, :], 0.0)
    want = p[:, :, -17:].mean(dim=1).double().numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-9)


def test_last_query_importance_closed_forms():
    """Equal scores spread 1/S over the keys; one key whose score dominates
    takes ~all the mass; a fully masked row gives zeros."""
    B, H, D, S = 1, 4, 64, 10
    q = np.zeros((B, H, D)); q[..., 0] = 1.0
    k = np.zeros((B, S, 1, D)); k[..., 0] = 2.0
    np.testing.assert_allclose(O.last_query_importance(q, k, 1, 1.0, O.F32), np.full((1, S), 1.0 / S))
    k[0, 3, 0, 0] = 100.0
    got = O.last_query_importance(q, k, 1, 1.0, O.F32)
    assert got[0, 3] >= 1 - 1e-12 and np.all(got[0, np.arange(S) != 3] < 1e-40)
    got = O.last_query_importance(q, k, 1, 1.0, O.F32, key_mask=np.zeros((1, S), dtype=bool))
    assert np.all(got == 0.0)
