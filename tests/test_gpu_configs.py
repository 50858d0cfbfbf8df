"""GPU parity of the BASELINE configurations the single-layer tests do not
cover at full size: config 1 (fp32 layer, N=256, d=64, C=1024), config 4
(the 48-layer stack, N=2048 per layer, keep_rate swept over
{0.1, 0.25, 0.5, 0.75, 0.9, 1.0}) and config 5 end to end (DeepSeek-VL2-style
layer, hidden 2560, 64 routed experts top-6 + shared experts: table search,
grouped recompute of the kept tokens' slots, shared experts, combine)."""

import numpy as np
import pytest
import torch

from oracle import tm_oracle as O
from parity_util import (assert_bf16_output, assert_projection_close, check_end_to_end_keep, check_end_to_end_topk,
                         check_topk_rows, np64, proj_abssum, ulp)

pytestmark = pytest.mark.gpu

KEYS = ("weights", "ids", "q", "qn", "dist", "idx", "keep", "out")
KEEP_RATES = [0.1, 0.25, 0.5, 0.75, 0.9, 1.0]


def _table(d, metric="l2"):
    from table_moe.cache_engine import GlobalTable

    return GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt), metric=metric)


def check_layer_vs_oracle(res, wl, dt, residual, topk, what, proj_min_exact=0.95):
    """Each stage of one mode-G layer call against the oracle, on the device's
    own inputs to that stage: router (near-tie rule), projection (one rounding
    of the exact value, within the fp32 accumulation bound), nearest centroid
    of the device's q (near-tie rule), keep set of the device's distances
    (bit-exact), and the combined rows (one rounding of the exact value)."""
    _, wids, p = O.topk_softmax(np64(wl.logits), topk)
    check_topk_rows(p, np64(res["ids"]), wids, True, f"{what} router")
    isv = np64(wl.is_vision)
    x = np64(wl.x)
    q = np64(res["q"])
    odt = {torch.bfloat16: O.BF16, torch.float16: O.F16, torch.float32: O.F32}[dt]
    ref_q = O.project_queries(x, isv, (np64(wl.proj_vis), np64(wl.bias_vis)), (np64(wl.proj_txt), np64(wl.bias_txt)),
                              False, odt)
    abssum = proj_abssum(x, isv, np64(wl.proj_vis), np64(wl.proj_txt))
    if dt == torch.float32:  # fp32 results: the recursive-summation bound over 512-term partials, no exact floor
        bad = np.abs(q - ref_q) > ulp(ref_q, dt) + 2.0**-14 * abssum
        assert not bad.any(), f"{what} projection: {bad.sum()} values off"
    else:
        assert_projection_close(q, ref_q, abssum, dt, min_exact=proj_min_exact)
    _, want_idx, exact = O.global_search(q, np64(wl.centroids), 1)
    gi = np64(res["idx"])
    check_topk_rows(exact, gi, want_idx, False, f"{what} search")
    near = np64(wl.cluster_of) >= 0
    assert np.mean(gi[near, 0] == np64(wl.cluster_of)[near]) > 0.99, f"{what}: near tokens off their clusters"
    gd = np64(res["dist"])
    keep = np64(res["keep"])
    n = q.shape[0]
    np.testing.assert_array_equal(keep, O.keep_select(gd[:, 0], int(keep.sum())), err_msg=f"{what} keep")
    # end to end from x: the oracle's search and keep set on its own queries
    vals_o, _, _ = check_end_to_end_topk(q, ref_q, np64(wl.centroids), gi, f"{what} search")
    check_end_to_end_keep(gd[:, 0], vals_o[:, 0], keep, int(keep.sum()), f"{what} keep")
    want = O.gather_combine(keep, np64(wl.slot_out), np64(res["weights"]), np64(wl.values), gi, gd,
                            np64(residual), O.F32)
    absw = O.gather_combine(keep, np.abs(np64(wl.slot_out)), np64(res["weights"]), np.abs(np64(wl.values)), gi, gd,
                            np.abs(np64(residual)), O.F32)
    assert_bf16_output(np64(res["out"]), want, absw, dtype=dt)
    return n


# ------------------------------------------------------------------ config 1
def test_config1_fp32_layer_vs_oracle_and_staged(hip_device):
    """Config 1 at its stated precision: fp32 hidden states, PCA, centroids
    and cached outputs (N=256, H=2048, d=64, C=1024, top-1, keep 0.6 -> 153
    kept).  The one-call layer equals the five stage calls bit for bit, and
    every stage matches the oracle."""
    from synth import make_workload

    wl = make_workload(1)
    assert wl.x.dtype == torch.float32 and wl.x.shape == (256, 2048) and wl.centroids.shape == (1024, 64)
    d = wl.to(hip_device)
    a, b = _table(d), _table(d)
    ra = a.layer_forward(d.x, d.is_vision, d.logits, d.slot_out, d.residual, 8, 1, 0.6)
    rb = b.layer_forward_staged(d.x, d.is_vision, d.logits, d.slot_out, d.residual, 8, 1, 0.6)
    torch.cuda.synchronize()
    for key in KEYS:
        assert torch.equal(ra[key], rb[key]), key
    assert int(ra["keep"].sum()) == O.keep_count(256, 0.6) == 153
    check_layer_vs_oracle(ra, wl, torch.float32, wl.residual, 8, "config 1")
    # the whole layer against the oracle's own layer where the selections agree (all of them here)
    ref = O.layer_forward_g(np64(wl.x), np64(wl.is_vision), (np64(wl.proj_vis), np64(wl.bias_vis)),
                            (np64(wl.proj_txt), np64(wl.bias_txt)), np64(wl.centroids), np64(wl.values),
                            np64(wl.logits), np64(wl.slot_out), np64(wl.residual), 8, 1, 0.6, dt=O.F32)
    np.testing.assert_array_equal(np64(ra["idx"]), ref["idx"])
    np.testing.assert_array_equal(np64(ra["keep"]), ref["keep"])
    np.testing.assert_allclose(np64(ra["out"]), ref["out"], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("n,n_experts,top_k", [(77, 64, 6), (300, 128, 8)])
def test_fp32_layer_router_in_search_launch(hip_device, n, n_experts, top_k):
    """The fp32 layer's router rides in the search launch (extra grid rows of
    32 tokens each, numbered along the row blocks): token counts that leave
    the last router workgroup and row block ragged, 64 and 128 experts, the
    one-call layer against the stage calls (router launched on its own) bit
    for bit."""
    from synth import make_workload

    wl = make_workload(1, n=n, n_experts=n_experts, router_top_k=top_k)
    d = wl.to(hip_device)
    a, b = _table(d), _table(d)
    ra = a.layer_forward(d.x, d.is_vision, d.logits, d.slot_out, d.residual, top_k, 1, 0.6)
    rb = b.layer_forward_staged(d.x, d.is_vision, d.logits, d.slot_out, d.residual, top_k, 1, 0.6)
    torch.cuda.synchronize()
    for key in KEYS:
        assert torch.equal(ra[key], rb[key]), key
    assert int(ra["keep"].sum()) == O.keep_count(n, 0.6)


def test_config1_fp32_search_topk_and_dot(hip_device):
    """The fp32 search path beyond config 1's top-1 L2: top-4 and top-8 lists,
    the dot metric, d = 128/256, ragged centroid ranges and a decode-sized
    batch, against the oracle's brute force under the near-tie rule."""
    from table_moe import _native as N

    dev = hip_device
    for n, c, dim, k, metric in ((256, 1024, 64, 4, "l2"), (300, 1000, 128, 8, "dot"), (5, 3000, 256, 1, "l2"),
                                 (1030, 777, 64, 1, "dot")):
        g = torch.Generator().manual_seed(n + c + dim)
        q = torch.randn(n, dim, generator=g)
        cents = torch.randn(c, dim, generator=g)
        qd, cd = q.to(dev), cents.to(dev)
        csq = torch.empty(c, device=dev)
        N.call("tm_centroid_sqnorms", N.TM_DT_F32, N.ptr(cd), c, dim, dim, N.ptr(csq), N.stream(dev))
        nbytes = N.lib().tm_search_global_workspace_size(n, c, dim, k)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        dist = torch.empty(n, k, device=dev)
        idx = torch.empty(n, k, dtype=torch.long, device=dev)
        N.call("tm_search_global", N.TM_DT_F32, N.ptr(qd), n, dim, None, N.ptr(cd), c, dim, N.ptr(csq), dim, k,
               N.TM_METRIC_L2 if metric == "l2" else N.TM_METRIC_DOT, N.ptr(dist), N.ptr(idx), N.ptr(ws), nbytes,
               N.stream(dev))
        torch.cuda.synchronize()
        vals, want, exact = O.global_search(np64(q), np64(cents), k, metric)
        check_topk_rows(exact, np64(idx), want, metric == "dot", f"f32 n={n} c={c} d={dim} k={k} {metric}")
        np.testing.assert_allclose(np64(dist), np.take_along_axis(exact, np64(idx), 1), rtol=1e-4, atol=1e-3)


# ------------------------------------------------------------------ config 4
@pytest.fixture(scope="module")
def stack(hip_device):
    """The 48 layers of config 4 on the device (tables, hidden states, router
    logits, slot outputs, residual), and two table objects per layer: one for
    the one-call layer, one for the stage calls (separate output buffers)."""
    from synth import make_stack

    wls = make_stack(48, device=hip_device)
    torch.cuda.synchronize()
    return wls, [_table(w) for w in wls], [_table(w) for w in wls]


@pytest.mark.parametrize("ki,keep_rate", list(enumerate(KEEP_RATES)))
def test_config4_stack_keep_sweep(stack, ki, keep_rate):
    """The full 48-layer stack at one keep_rate, layers run in sequence with
    the residual stream chained (layer l's output is layer l + 1's
    residual): on every layer the keep count is max(1, int(2048 r)) and the
    one-call layer equals the stage calls bit for bit; two layers per
    keep_rate are checked stage by stage against the oracle."""
    wls, A, B = stack
    n = wls[0].x.shape[0]
    n_keep = O.keep_count(n, keep_rate)
    assert n_keep == max(1, int(n * keep_rate))
    check = {ki, 47 - ki}
    resid_a = resid_b = wls[0].residual
    outs_a = [torch.empty_like(w.residual) for w in wls]
    outs_b = [torch.empty_like(w.residual) for w in wls]
    for layer, w in enumerate(wls):
        if layer % 16 == 0:
            print(f"[config4] keep_rate {keep_rate} layer {layer}", flush=True)
        ra = A[layer].layer_forward(w.x, w.is_vision, w.logits, w.slot_out, resid_a, 8, 1, keep_rate,
                                    out=outs_a[layer])
        rb = B[layer].layer_forward_staged(w.x, w.is_vision, w.logits, w.slot_out, resid_b, 8, 1, keep_rate,
                                           out=outs_b[layer])
        torch.cuda.synchronize()
        for key in KEYS:
            assert torch.equal(ra[key], rb[key]), (layer, key)
        assert int(ra["keep"].sum()) == n_keep, layer
        if layer in check:
            check_layer_vs_oracle(ra, w, torch.bfloat16, resid_a, 8, f"config 4 layer {layer} keep {keep_rate}")
        resid_a, resid_b = outs_a[layer], outs_b[layer]


# ------------------------------------------------------------------ config 5
def test_config5_layer_end_to_end(hip_device):
    """Config 5 (hidden 2560, 64 routed experts top-6 + shared experts of
    intermediate 2 x 1536, N=4096, C=8192, d=128, keep 0.6) through
    GlobalTable.layer_forward_recompute: the layer call up to the keep set,
    GroupedExperts on the kept tokens' slots, the shared experts folded into
    the residual, the combine.  The full-size outputs equal the stage calls
    bit for bit; a token subset (kept and reused tokens of both modalities)
    is checked against the oracle: slot outputs against swiglu_expert,
    residual + shared against swiglu_expert with the addend, and the combined
    rows against gather_combine on the device's selections."""
    from synth import make_workload
    from table_moe.ops import GroupedExperts, expert_swiglu

    dev = hip_device
    wl = make_workload(5, with_slot_out=False, device=dev, gen_device=dev)
    cfg = wl.cfg
    n, h, e, k, inter = cfg["n"], cfg["hidden"], cfg["n_experts"], cfg["router_top_k"], 1536
    g = torch.Generator(device=dev).manual_seed(55)
    rnd = lambda *shape: (torch.randn(*shape, generator=g, device=dev) * 0.02).to(torch.bfloat16)  # noqa: E731
    w1, w3, w2 = rnd(e, inter, h), rnd(e, inter, h), rnd(e, h, inter)
    s1, s3, s2 = rnd(2 * inter, h), rnd(2 * inter, h), rnd(h, 2 * inter)
    a, b = _table(wl), _table(wl)
    ea, eb = GroupedExperts(w1, w3, w2), GroupedExperts(w1, w3, w2)
    ra = a.layer_forward_recompute(wl.x, wl.is_vision, wl.logits, ea, wl.residual, k, 0.6, shared=(s1, s3, s2))
    # the same layer as separate stage calls
    w, ids = b.route(wl.logits, k)
    q, qn = b.project(wl.x, wl.is_vision)
    dist, idx = b.search(q, 1, qn)
    keep = b.keep_select(dist[:, 0], b.keep_count(n, 0.6))
    slot = torch.empty(n, k, h, dtype=torch.bfloat16, device=dev)
    eb.forward(wl.x, ids, keep, slot)
    base = expert_swiglu(wl.x, s1, s3, s2, addend=wl.residual)
    out = b.gather_combine(keep, slot, w, idx, dist, base, torch.empty_like(wl.residual))
    torch.cuda.synchronize()
    for key, want in (("weights", w), ("ids", ids), ("q", q), ("qn", qn), ("dist", dist), ("idx", idx),
                      ("keep", keep), ("out", out)):
        assert torch.equal(ra[key], want), key
    kb = keep.bool()
    assert int(kb.sum()) == 2457
    assert torch.equal(ra["slot_out"][kb], slot[kb])
    # oracle on a subset: 24 kept and 24 reused tokens, vision and text
    isv = wl.is_vision.cpu().numpy()
    kp = kb.cpu().numpy()
    rows = np.concatenate([np.nonzero(kp & isv)[0][:16], np.nonzero(kp & ~isv)[0][:8],
                           np.nonzero(~kp & isv)[0][:16], np.nonzero(~kp & ~isv)[0][:8]])
    x = np64(wl.x)[rows]
    ids_h = np64(ids)[rows]
    slot_h = np64(ra["slot_out"])[rows]
    kept_i = [i for i, r in enumerate(rows) if kp[r]]
    for ex in sorted({int(ids_h[i, s]) for i in kept_i for s in range(k)}):  # one expert's weights at a time
        pairs = [(i, s) for i in kept_i for s in range(k) if int(ids_h[i, s]) == ex]
        want, _ = O.swiglu_expert(x[[i for i, _ in pairs]], np64(w1[ex]), np64(w3[ex]), np64(w2[ex]), O.BF16)
        got = np.stack([slot_h[i, s] for i, s in pairs])
        small = np.abs(want) < 8
        np.testing.assert_allclose(got[small], want[small], atol=1e-2, rtol=2e-3, err_msg=f"expert {ex}")
    want_base, _ = O.swiglu_expert(x, np64(s1), np64(s3), np64(s2), O.BF16, addend=np64(wl.residual)[rows])
    got_base = np64(base)[rows]
    small = np.abs(want_base) < 8
    np.testing.assert_allclose(got_base[small], want_base[small], atol=1e-2, rtol=2e-3)
    assert np.mean(got_base == want_base) > 0.9
    sel = np.arange(len(rows))
    keep_s = kp[rows]
    want = O.gather_combine(keep_s, slot_h, np64(w)[rows], np64(wl.values), np64(idx)[rows], np64(dist)[rows],
                            got_base, O.F32)
    absw = O.gather_combine(keep_s, np.abs(slot_h), np64(w)[rows], np.abs(np64(wl.values)), np64(idx)[rows],
                            np64(dist)[rows], np.abs(got_base), O.F32)
    assert_bf16_output(np64(out)[rows][sel], want, absw)
    # The reference rounds in another order: the shared MLP output and the
    # routed combine are each rounded, added and rounded
    # (deepseek_layers.py:743), and the decoder layer adds the residual:
    # ref = bf16(R + bf16(bf16(S) + bf16(Y))).  This layer computes
    # bf16(bf16(R + S) + Y).  With u = 2^-8 (bf16 unit roundoff) both are
    # within u-multiples of the exact R + S + Y, so they differ by at most
    # u * (|R + S| + |S| + |Y| + |S + Y| + 2 |R + S + Y|) (+ the fp32 sums).
    _, f_s = O.swiglu_expert(x, np64(s1), np64(s3), np64(s2), O.BF16)
    big_s = f_s @ np64(s2).T  # the shared experts' down projection, unrounded
    resid = np64(wl.residual)[rows]
    big_y = O.gather_combine(keep_s, slot_h, np64(w)[rows], np64(wl.values), np64(idx)[rows], np64(dist)[rows],
                             np.zeros_like(resid), O.F32)
    bf = lambda v: O.round_to(v, O.BF16)  # noqa: E731
    ref_order = bf(resid + bf(bf(big_s) + bf(big_y)))
    exact = resid + big_s + big_y
    u = 2.0 ** -8
    bound = u * (np.abs(resid + big_s) + np.abs(big_s) + np.abs(big_y) + np.abs(big_s + big_y) + 2 * np.abs(exact))
    got = np64(out)[rows]
    diff = np.abs(got - ref_order)
    assert np.all(diff <= bound * 1.001 + 1e-6), float(np.max(diff - bound))
    same = float(np.mean(got == ref_order))
    print(f"[config5] rounding order: {same:.4f} of subset elements equal the reference order's bits, "
          f"max |diff| {float(diff.max()):.3g} (bound {float(bound.max()):.3g})", flush=True)
    # the subset's search and projection against the oracle
    q_h = np64(q)[rows]
    ref_q = O.project_queries(x, isv[rows], (np64(wl.proj_vis), np64(wl.bias_vis)),
                              (np64(wl.proj_txt), np64(wl.bias_txt)), False, O.BF16)
    assert_projection_close(q_h, ref_q, proj_abssum(x, isv[rows], np64(wl.proj_vis), np64(wl.proj_txt)),
                            torch.bfloat16, min_exact=0.9)
    _, want_idx, exact = O.global_search(q_h, np64(wl.centroids), 1)
    check_topk_rows(exact, np64(idx)[rows], want_idx, False, "config 5 search")
    # end to end from x on every token: the oracle's search and keep set on its own queries
    isv_all = np64(wl.is_vision).astype(bool)
    ref_q_all = O.project_queries(np64(wl.x), isv_all, (np64(wl.proj_vis), np64(wl.bias_vis)),
                                  (np64(wl.proj_txt), np64(wl.bias_txt)), False, O.BF16)
    vals_o, _, _ = check_end_to_end_topk(np64(q), ref_q_all, np64(wl.centroids), np64(idx), "config 5 search")
    check_end_to_end_keep(np64(dist)[:, 0], vals_o[:, 0], kp, 2457, "config 5 keep")


def test_config5_layer_graph_replays(hip_device):
    """The config-5 layer call runs its shared experts on a second stream
    (forked from the caller's stream, joined before the combine).  With the
    shared experts as a SharedExperts (packed weights) the eager call equals
    the call with the plain weight tuple bit for bit; captured in a HIP graph
    and replayed three times, with the output cleared and other eager work on
    the caller's stream between replays, every replay equals the eager call
    bit for bit (slot outputs of the kept tokens, search outputs and combined
    rows)."""
    from synth import make_workload
    from table_moe.ops import GroupedExperts, SharedExperts

    dev = hip_device
    wl = make_workload(5, with_slot_out=False, device=dev, gen_device=dev)
    cfg = wl.cfg
    n, h, e, k, inter = cfg["n"], cfg["hidden"], cfg["n_experts"], cfg["router_top_k"], 1536
    g = torch.Generator(device=dev).manual_seed(56)
    rnd = lambda *shape: (torch.randn(*shape, generator=g, device=dev) * 0.02).to(torch.bfloat16)  # noqa: E731
    ex = GroupedExperts(rnd(e, inter, h), rnd(e, inter, h), rnd(e, h, inter))
    shared_plain = (rnd(2 * inter, h), rnd(2 * inter, h), rnd(h, 2 * inter))
    shared = SharedExperts(*shared_plain)
    tbl = _table(wl)
    out = torch.empty_like(wl.residual)
    want_plain = tbl.layer_forward_recompute(wl.x, wl.is_vision, wl.logits, ex, wl.residual, k, 0.6,
                                             shared=shared_plain, out=torch.empty_like(wl.residual))["out"].clone()

    def layer():
        return tbl.layer_forward_recompute(wl.x, wl.is_vision, wl.logits, ex, wl.residual, k, 0.6, shared=shared,
                                           out=out)

    res = layer()
    torch.cuda.synchronize()
    kb = res["keep"].bool()
    want = {key: res[key].clone() for key in ("ids", "idx", "dist", "keep", "out")}
    assert torch.equal(want["out"], want_plain)
    want_slot = res["slot_out"][kb].clone()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        layer()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        layer()
    torch.cuda.synchronize()
    for rep in range(3):
        out.zero_()
        res["slot_out"].zero_()
        scratch = (wl.x.float() * (rep + 1)).sum()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(scratch)
        for key, val in want.items():
            assert torch.equal(res[key], val), (rep, key)
        assert torch.equal(res["slot_out"][kb], want_slot), rep
