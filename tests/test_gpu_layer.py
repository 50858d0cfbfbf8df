"""GPU parity of the router, selection, gather/combine and online-window
kernels, the drop-in Python surface, and the full mode-G layer at the
config-2 (Qwen3-VL-30B-A3B prefill) shape."""

import numpy as np
import pytest
import torch

from oracle import tm_oracle as O
from parity_util import (ODT, assert_bf16_output, assert_projection_close, assert_within_ulps, check_end_to_end_keep,
                         check_end_to_end_topk, check_pick, check_topk_rows, np64, proj_abssum, ulp)
from table_moe import _native as N

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def test_single_hip_runtime_in_process(hip_device):
    """Our library and torch share one HIP runtime instance."""
    torch.zeros(1, device=hip_device)
    N.load()
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64" in line:
                paths.add(line.split()[-1])
    assert len(paths) == 1, paths


# ---------------------------------------------------------------- a1 router
@pytest.mark.parametrize("n,e,k,renorm", [(4096, 128, 8, False), (300, 64, 6, True), (77, 300, 5, False),
                                          (5, 2048, 32, False), (1, 8, 8, True), (1001, 256, 12, True),
                                          (13, 128, 1, False), (9, 100, 8, False)])
def test_topk_softmax_vs_oracle(hip_device, n, e, k, renorm):
    from table_moe.ops import qwen_topk_softmax

    g = _gen(61 + e)
    logits = torch.randn(n, e, generator=g) * 2
    logits[0, :4] = 20.0  # exact ties above every other logit: lower id first
    w, ids = qwen_topk_softmax(logits.to(hip_device), k, normalize_topk=renorm)
    torch.cuda.synchronize()
    ww, wids, p = O.topk_softmax(np64(logits), k, renorm)
    gi = np64(ids)
    check_topk_rows(p, gi, wids, larger_is_better=True, what="router")
    np.testing.assert_array_equal(gi[0, : min(4, k)], np.arange(min(4, k)))
    got_p = np.take_along_axis(p, gi, axis=1)
    if renorm:
        got_p = got_p / got_p.sum(1, keepdims=True)
    np.testing.assert_allclose(np64(w), got_p, rtol=2e-6, atol=1e-9)


# ------------------------------------------------------------ a3 keep masks
def test_fixed_keep_mask_reference_kat(hip_device):
    from table_moe.skip import build_decode_keep_mask, build_fixed_keep_mask

    sel = torch.tensor([[0, 1, 2, 3], [4, 5, 6, 7]], device=hip_device)
    want = torch.tensor([[True, True, False, False], [True, True, False, False]], device=hip_device)
    assert torch.equal(build_fixed_keep_mask(sel, 2), want)
    assert torch.equal(build_decode_keep_mask(sel, None), torch.ones_like(want))
    assert torch.equal(build_fixed_keep_mask(sel, 0), torch.zeros_like(want))


@pytest.mark.parametrize("n,k,e,use_attn,keep_rate", [(4096, 8, 128, True, 0.6), (4096, 8, 128, False, 0.6),
                                                      (513, 6, 64, True, 0.25), (7, 2, 1000, True, 0.9),
                                                      (1, 8, 128, False, 0.6)])
def test_expert_keep_mask_vs_oracle(hip_device, n, k, e, use_attn, keep_rate):
    from table_moe.skip import build_prefill_keep_mask

    g = _gen(71 + n)
    sel = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    w = torch.rand(n, k, generator=g)
    attn = torch.rand(n, generator=g) if use_attn else None
    dev = hip_device
    mask = build_prefill_keep_mask(sel.to(dev), w.to(dev), None if attn is None else attn.to(dev), e, keep_rate)
    torch.cuda.synchronize()
    want, sums = O.build_prefill_keep_mask(sel.numpy(), np64(w), None if attn is None else np64(attn), e, keep_rate)
    got = np64(mask)
    if not np.array_equal(got, want):
        # only experts whose exact scores tie the keep boundary within fp32 summation error may differ
        kept_got = set(sel.numpy()[got].tolist())
        kept_want = set(sel.numpy()[want].tolist())
        diff = kept_got ^ kept_want
        boundary = min(sums[list(kept_want)])
        for ex in diff:
            assert abs(sums[ex] - boundary) <= 1e-5 * abs(boundary), (ex, sums[ex], boundary)
        assert len(kept_got) == len(kept_want)


@pytest.mark.parametrize("dtype,target", [(torch.float32, None), (torch.float32, "orig"), (torch.bfloat16, None),
                                          (torch.float16, "orig")])
def test_renormalize_vs_oracle(hip_device, dtype, target):
    from table_moe.skip import renormalize_surviving_weights

    g = _gen(81)
    n, k = 1000, 8
    w = torch.rand(n, k, generator=g).to(dtype)
    m = torch.rand(n, k, generator=g) < 0.5
    m[:3] = False  # zero-survivor rows
    dev = hip_device
    tgt = w.float().sum(-1, keepdim=True).to(dtype) if target else None
    out = renormalize_surviving_weights(w.to(dev), m.to(dev), None if tgt is None else tgt.to(dev))
    torch.cuda.synchronize()
    want = O.renormalize_surviving_weights(np64(w), m.numpy(), None if tgt is None else np64(tgt), dt=ODT[dtype])
    got = np64(out)
    assert (got[:3] == 0).all()
    if dtype == torch.float32:
        np.testing.assert_allclose(got, want, rtol=5e-7, atol=0)
    else:
        assert_within_ulps(got, want, dtype, n_ulp=1, min_exact=0.95)


def test_renormalize_reference_kat(hip_device):
    from table_moe.skip import renormalize_surviving_weights

    dev = hip_device
    out = renormalize_surviving_weights(torch.tensor([[0.4, 0.3, 0.2, 0.1]], device=dev),
                                        torch.tensor([[True, True, False, False]], device=dev))
    torch.testing.assert_close(out.cpu(), torch.tensor([[4 / 7, 3 / 7, 0.0, 0.0]]), atol=1e-6, rtol=0)


# ----------------------------------------------------------- a10 gather rows
@pytest.mark.parametrize("dtype,hidden", [(torch.bfloat16, 2048), (torch.float16, 1004), (torch.float32, 64)])
def test_gather_rows_bit_exact(hip_device, dtype, hidden):
    from table_moe.cache_engine import CacheConfig, HybridStorageManager

    g = _gen(91)
    dev = hip_device
    old = CacheConfig.MODEL_DTYPE
    CacheConfig.MODEL_DTYPE = dtype
    try:
        mgr = HybridStorageManager(0, 8, hidden, dev)
    finally:
        CacheConfig.MODEL_DTYPE = old
    mgr.values_buffer.copy_(torch.randn(mgr.values_buffer.shape, generator=g).to(dtype))
    n = 300
    e = torch.randint(0, 8, (n,), generator=g)
    m = torch.randint(0, 2, (n,), generator=g)
    c = torch.randint(0, mgr.values_buffer.shape[2], (n,), generator=g)
    got = mgr.gather_values(e, m, c)  # host indices, as the reference caller passes them
    torch.cuda.synchronize()
    assert got.device.type == "cuda"
    assert torch.equal(got.cpu(), mgr.values_buffer.cpu()[e, m, c])
    out = torch.zeros(8, hidden, dtype=dtype, device=dev)
    slots = torch.tensor([1, 5, 6])
    mgr.gather_values_decode_bs1(e[:3].to(dev), 1, c[:3].to(dev), slots.to(dev), out)
    torch.cuda.synchronize()
    ref = torch.zeros(8, hidden, dtype=dtype)
    ref[slots] = mgr.values_buffer.cpu()[e[:3], 1, c[:3]]
    assert torch.equal(out.cpu(), ref)


# ----------------------------------------------------------- a12 online window
def test_online_update_vs_oracle(hip_device):
    from table_moe.cache_engine import CacheConfig, HybridStorageManager

    g = _gen(101)
    dev = hip_device
    H, k = 256, 8
    saved = (CacheConfig.ONLINE_CACHE_SIZE, CacheConfig.ONLINE_TOP_K, CacheConfig.MODEL_DTYPE)
    CacheConfig.ONLINE_CACHE_SIZE, CacheConfig.ONLINE_TOP_K, CacheConfig.MODEL_DTYPE = 16, k, torch.bfloat16
    try:
        mgr = HybridStorageManager(3, 8, H, dev)
    finally:
        CacheConfig.ONLINE_CACHE_SIZE, CacheConfig.ONLINE_TOP_K, CacheConfig.MODEL_DTYPE = saved
    st = dict(keys=np.zeros((16, H)), ids=np.full((16, k), -1), values=np.zeros((16, k, H)), ptr=0, full=False,
              size=16)
    for step, n in enumerate([5, 9, 1, 20, 3, 16, 2]):
        hid = torch.randn(n, H, generator=g).to(torch.bfloat16)
        ids = torch.randint(0, 8, (n, k), generator=g)
        outs = torch.randn(n, k, H, generator=g).to(torch.bfloat16)
        valid = torch.rand(n, k, generator=g) < 0.7
        if n == 1:
            mgr.update_online_cache_bs1(hid[0].to(dev), ids[0].to(dev), outs[0].to(dev), valid[0].to(dev))
        else:
            mgr.update_online_cache(hid.to(dev), ids.to(dev), outs.to(dev), valid.to(dev))
        st = O.online_update(st, np64(hid), ids.numpy(), np64(outs), valid.numpy())
        torch.cuda.synchronize()
        assert mgr.online_ptr == st["ptr"] and mgr.online_full == st["full"]
        np.testing.assert_array_equal(np64(mgr.online_keys), st["keys"])
        np.testing.assert_array_equal(np64(mgr.online_expert_ids), st["ids"])
        np.testing.assert_array_equal(np64(mgr.online_values), st["values"])


# ------------------------------------------------------- a10+a11 slot combine
@pytest.mark.parametrize("target", ["one", "orig_sum"])
@pytest.mark.parametrize("with_residual", [False, True])
def test_slot_combine_vs_oracle(hip_device, target, with_residual):
    g = _gen(111)
    dev = hip_device
    n, k, H, E, K, W, wk = 200, 8, 1024, 16, 64, 8, 8
    dt = torch.bfloat16
    w = torch.rand(n, k, generator=g)
    compute = torch.zeros(n, k, dtype=torch.bool)
    compute[:, :3] = True
    off_hit = (torch.rand(n, k, generator=g) < 0.4) & ~compute
    on_hit = (torch.rand(n, k, generator=g) < 0.3) & ~compute & ~off_hit
    on_hit[:5] = False
    off_hit[:5] = False
    compute[:2] = False  # rows with no survivor
    sel = torch.randint(0, E, (n, k), generator=g)
    off_idx = torch.randint(0, K, (n, k), generator=g)
    on_idx = torch.randint(0, W, (n,), generator=g)
    on_slot = torch.randint(0, wk, (n, k), generator=g)
    vis = torch.rand(n, generator=g) < 0.5
    computed = torch.randn(n, k, H, generator=g).to(dt)
    values = torch.randn(E, 2, K, H, generator=g).to(dt)
    online = torch.randn(W, wk, H, generator=g).to(dt)
    resid = torch.randn(n, H, generator=g).to(dt) if with_residual else None
    # device copies stay bound to names until the kernel has run
    wd, cmd, ohd, oid, seld, visd, onhd, onid, onsd = (t.to(dev) for t in (w, compute, off_hit, off_idx, sel, vis,
                                                                            on_hit, on_idx, on_slot))
    vd, od, cd = values.to(dev), online.to(dev), computed.to(dev)
    rd = None if resid is None else resid.to(dev)
    out = torch.empty(n, H, dtype=dt, device=dev)
    N.call("tm_slot_combine", N.TM_DT_BF16, n, k, H, wd.data_ptr(), k, N.as_u8(cmd).data_ptr(),
           cd.data_ptr(), cd.stride(0), cd.stride(1), N.as_u8(ohd).data_ptr(), oid.data_ptr(),
           seld.data_ptr(), k, N.as_u8(visd).data_ptr(), vd.data_ptr(), E, K, vd.stride(0), vd.stride(1),
           vd.stride(2), N.as_u8(onhd).data_ptr(), onid.data_ptr(), onsd.data_ptr(), od.data_ptr(), W,
           wk, od.stride(0), od.stride(1), N.TM_TARGET_ONE if target == "one" else N.TM_TARGET_ORIG_SUM,
           None if rd is None else rd.data_ptr(), H, out.data_ptr(), H, N.stream(dev))
    torch.cuda.synchronize()
    # the collected buffer of the reference (cached_layers.py:439-461), built on the host
    coll = np.zeros((n, k, H))
    m = np.where(vis.numpy(), 0, 1)
    cn, vn, onn = np64(computed), np64(values), np64(online)
    for b in range(n):
        for s in range(k):
            if compute[b, s]:
                coll[b, s] = cn[b, s]
            if on_hit[b, s]:
                coll[b, s] = onn[on_idx[b], on_slot[b, s]]
            if off_hit[b, s]:
                coll[b, s] = vn[sel[b, s], m[b], off_idx[b, s]]
    surv = (compute | on_hit | off_hit).numpy()
    r = None if resid is None else np64(resid)
    exact, _ = O.slot_combine(coll, np64(w), surv, O.BF16, target_mode=target, residual=r, out_dt=O.F32)
    abssum, _ = O.slot_combine(np.abs(coll), np64(w), surv, O.BF16, target_mode=target,
                               residual=None if r is None else np.abs(r), out_dt=O.F32)
    got = np64(out)
    assert_bf16_output(got, exact, abssum)
    assert (got[:2] == (0 if resid is None else np64(resid)[:2])).all()


# ---------------------------------------------- mode R engine (drop-in API)
def _mode_r_manager(dev, E=16, H=512, d=64, K=256, seed=121, dtype=torch.bfloat16):
    from table_moe.cache_engine import CacheConfig, HybridStorageManager

    g = _gen(seed)
    saved = {k: getattr(CacheConfig, k) for k in ("FIXED_K", "COMPRESSED_DIM", "MODEL_DTYPE", "ONLINE_CACHE_SIZE",
                                                  "ONLINE_TOP_K")}
    CacheConfig.FIXED_K, CacheConfig.COMPRESSED_DIM, CacheConfig.MODEL_DTYPE = K, d, dtype
    CacheConfig.ONLINE_CACHE_SIZE, CacheConfig.ONLINE_TOP_K = 64, 8
    try:
        mgr = HybridStorageManager(2, E, H, dev)
    finally:
        for k_, v in saved.items():
            setattr(CacheConfig, k_, v)
    for mod in ("vision", "text"):
        p = torch.linalg.qr(torch.randn(H, d, generator=g, dtype=torch.float64))[0].to(dtype)
        mgr.pca[mod] = {"proj": p.to(dev), "bias": (torch.randn(d, generator=g) * 0.05).to(dtype).to(dev)}
    for e in range(E):
        for m in range(2):
            mgr.load_table_entry(e, m, torch.randn(K, d, generator=g), torch.randn(K, H, generator=g))
    return mgr, g


def test_engine_prefill_offline_end_to_end(hip_device):
    from table_moe.cache_engine import CacheConfig, VectorSearchEngine

    dev = hip_device
    mgr, g = _mode_r_manager(dev)
    eng = VectorSearchEngine(mgr)
    n, k = 700, 8
    x = torch.randn(n, 512, generator=g).to(torch.bfloat16)
    pvn = mgr.pca["vision"]["proj"].cpu()
    c = mgr.keys_buffer.cpu()[torch.randint(0, 16, (n,), generator=g), 0, torch.randint(0, 256, (n,), generator=g)]
    x[: n // 2] = (x[: n // 2].float() * 0.3 + (c[: n // 2].float() @ pvn.float().T) * 3).to(torch.bfloat16)
    sel = torch.stack([torch.randperm(16, generator=g)[:k] for _ in range(n)])
    vis = torch.rand(n, generator=g) < 0.7
    reuse = torch.rand(n, k, generator=g) < 0.5
    hit, idx = eng.search_prefill_offline(0, x.to(dev), sel.to(dev), vis.to(dev), reuse.to(dev))
    torch.cuda.synchronize()
    assert hit.dtype == torch.bool and idx.dtype == torch.long and hit.shape == (n, k)
    # stage 1: the engine's projected + normalised queries
    q = np64(eng.prefill_query_workspace[:n])
    pca = mgr.pca
    ref_q = O.project_queries(np64(x), vis.numpy(), (np64(pca["vision"]["proj"]), np64(pca["vision"]["bias"])),
                              (np64(pca["text"]["proj"]), np64(pca["text"]["bias"])), True, O.BF16)
    assert_within_ulps(q, ref_q, torch.bfloat16, n_ulp=1, min_exact=0.9)
    # stage 2: cosine search on those queries
    thr_v, thr_t = CacheConfig.OFFLINE_COSINE_THRESHOLD_VISION, CacheConfig.OFFLINE_COSINE_THRESHOLD_TEXT
    wh, wi, mx, scores = O.search_gated(q, np64(mgr.keys_buffer), sel.numpy(), vis.numpy(), reuse.numpy(), thr_v,
                                        thr_t, O.CMP_GE)
    gh, gi = np64(hit), np64(idx)
    assert 0 < gh.sum() < reuse.sum()
    for b, s in zip(*np.nonzero(reuse.numpy())):
        thr = float(np.float32(thr_v if vis[b] else thr_t))
        assert O.threshold_ok(mx[b, s], thr, gh[b, s], wh[b, s])
        if gh[b, s]:
            check_pick(scores[b, s], gi[b, s], int(np.argmax(scores[b, s])), True)
    assert not gh[~reuse.numpy()].any()


def test_engine_decode_hybrid_with_window(hip_device):
    from table_moe.cache_engine import VectorSearchEngine

    dev = hip_device
    mgr, g = _mode_r_manager(dev, seed=131)
    eng = VectorSearchEngine(mgr)
    H, k = 512, 8
    hist = torch.randn(40, H, generator=g).to(torch.bfloat16)
    hist_ids = torch.stack([torch.randperm(16, generator=g)[:k] for _ in range(40)])
    mgr.update_online_cache(hist.to(dev), hist_ids.to(dev), torch.randn(40, k, H, generator=g).to(torch.bfloat16).to(dev))
    n = 6
    x = (hist[torch.tensor([3, 9, 30, 31, 0, 5])].float() + 0.3 * torch.randn(n, H, generator=g)).to(torch.bfloat16)
    sel = hist_ids[torch.tensor([3, 9, 30, 31, 0, 5])].clone()
    sel[:, ::2] = torch.randint(0, 16, (n, 4), generator=g)
    vis = torch.zeros(n, dtype=torch.bool)
    on_hit, on_idx, off_hit, off_idx, on_slot = eng.search_decode_hybrid(0, x.to(dev), sel.to(dev), vis.to(dev), 4)
    torch.cuda.synchronize()
    assert on_hit.data_ptr() == eng.workspace["on_hit"].data_ptr()  # workspace views, as the reference
    ref = O.search_hybrid(np64(x), vis.numpy(), (np64(mgr.pca["vision"]["proj"]), np64(mgr.pca["vision"]["bias"])),
                          (np64(mgr.pca["text"]["proj"]), np64(mgr.pca["text"]["bias"])), O.BF16,
                          np64(mgr.keys_buffer), sel.numpy(), 4, np64(mgr.online_keys), np64(mgr.online_expert_ids),
                          40)
    np.testing.assert_array_equal(np64(on_idx), ref["on_idx"])
    np.testing.assert_array_equal(np64(on_hit), ref["on_hit"])
    np.testing.assert_array_equal(np64(on_slot), ref["on_slot"])
    assert np64(on_hit).any()
    # bs1 entry writes the caller's buffers
    bufs = [torch.empty(k, dtype=torch.bool, device=dev), torch.empty(1, dtype=torch.long, device=dev),
            torch.empty(k, dtype=torch.bool, device=dev), torch.empty(k, dtype=torch.long, device=dev),
            torch.empty(k, dtype=torch.long, device=dev)]
    eng.search_decode_hybrid_bs1_into(x[1].to(dev), sel[1].to(dev), vis[1].to(dev), 4, *bufs)
    torch.cuda.synchronize()
    assert int(bufs[1].item()) == int(on_idx[1].item())
    assert torch.equal(bufs[0], on_hit[1]) and torch.equal(bufs[4], on_slot[1])
    assert torch.equal(bufs[2], off_hit[1]) and torch.equal(bufs[3], off_idx[1])
    # every token through the bs1 entry, outputs as strided columns (element
    # stride 2, the other column untouched), a non-unit-stride expert row and
    # 0-d vision flags: the same values as the batch call
    for t in range(n):
        cols = [torch.zeros(k, 2, dtype=torch.bool, device=dev), torch.full((1,), -7, dtype=torch.long, device=dev),
                torch.zeros(k, 2, dtype=torch.bool, device=dev), torch.full((k, 2), -7, dtype=torch.long, device=dev),
                torch.full((k, 2), -7, dtype=torch.long, device=dev)]
        outs = [c[:, 1] if c.dim() == 2 else c for c in cols]
        sel_row = torch.stack([sel[t], sel[t]], 1).to(dev)[:, 0]
        eng.search_decode_hybrid_bs1_into(x[t].to(dev), sel_row, vis[t].to(dev), 4, *outs)
        torch.cuda.synchronize()
        assert int(outs[1].item()) == int(on_idx[t].item()), t
        assert torch.equal(outs[0], on_hit[t]) and torch.equal(outs[4], on_slot[t]), t
        assert torch.equal(outs[2], off_hit[t]) and torch.equal(outs[3], off_idx[t]), t
        assert not cols[0][:, 0].any() and not cols[2][:, 0].any(), t
        assert bool((cols[3][:, 0] == -7).all()) and bool((cols[4][:, 0] == -7).all()), t


def test_engine_rejects_host_tensors():
    """No CPU fallback: host tensors raise instead of silently running elsewhere."""
    from table_moe.skip import renormalize_surviving_weights

    with pytest.raises(RuntimeError, match="HIP device"):
        renormalize_surviving_weights(torch.rand(2, 4), torch.ones(2, 4, dtype=torch.bool))


# ------------------------------------------------ mode G: gather + combine
@pytest.mark.parametrize("k,nn,hidden,with_residual", [(8, 1, 2048, True), (8, 4, 2048, True), (8, 4, 1004, False),
                                                        (6, 1, 2560, True), (6, 4, 2560, False), (5, 2, 2048, True),
                                                        (8, 1, 4096, False), (8, 1, 8, True), (6, 4, 520, True),
                                                        (8, 1, 8192, True), (6, 4, 8200, False)])
def test_gather_combine_vs_oracle(hip_device, k, nn, hidden, with_residual):
    """Shape-specialised kernels (top-8/top-6 x 1/4 nearest, 16-byte rows):
    one 8-element chunk per thread up to hidden 8192 (a single chunk, a
    partial last wave, 1024 threads), the chunk loop beyond it; and the
    general kernels (other shapes, unaligned rows)."""
    from table_moe.cache_engine import GlobalTable

    g = _gen(141 + k + nn + hidden)
    dev = hip_device
    n, C, d = 257, 500, 64
    dt = torch.bfloat16
    values = torch.randn(C, hidden, generator=g).to(dt)
    slot_out = torch.randn(n, k, hidden, generator=g).to(dt)
    w = torch.rand(n, k, generator=g) + 0.01
    idx = torch.randint(0, C, (n, nn), generator=g)
    dist = torch.rand(n, nn, generator=g) * 10
    dist[:, 0] = 0.0  # exact hit of a centroid
    keep = torch.rand(n, generator=g) < 0.6
    resid = torch.randn(n, hidden, generator=g).to(dt) if with_residual else None
    tbl = GlobalTable(torch.zeros(C, d, dtype=dt, device=dev), values.to(dev),
                      (torch.zeros(hidden, d, dtype=dt, device=dev), torch.zeros(d, dtype=dt, device=dev)))
    out = tbl.gather_combine(keep.to(dev), slot_out.to(dev), w.to(dev), idx.to(dev), dist.to(dev),
                             None if resid is None else resid.to(dev))
    torch.cuda.synchronize()
    r = np.zeros((n, hidden)) if resid is None else np64(resid)
    exact = O.gather_combine(keep.numpy(), np64(slot_out), np64(w), np64(values), idx.numpy(), np64(dist), r, O.F32)
    abssum = O.gather_combine(keep.numpy(), np.abs(np64(slot_out)), np64(w), np.abs(np64(values)), idx.numpy(),
                              np64(dist), np.abs(r), O.F32)
    assert_bf16_output(np64(out), exact, abssum)


@pytest.mark.parametrize("n,k,hidden,with_residual,ties,dt", [
    (4096, 8, 2048, True, False, torch.bfloat16), (4096, 8, 2048, True, True, torch.bfloat16),
    (1001, 6, 1000, False, True, torch.float16), (5, 8, 64, True, False, torch.bfloat16),
    (515, 8, 2048, True, False, torch.bfloat16), (1, 8, 2048, True, False, torch.bfloat16),
    (6000, 6, 2048, False, True, torch.bfloat16)])
def test_gather_combine_ranked_matches_keep_select(hip_device, n, k, hidden, with_residual, ties, dt):
    """tm_gather_combine_ranked (keep set ranked inside the combine) gives the
    keep mask of tm_keep_select and the output of tm_gather_combine with that
    mask, bit for bit: ragged token counts (not a multiple of 4), tied
    distances across the keep boundary, no residual, fp16, hidden < 2048,
    every n_keep from 1 to n at the boundaries; the output is also checked
    against the oracle."""
    from table_moe.cache_engine import GlobalTable

    g = _gen(907 + n + k + hidden)
    dev = hip_device
    C, d = 300, 64
    values = torch.randn(C, hidden, generator=g).to(dt)
    slot_out = torch.randn(n, k, hidden, generator=g).to(dt)
    w = torch.rand(n, k, generator=g) + 0.01
    w[0] = 0.0  # weights summing to 0: no slot contribution
    idx = torch.randint(0, C, (n, 1), generator=g)
    if n > 1:
        idx[1, 0] = -1  # no centroid: residual only when not kept
    dist = torch.rand(n, 1, generator=g) * 10
    if ties:  # a few distinct values only: many ties at every boundary
        dist = torch.floor(dist * 2) / 2
    resid = torch.randn(n, hidden, generator=g).to(dt) if with_residual else None
    tbl = GlobalTable(torch.zeros(C, d, dtype=dt, device=dev), values.to(dev),
                      (torch.zeros(hidden, d, dtype=dt, device=dev), torch.zeros(d, dtype=dt, device=dev)))
    dd, so, wd, idd = dist.to(dev), slot_out.to(dev), w.to(dev), idx.to(dev)
    rd = None if resid is None else resid.to(dev)
    for n_keep in sorted({1, max(1, int(n * 0.6)), n - 1 if n > 1 else 1, n}):
        out, keep = tbl.gather_combine_ranked(so, wd, idd, dd, n_keep, rd, out=torch.empty(n, hidden, dtype=dt,
                                                                                           device=dev),
                                              keep=torch.zeros(n, dtype=torch.bool, device=dev))
        want_keep = tbl.keep_select(dd[:, 0], n_keep).clone()
        want = tbl.gather_combine(want_keep, so, wd, idd, dd, rd, out=torch.empty(n, hidden, dtype=dt, device=dev))
        torch.cuda.synchronize()
        assert torch.equal(keep, want_keep), n_keep
        assert int(keep.sum()) == n_keep
        assert torch.equal(out, want), n_keep
    kn = keep.cpu().numpy()
    np.testing.assert_array_equal(kn, O.keep_select(np64(dist)[:, 0], n_keep))
    if n <= 2:
        return
    # the oracle's combine on the rows without the zero-weight / no-centroid cases
    r = np.zeros((n, hidden)) if resid is None else np64(resid)
    sl = slice(2, None)
    exact = O.gather_combine(kn[sl], np64(slot_out)[sl], np64(w)[sl], np64(values), idx.numpy()[sl], np64(dist)[sl],
                             r[sl], O.F32)
    abssum = O.gather_combine(kn[sl], np.abs(np64(slot_out))[sl], np64(w)[sl], np.abs(np64(values)),
                              idx.numpy()[sl], np64(dist)[sl], np.abs(r)[sl], O.F32)
    assert_bf16_output(np64(out)[sl], exact, abssum)


# ------------------------------------------ mode G: full layer at config 2
def test_layer_forward_config2_end_to_end(hip_device):
    from table_moe.cache_engine import GlobalTable
    from synth import make_workload

    wl = make_workload(2)
    dev = hip_device
    d = wl.to(dev)
    tbl = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt))
    res = tbl.layer_forward(d.x, d.is_vision, d.logits, d.slot_out, d.residual, router_top_k=8, n_nearest=1,
                            keep_rate=0.6)
    torch.cuda.synchronize()
    # router
    ww, wids, p = O.topk_softmax(np64(wl.logits), 8)
    check_topk_rows(p, np64(res["ids"]), wids, True, "router")
    # projection
    q = np64(res["q"])
    ref_q = O.project_queries(np64(wl.x), wl.is_vision.numpy(), (np64(wl.proj_vis), np64(wl.bias_vis)),
                              (np64(wl.proj_txt), np64(wl.bias_txt)), False, O.BF16)
    abssum = proj_abssum(np64(wl.x), wl.is_vision.numpy(), np64(wl.proj_vis), np64(wl.proj_txt))
    assert_projection_close(q, ref_q, abssum, torch.bfloat16, min_exact=0.97)
    # search on the device's queries
    vals, want_idx, exact = O.global_search(q, np64(wl.centroids), 1)
    gi = np64(res["idx"])
    n_mis = check_topk_rows(exact, gi, want_idx, False, "search")
    assert n_mis <= 3
    near = wl.cluster_of.numpy() >= 0
    assert np.mean(gi[near, 0] == wl.cluster_of.numpy()[near]) > 0.99
    # keep selection: bit-exact on the device's distances
    gd = np64(res["dist"])
    keep = np64(res["keep"])
    assert keep.sum() == O.keep_count(4096, 0.6) == 2457
    np.testing.assert_array_equal(keep, O.keep_select(gd[:, 0].astype(np.float32).astype(np.float64), 2457))
    # end to end from x: the oracle's search and keep set on its own queries
    vals_o, _, _ = check_end_to_end_topk(q, ref_q, np64(wl.centroids), gi, "config 2 search")
    check_end_to_end_keep(gd[:, 0], vals_o[:, 0], keep, 2457, "config 2 keep")
    # combine on the device's selections
    exact = O.gather_combine(keep, np64(wl.slot_out), np64(res["weights"]), np64(wl.values), gi, gd,
                             np64(wl.residual), O.F32)
    abssum = O.gather_combine(keep, np.abs(np64(wl.slot_out)), np64(res["weights"]), np.abs(np64(wl.values)), gi,
                              gd, np.abs(np64(wl.residual)), O.F32)
    assert_bf16_output(np64(res["out"]), exact, abssum)


def check_decode_plan_stagewise(b, ra, d, is_vision, residual, wl, nn, keep_rate=0.6):
    """A decode-plan layer call (n <= 64) against the stage calls run on the
    layer's own queries: the projection reduces across workgroups in its own
    fp32 order, so q may differ from tm_project's in the last bit; given the
    same q and |q|^2, search, keep and combine must agree bit for bit.  q is
    checked against the oracle and |q|^2 against the exact sum of squares."""
    n = d.x.shape[0]
    topk = d.cfg["router_top_k"]
    w, ids = b.route(d.logits, topk)
    assert torch.equal(ra["weights"], w) and torch.equal(ra["ids"], ids)
    dist, idx = b.search(ra["q"], nn, ra["qn"])
    assert torch.equal(ra["dist"], dist) and torch.equal(ra["idx"], idx)
    keep = b.keep_select(dist[:, 0], b.keep_count(n, keep_rate))
    assert torch.equal(ra["keep"], keep)
    out = b.gather_combine(keep, d.slot_out, w, idx, dist, residual)
    torch.cuda.synchronize()
    assert torch.equal(ra["out"], out)
    dt = d.x.dtype
    q = np64(ra["q"])
    isv = is_vision.cpu().numpy()
    ref_q = O.project_queries(np64(wl.x), isv, (np64(wl.proj_vis), np64(wl.bias_vis)),
                              (np64(wl.proj_txt), np64(wl.bias_txt)), False, ODT[dt])
    abssum = proj_abssum(np64(wl.x), isv, np64(wl.proj_vis), np64(wl.proj_txt))
    assert_projection_close(q, ref_q, abssum, dt, min_exact=0.95)
    qn_exact = (q * q).sum(axis=1)
    np.testing.assert_allclose(np64(ra["qn"]), qn_exact, rtol=2e-6, atol=1e-6)


def test_layer_forward_one_call_matches_staged(hip_device):
    """tm_table_forward (one call, router fused into the projection launch for
    64/128 experts) and the five stage calls give identical bits; config 5
    shapes (64 experts, top-6, hidden 2560) at a token count that leaves a
    partial routing workgroup."""
    from table_moe.cache_engine import GlobalTable
    from synth import make_workload

    dev = hip_device
    for cfg, n, nn in ((2, 1000, 1), (3, 32, 4), (5, 77, 1)):
        wl = make_workload(cfg, n=n)
        d = wl.to(dev)
        a = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt))
        b = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt))
        topk = d.cfg["router_top_k"]
        ra = a.layer_forward(d.x, d.is_vision, d.logits, d.slot_out, d.residual, topk, nn, 0.6)
        if n <= 64:  # decode plan
            check_decode_plan_stagewise(b, ra, d, d.is_vision, d.residual, wl, nn)
            continue
        rb = b.layer_forward_staged(d.x, d.is_vision, d.logits, d.slot_out, d.residual, topk, nn, 0.6)
        torch.cuda.synchronize()
        for key in ("weights", "ids", "q", "qn", "dist", "idx", "keep", "out"):
            assert torch.equal(ra[key], rb[key]), key


@pytest.mark.parametrize("n,hidden,dim,mix,n_cent,dup", [
    (300, 1000, 128, False, 1024, False), (515, 2080, 64, True, 1024, False), (96, 264, 128, True, 1024, False),
    (4096, 2048, 128, True, 1024, False),
    # hidden 2048 / 2560 (pipelined projection: 4 / 5 chunks per wave) with a
    # ragged row tile and mixed tiles; other multiples of 32 (register kernel)
    (300, 2560, 128, True, 1024, False), (777, 2048, 128, True, 2048, False),
    (200, 480, 128, True, 1024, False), (777, 1056, 128, True, 2048, False),
    # ranked form (wide search decoding the keys, keep set ranked in the
    # combine): config-2 shape, repeated tokens (tied distances at the keep
    # boundary), d = 64, a ragged last query tile and centroid range
    (4096, 2048, 128, True, 8192, False), (4096, 2048, 128, False, 8192, True), (4096, 1000, 64, False, 16384, False),
    (4000, 2080, 128, True, 12000, False),
    # either side of the projection's switch to 32-column groups (n <= 2048):
    # 32-column groups at hidden 2560 with tied tokens (one modality, so a
    # repeated token's distance equals its original's), 64-column groups from
    # n = 2049 (a ragged last row tile, mixed tiles)
    (2048, 2560, 128, False, 4096, True), (2049, 2048, 128, True, 4096, False),
    # above the ranked form's token limit: keep select launch
    (8192, 1024, 128, False, 8192, False)])
def test_layer_forward_fused_shapes_match_staged(hip_device, n, hidden, dim, mix, n_cent, dup):
    """Top-1 layer calls take the fused plan (column-split projection, search
    merged by atomic minimum, keep select decoding the packed keys; for up to
    4096 tokens the search decodes the keys and the combine ranks the keep
    set); the result must equal the stage calls bit for bit.  Hidden sizes
    that end inside a k-step or a 4-k-step chunk, d = 64, ragged row tiles and
    centroid ranges, modality patterns that mix vision and text rows inside
    every tile, and repeated tokens.  Each table is called twice: the second
    call checks that the arrival counters were left at zero."""
    from table_moe.cache_engine import GlobalTable
    from synth import make_workload

    dev = hip_device
    wl = make_workload(2, n=n, hidden=hidden, dim=dim, n_cent=n_cent)
    d = wl.to(dev)
    if dup:  # every token of the second quarter repeats one of the first: equal distances
        src = torch.arange(n // 4, device=dev) % (n // 8)
        d.x[n // 4:n // 2] = d.x[src]
    is_vision = d.is_vision
    if mix:
        g = torch.Generator().manual_seed(n)
        is_vision = (torch.rand(n, generator=g) < 0.5).to(dev)
    a = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt))
    b = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt))
    rb = b.layer_forward_staged(d.x, is_vision, d.logits, d.slot_out, d.residual, 8, 1, 0.6)
    for rep in range(2):
        ra = a.layer_forward(d.x, is_vision, d.logits, d.slot_out, d.residual, 8, 1, 0.6)
        torch.cuda.synchronize()
        for key in ("weights", "ids", "q", "qn", "dist", "idx", "keep", "out"):
            assert torch.equal(ra[key], rb[key]), (key, rep)
    # and the projection against the oracle
    q = np64(ra["q"])
    x = np64(d.x)
    ref_q = O.project_queries(x, is_vision.cpu().numpy(), (np64(wl.proj_vis), np64(wl.bias_vis)),
                              (np64(wl.proj_txt), np64(wl.bias_txt)), False, O.BF16)
    abssum = proj_abssum(x, is_vision.cpu().numpy(), np64(wl.proj_vis), np64(wl.proj_txt))
    assert_projection_close(q, ref_q, abssum, torch.bfloat16, min_exact=0.95)
    if dup:  # the repeated tokens tie with their originals, and some ties sit at the keep boundary
        dist = ra["dist"][:, 0]
        src = torch.arange(n // 4, device=dev) % (n // 8)
        assert torch.equal(dist[n // 4:n // 2], dist[src])
        keep = ra["keep"].bool()
        kept_d = dist[keep]
        assert (dist[~keep] <= kept_d.min()).all()


@pytest.mark.parametrize("dtype,n", [(torch.bfloat16, 1000), (torch.float16, 4096), (torch.bfloat16, 4096)])
def test_layer_forward_general_ranked_matches_staged(hip_device, dtype, n):
    """A projection bias that does not start on a 16-byte boundary keeps the
    table's P in the strided layout (no packed copy), so a top-1 layer takes
    the general plan (tm_project, the split search and its merge); for up to
    4096 tokens the combine ranks the keep set itself (no keep-select
    launch).  The result must equal the stage calls bit for bit, on two calls
    in a row."""
    from table_moe.cache_engine import GlobalTable
    from synth import make_workload

    dev = hip_device
    wl = make_workload(2, n=n, dim=64, n_cent=2048, dtype=dtype)
    d = wl.to(dev)
    g = torch.Generator().manual_seed(n)
    is_vision = (torch.rand(n, generator=g) < 0.5).to(dev)

    def unaligned(b):  # the same values, 2 bytes past a 16-byte boundary
        t = torch.empty(b.numel() + 1, dtype=b.dtype, device=dev)[1:]
        t.copy_(b)
        assert t.data_ptr() % 16 != 0
        return t

    bv, bt = unaligned(d.bias_vis), unaligned(d.bias_txt)
    a = GlobalTable(d.centroids, d.values, (d.proj_vis, bv), (d.proj_txt, bt))
    b = GlobalTable(d.centroids, d.values, (d.proj_vis, bv), (d.proj_txt, bt))
    assert a.ps != (0, 0), "the table kept a packed projection: the fused plan would run"
    rb = b.layer_forward_staged(d.x, is_vision, d.logits, d.slot_out, d.residual, 8, 1, 0.6)
    for rep in range(2):
        ra = a.layer_forward(d.x, is_vision, d.logits, d.slot_out, d.residual, 8, 1, 0.6)
        torch.cuda.synchronize()
        for key in ("weights", "ids", "q", "qn", "dist", "idx", "keep", "out"):
            assert torch.equal(ra[key], rb[key]), (key, rep)
    assert int(ra["keep"].sum()) == O.keep_count(n, 0.6)


@pytest.mark.parametrize("dtype,metric", [(torch.float16, "l2"), (torch.bfloat16, "dot"), (torch.float16, "dot")])
def test_layer_forward_ranked_plan_dtypes_metrics(hip_device, dtype, metric):
    """The ranked top-1 plan (wide search decoding its keys, keep set ranked
    in the combine) with fp16 data and the dot metric equals the stage calls
    bit for bit, on two calls in a row."""
    from table_moe.cache_engine import GlobalTable
    from synth import make_workload

    dev = hip_device
    wl = make_workload(2, dtype=dtype)
    d = wl.to(dev)
    a = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt), metric=metric)
    b = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt), metric=metric)
    rb = b.layer_forward_staged(d.x, d.is_vision, d.logits, d.slot_out, d.residual, 8, 1, 0.6)
    for rep in range(2):
        ra = a.layer_forward(d.x, d.is_vision, d.logits, d.slot_out, d.residual, 8, 1, 0.6)
        torch.cuda.synchronize()
        for key in ("weights", "ids", "q", "qn", "dist", "idx", "keep", "out"):
            assert torch.equal(ra[key], rb[key]), (key, rep)
    assert int(ra["keep"].sum()) == 2457


@pytest.mark.parametrize("cfg,n,hidden,dim,n_cent,nn,variant", [
    (3, 1, 2048, 128, 16384, 4, "base"), (3, 8, 2048, 128, 16384, 4, "base"), (3, 32, 2048, 128, 16384, 1, "base"),
    (3, 64, 1000, 64, 1024, 4, "mix"), (5, 33, 2560, 256, 20000, 4, "mix"), (3, 17, 264, 128, 300, 1, "mix"),
    (3, 40, 2048, 128, 4096, 4, "nores"), (3, 24, 1504, 128, 2048, 4, "fp16"), (3, 64, 2048, 128, 16384, 4, "base")])
def test_layer_forward_decode_plan_matches_staged(hip_device, cfg, n, hidden, dim, n_cent, nn, variant):
    """Batches of at most 64 tokens take the decode plan (split projection
    reduced by the last workgroup to arrive, stream search with replicated
    atomic best keys, one finishing launch that merges, ranks and combines),
    checked stage by stage (check_decode_plan_stagewise).  Covers d =
    64/128/256, hidden sizes that end inside a k-step or split unevenly over
    the slices, 1 to 64 tokens, top-1 and top-4, 64/128 experts, up to 157
    search splits, modality patterns mixed inside the 16-row tiles, no
    residual, and fp16; each case runs twice on one workspace (the arrival
    counters must be left at zero)."""
    from table_moe.cache_engine import GlobalTable
    from synth import make_workload

    dev = hip_device
    dtype = torch.float16 if variant == "fp16" else None
    wl = make_workload(cfg, n=n, hidden=hidden, dim=dim, n_cent=n_cent, dtype=dtype, bias_scale=0.3)
    d = wl.to(dev)
    is_vision = d.is_vision
    if variant == "mix":
        g = torch.Generator().manual_seed(n)
        is_vision = (torch.rand(n, generator=g) < 0.5).to(dev)
    residual = None if variant == "nores" else d.residual
    a = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt))
    b = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt))
    topk = d.cfg["router_top_k"]
    for rep in range(2):
        ra = a.layer_forward(d.x, is_vision, d.logits, d.slot_out, residual, topk, nn, 0.6)
        torch.cuda.synchronize()
        if rep == 0:
            first = {k: v.clone() for k, v in ra.items()}
        else:
            for key, v in first.items():
                assert torch.equal(ra[key], v), ("second call", key)
    check_decode_plan_stagewise(b, ra, d, is_vision, residual, wl, nn)
    assert int(ra["keep"].sum()) == O.keep_count(n, 0.6)


@pytest.mark.parametrize("n", [1, 8, 32])
def test_layer_forward_config3_decode_end_to_end(hip_device, n):
    """Config 3 (decode, N = 1, 8, 32 text tokens, C=16384, top-4
    inverse-distance blend) through the one-call layer (the decode plan),
    checked stage by stage against the oracle: router, projection, top-4
    lists on the device's queries, the keep set on the device's distances,
    and the combined rows."""
    from table_moe.cache_engine import GlobalTable
    from synth import make_workload

    wl = make_workload(3, n=n)
    d = wl.to(hip_device)
    tbl = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt))
    res = tbl.layer_forward(d.x, d.is_vision, d.logits, d.slot_out, d.residual, router_top_k=8, n_nearest=4,
                            keep_rate=0.6)
    torch.cuda.synchronize()
    ww, wids, p = O.topk_softmax(np64(wl.logits), 8)
    check_topk_rows(p, np64(res["ids"]), wids, True, "router")
    q = np64(res["q"])
    ref_q = O.project_queries(np64(wl.x), wl.is_vision.numpy(), (np64(wl.proj_vis), np64(wl.bias_vis)),
                              (np64(wl.proj_txt), np64(wl.bias_txt)), False, O.BF16)
    abssum = proj_abssum(np64(wl.x), wl.is_vision.numpy(), np64(wl.proj_vis), np64(wl.proj_txt))
    assert_projection_close(q, ref_q, abssum, torch.bfloat16, min_exact=0.95)
    vals, want_idx, exact = O.global_search(q, np64(wl.centroids), 4)
    gi = np64(res["idx"])
    check_topk_rows(exact, gi, want_idx, False, "search")
    gd = np64(res["dist"])
    np.testing.assert_allclose(gd, exact[np.arange(n)[:, None], gi], rtol=1e-5, atol=1e-3)
    keep = np64(res["keep"])
    n_keep = O.keep_count(n, 0.6)
    assert keep.sum() == n_keep == {1: 1, 8: 4, 32: 19}[n]
    np.testing.assert_array_equal(keep, O.keep_select(gd[:, 0].astype(np.float32).astype(np.float64), n_keep))
    # end to end from x: the oracle's top-4 lists and keep set on its own queries
    vals_o, _, _ = check_end_to_end_topk(q, ref_q, np64(wl.centroids), gi, f"config 3 N={n} search")
    check_end_to_end_keep(gd[:, 0], vals_o[:, 0], keep, n_keep, f"config 3 N={n} keep")
    exact = O.gather_combine(keep, np64(wl.slot_out), np64(res["weights"]), np64(wl.values), gi, gd,
                             np64(wl.residual), O.F32)
    abssum = O.gather_combine(keep, np.abs(np64(wl.slot_out)), np64(res["weights"]), np.abs(np64(wl.values)), gi,
                              gd, np.abs(np64(wl.residual)), O.F32)
    assert_bf16_output(np64(res["out"]), exact, abssum)


def test_layer_forward_alternating_shapes_match_fresh_tables(hip_device):
    """One table serving calls of changing shape (token count, n_nearest),
    its stage buffers growing part-way (the per-shape layer descriptions it
    keeps must follow the reallocations), equals a fresh table on every call,
    bit for bit, in every stage output."""
    from table_moe.cache_engine import GlobalTable
    from synth import make_workload

    d = make_workload(3, n=64).to(hip_device)
    tables = lambda: GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt))
    tbl = tables()
    for n, nn, off in [(1, 4, 0), (8, 4, 3), (1, 4, 7), (32, 4, 1), (8, 1, 20), (64, 4, 0), (1, 1, 9), (8, 4, 3)]:
        sl = slice(off, off + n)
        args = (d.x[sl], d.is_vision[sl], d.logits[sl], d.slot_out[sl], d.residual[sl])
        got = tbl.layer_forward(*args, router_top_k=8, n_nearest=nn, keep_rate=0.6)
        got = {k: v.clone() for k, v in got.items()}
        want = tables().layer_forward(*args, router_top_k=8, n_nearest=nn, keep_rate=0.6)
        torch.cuda.synchronize()
        for k in ("weights", "ids", "q", "dist", "idx", "keep", "out"):
            assert got[k].shape == want[k].shape, (n, nn, k)
            assert torch.equal(got[k], want[k]), (n, nn, off, k)


def _gen_word(table):
    """Generation word of the one-launch decode plan in a table's layer workspace
    (byte 256 of the sync region): advanced once by every one-launch call."""
    ws = table._bufs["layer_ws"]
    return int(ws[256:260].view(torch.int32).item())



@pytest.mark.parametrize("cfg,n,nn,variant", [
    (3, 1, 4, "base"), (3, 8, 4, "base"), (3, 32, 4, "base"), (3, 33, 1, "mix"), (3, 64, 4, "mix"),
    (5, 17, 4, "base"), (5, 64, 1, "nores"), (3, 24, 4, "fp16"), (3, 40, 4, "dot"), (3, 32, 4, "small_c"),
    (5, 5, 1, "fp16"), (3, 12, 4, "mix"), (5, 16, 1, "mix"), (3, 8, 4, "small_c")])
def test_decode_one_launch_matches_three_launches(hip_device, cfg, n, nn, variant):
    """Decode batches with d = 128, hidden 2048 or 2560 and at most 128
    search splits run as one launch whose three phases hand q and the search
    results between workgroups through flags; with stage events the same
    call runs the three-launch plan.  Both give identical bits on three calls
    in a row on one workspace (new tokens each call: the flags' generation
    advances every call), the one-launch plan really ran (its generation word
    counts the calls), and no bounded wait ran out.  Covers 1 to 64 tokens
    (one and two query slabs; one row tile, whose projection groups reduce in
    LDS, and more, whose slices reduce through device memory), top-1 and
    top-4, 64 and 128 experts (top-6 and top-8), mixed modalities in both
    projection layouts, no residual, fp16, the dot metric and a table of 8
    splits (most workgroups idle in the search phase)."""
    from table_moe.cache_engine import GlobalTable
    from synth import make_workload

    dev = hip_device
    over = {"n_cent": 1000} if variant == "small_c" else {}
    dtype = torch.float16 if variant == "fp16" else None
    wl = make_workload(cfg, n=n, dtype=dtype, bias_scale=0.3, **over)
    d = wl.to(dev)
    is_vision = d.is_vision
    if variant == "mix":
        is_vision = (torch.rand(n, generator=_gen(n)) < 0.5).to(dev)
    residual = None if variant == "nores" else d.residual
    metric = "dot" if variant == "dot" else "l2"
    a = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt), metric=metric)
    b = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt), metric=metric)
    evs = [torch.cuda.Event() for _ in range(6)]
    topk = d.cfg["router_top_k"]
    g = _gen(7 + n)
    for rep in range(3):
        x = d.x if rep == 0 else d.x[torch.randperm(n, generator=g).to(dev)].contiguous()
        logits = d.logits if rep == 0 else torch.randn(d.logits.shape, generator=g).to(dev)
        ra = a.layer_forward(x, is_vision, logits, d.slot_out, residual, topk, nn, 0.6)
        rb = b.layer_forward(x, is_vision, logits, d.slot_out, residual, topk, nn, 0.6, stage_events=evs)
        torch.cuda.synchronize()
        for key in ("weights", "ids", "q", "qn", "dist", "idx", "keep", "out"):
            if key == "out" and ra[key] is None:
                continue
            assert torch.equal(ra[key], rb[key]), (key, rep)
        assert _gen_word(a) == rep + 1
    assert _gen_word(b) == 0  # the staged calls never touch the one-launch words
    assert a.wait_errors() == 0
    assert torch.isfinite(ra["out"].float()).all()
    # and the one-launch plan's stage outputs against the stage calls (as the three-launch plan's are)
    check_decode_plan_stagewise(b, ra, _with(d, x, logits), is_vision, residual, _with(wl, x.cpu(), logits.cpu()), nn)


def _with(wl, x, logits):
    """A copy of a workload record with other tokens and router logits."""
    kw = dict(wl.__dict__)
    kw["x"], kw["logits"] = x, logits
    return type(wl)(**kw)


@pytest.mark.parametrize("cfg,n,nn", [(2, 768, 1), (2, 4096, 1), (3, 32, 4)])
def test_layer_graph_replays_match_eager(hip_device, cfg, n, nn):
    """A captured tm_table_forward replays correctly: several replays with new
    inputs copied in and eager work in between, each checked against an eager
    call on the same inputs (the fused top-1 plan, and the decode plan whose
    arrival counters persist from replay to replay)."""
    from table_moe.cache_engine import GlobalTable
    from synth import make_workload

    dev = hip_device
    d = make_workload(cfg, n=n).to(dev)
    tg = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt))
    te = GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt))
    x = d.x.clone()
    logits = d.logits.clone()
    topk = d.cfg["router_top_k"]
    args = lambda xx, ll: (xx, d.is_vision, ll, d.slot_out, d.residual, topk, nn, 0.6)  # noqa: E731
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        tg.layer_forward(*args(x, logits))
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        res = tg.layer_forward(*args(x, logits))
    gen = torch.Generator(device=dev).manual_seed(5)
    for rep in range(4):
        if rep:
            x.copy_(d.x[torch.randperm(n, device=dev, generator=gen)])
            logits.copy_(torch.randn(logits.shape, device=dev, generator=gen))
        g.replay()
        ref = te.layer_forward(*args(x, logits))
        junk = torch.randn(1 << 20, device=dev).sum()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        for key in ("weights", "ids", "q", "dist", "idx", "keep", "out"):
            assert torch.equal(res[key], ref[key]), (rep, key)
        assert tg.wait_errors() == 0, rep


@pytest.mark.parametrize("hazard", [True, False])
def test_decode_combine_update_matches_unfused(hip_device, hazard):
    """The fused decode tail (tm_decode_combine_update) equals tm_slot_combine
    followed by update_online_cache_bs1 with the collected slot rows and the
    survivor mask, bit for bit, in the output and in the whole ring state --
    also when an online source is the ring row being overwritten."""
    from table_moe import _native as N

    dev = hip_device
    mgr, g = _mode_r_manager(dev, seed=201)
    H, k, W = 512, 8, 64
    hist = torch.randn(W, H, generator=g).to(torch.bfloat16).to(dev)
    hist_ids = torch.stack([torch.randperm(16, generator=g)[:k] for _ in range(W)]).to(dev)
    mgr.update_online_cache(hist, hist_ids, torch.randn(W, k, H, generator=g).to(torch.bfloat16).to(dev))
    assert mgr.online_ptr == 0 and mgr.online_full
    x = torch.randn(H, generator=g).to(torch.bfloat16).to(dev)
    sel = torch.randperm(16, generator=g)[:k].to(dev)
    w = torch.softmax(torch.randn(k, generator=g), 0).to(dev)
    compute = torch.tensor([1, 1, 1, 1, 0, 0, 0, 0], dtype=torch.bool, device=dev)
    computed = torch.randn(k, H, generator=g).to(torch.bfloat16).to(dev)
    on_hit = torch.tensor([0, 0, 0, 0, 1, 0, 1, 0], dtype=torch.bool, device=dev)
    on_idx = torch.tensor([0 if hazard else 17], device=dev)  # row 0 is the next ring row
    on_slot = torch.tensor([0, 0, 0, 0, 2, 0, 7, 0], device=dev)
    off_hit = torch.tensor([0, 0, 0, 0, 0, 1, 0, 0], dtype=torch.bool, device=dev)
    off_idx = torch.tensor([0, 0, 0, 0, 0, 33, 0, 0], device=dev)
    vis = torch.tensor(False, device=dev)
    state0 = [t.clone() for t in (mgr.online_keys, mgr.online_expert_ids, mgr.online_values)]

    out_f = torch.empty(H, dtype=torch.bfloat16, device=dev)
    mgr.combine_and_update_bs1(x, w, sel, vis, compute, computed, on_hit, on_idx, on_slot, off_hit, off_idx, out_f)
    torch.cuda.synchronize()
    fused = [t.clone() for t in (mgr.online_keys, mgr.online_expert_ids, mgr.online_values)]
    assert mgr.online_ptr == 1

    for t, s0 in zip((mgr.online_keys, mgr.online_expert_ids, mgr.online_values), state0):
        t.copy_(s0)
    mgr.online_ptr = 0
    out_u = torch.empty(1, H, dtype=torch.bfloat16, device=dev)
    v = mgr.values_buffer
    ov = mgr.online_values
    u8 = N.as_u8
    N.call("tm_slot_combine", N.dtype_tag(torch.bfloat16), 1, k, H, N.ptr(w.float()), k, N.ptr(u8(compute)),
           N.ptr(computed), 0, computed.stride(0), N.ptr(u8(off_hit)), N.ptr(off_idx), N.ptr(sel), k,
           N.ptr(u8(vis.reshape(1))), N.ptr(v), v.shape[0], v.shape[2], v.stride(0), v.stride(1), v.stride(2),
           N.ptr(u8(on_hit)), N.ptr(on_idx), N.ptr(on_slot), N.ptr(ov), W, ov.shape[1], ov.stride(0), ov.stride(1),
           N.TM_TARGET_ONE, None, 0, N.ptr(out_u), H, N.stream(dev))
    collected = torch.zeros(k, H, dtype=torch.bfloat16, device=dev)
    collected[:4] = computed[:4]
    collected[4] = state0[2][on_idx[0], 2]
    collected[6] = state0[2][on_idx[0], 7]
    collected[5] = v[sel[5], 1, 33]
    survivor = compute | on_hit | off_hit
    mgr.update_online_cache_bs1(x, sel, collected, survivor)
    torch.cuda.synchronize()
    assert torch.equal(out_f, out_u[0])
    for a, b_ in zip(fused, (mgr.online_keys, mgr.online_expert_ids, mgr.online_values)):
        assert torch.equal(a, b_)
    assert int(mgr.online_expert_ids[0, 7]) == -1 and torch.all(mgr.online_values[0, 7] == 0)


@pytest.mark.parametrize("hazard", [True, False])
@pytest.mark.parametrize("pattern", ["mixed", "all_survive", "none_survive"])
def test_decode_combine_update_vs_oracle(hip_device, hazard, pattern):
    """The fused decode tail against the reference's semantics restated in
    numpy: the slot sources of _forward_decode_bs1
    (models/qwen3_vl_moe/cached_layers.py:213-247: kept slots recomputed,
    online hits from online_values[on_idx, on_slot], offline hits from
    values[expert, modality, off_idx], other slots zero), the effective
    weights and matmul (:141-159, :252-259) as O.slot_combine, and the ring
    write of update_online_cache_bs1 (manager.py:89-106) as O.online_update
    -- including an online source in the ring row being overwritten."""
    dev = hip_device
    mgr, g = _mode_r_manager(dev, seed=211)
    H, k, W = 512, 8, 64
    hist = torch.randn(W, H, generator=g).to(torch.bfloat16).to(dev)
    hist_ids = torch.stack([torch.randperm(16, generator=g)[:k] for _ in range(W)]).to(dev)
    mgr.update_online_cache(hist, hist_ids, torch.randn(W, k, H, generator=g).to(torch.bfloat16).to(dev))
    ring_row = mgr.online_ptr
    x = torch.randn(H, generator=g).to(torch.bfloat16).to(dev)
    sel = torch.randperm(16, generator=g)[:k].to(dev)
    w = torch.softmax(torch.randn(k, generator=g), 0).to(dev)
    keep_k = 0 if pattern == "none_survive" else 3
    compute = torch.zeros(k, dtype=torch.bool, device=dev)
    compute[:keep_k] = True
    computed = torch.randn(k, H, generator=g).to(torch.bfloat16).to(dev)
    if pattern == "mixed":
        on_hit = torch.tensor([0, 0, 0, 1, 0, 1, 0, 0], dtype=torch.bool, device=dev)
        off_hit = torch.tensor([0, 0, 0, 0, 1, 0, 1, 0], dtype=torch.bool, device=dev)
    elif pattern == "all_survive":
        on_hit = torch.tensor([0, 0, 0, 1, 1, 0, 0, 0], dtype=torch.bool, device=dev)
        off_hit = torch.tensor([0, 0, 0, 0, 0, 1, 1, 1], dtype=torch.bool, device=dev)
    else:
        on_hit = torch.zeros(k, dtype=torch.bool, device=dev)
        off_hit = torch.zeros(k, dtype=torch.bool, device=dev)
    on_idx = torch.tensor([ring_row if hazard else (ring_row + 17) % W], device=dev)
    on_slot = torch.tensor([0, 0, 0, 2, 5, 7, 0, 0], device=dev)
    off_idx = torch.tensor([0, 0, 0, 0, 41, 200, 7, 255], device=dev)
    vis = torch.tensor(True, device=dev)
    st0 = dict(keys=np64(mgr.online_keys), ids=np64(mgr.online_expert_ids), values=np64(mgr.online_values),
               ptr=ring_row, full=True, size=W)
    out = torch.empty(H, dtype=torch.bfloat16, device=dev)
    mgr.combine_and_update_bs1(x, w, sel, vis, compute, computed, on_hit, on_idx, on_slot, off_hit, off_idx, out)
    torch.cuda.synchronize()
    # the reference's collected rows, from the state before the call
    c, oh, fh = np64(compute).astype(bool), np64(on_hit).astype(bool), np64(off_hit).astype(bool)
    collected = np.zeros((k, H))
    vals = np64(mgr.values_buffer)
    for s_ in range(k):
        if c[s_]:
            collected[s_] = np64(computed)[s_]
        elif oh[s_]:
            collected[s_] = st0["values"][int(on_idx[0]), int(on_slot[s_])]
        elif fh[s_]:
            collected[s_] = vals[int(sel[s_]), 0, int(off_idx[s_])]
    survivor = c | oh | fh
    want, _ = O.slot_combine(collected[None], np64(w)[None], survivor[None], O.BF16)
    absw, _ = O.slot_combine(np.abs(collected)[None], np64(w)[None], survivor[None], O.F32)
    got = np64(out)[None]
    if not survivor.any():
        assert (got == 0).all()
    else:
        tol = ulp(want, torch.bfloat16) + 2.0**-20 * absw
        assert np.all(np.abs(got - want) <= tol), np.abs(got - want).max()
    st1 = O.online_update(st0, np64(x)[None], np64(sel)[None], collected[None], survivor[None])
    np.testing.assert_array_equal(np64(mgr.online_keys), st1["keys"])
    np.testing.assert_array_equal(np64(mgr.online_expert_ids), st1["ids"])
    np.testing.assert_array_equal(np64(mgr.online_values), st1["values"])
    assert mgr.online_ptr == st1["ptr"]
