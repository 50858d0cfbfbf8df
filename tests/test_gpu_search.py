"""GPU parity of the search kernels against the CPU oracle.

Projection (tm_project), gated per-(expert, modality) search
(tm_search_gated), decode hybrid search (tm_search_hybrid), global-table
search (tm_search_global) and keep-rate selection (tm_keep_select).  Searches
are checked stage-wise: the oracle scores the device's own projected queries,
so a one-ulp difference in a query cannot be mistaken for a search error.
"""

import numpy as np
import pytest
import torch

from oracle import tm_oracle as O
from parity_util import ODT, assert_projection_close, assert_within_ulps, check_pick, check_topk_rows, np64, proj_abssum, ulp
from table_moe import _native as N

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _rand_proj(g, hidden, dim):
    return torch.linalg.qr(torch.randn(hidden, dim, generator=g, dtype=torch.float64))[0].float()


# ------------------------------------------------------------------ projection
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim", [16, 64, 128, 256])
@pytest.mark.parametrize("layout", ["kmajor", "rowmajor"])
@pytest.mark.parametrize("normalize", [0, 1])
@pytest.mark.parametrize("split", [True, False])
def test_project_mfma_vs_oracle(hip_device, dtype, dim, layout, normalize, split):
    g = _gen(100 + dim)
    n, hidden = 133, 512
    x = torch.randn(n, hidden, generator=g).to(dtype)
    pv, pt = _rand_proj(g, hidden, dim).to(dtype), _rand_proj(g, hidden, dim).to(dtype)
    bv, bt = (torch.randn(dim, generator=g) * 0.1).to(dtype), (torch.randn(dim, generator=g) * 0.1).to(dtype)
    vis = torch.rand(n, generator=g) < 0.5
    dev = hip_device
    xd, visd = x.to(dev), vis.to(dev)
    if layout == "kmajor":
        Pv, Pt, ps_h, ps_d = pv.t().contiguous().to(dev), pt.t().contiguous().to(dev), 1, hidden
    else:
        Pv, Pt, ps_h, ps_d = pv.contiguous().to(dev), pt.contiguous().to(dev), dim, 1
    bvd, btd = bv.to(dev), bt.to(dev)
    q = torch.empty(n, dim, dtype=dtype, device=dev)
    qn = torch.empty(n, dtype=torch.float32, device=dev)
    nbytes = N.lib().tm_project_workspace_size(n, hidden, dim)
    assert nbytes > 0  # 5 row blocks: the planner splits hidden
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev) if split else None
    N.call("tm_project", N.dtype_tag(dtype), xd.data_ptr(), n, hidden, hidden, N.as_u8(visd).data_ptr(),
           Pv.data_ptr(), bvd.data_ptr(), Pt.data_ptr(), btd.data_ptr(), ps_h, ps_d, dim, normalize, 1e-6,
           q.data_ptr(), dim, qn.data_ptr(), None if ws is None else ws.data_ptr(), nbytes if split else 0,
           N.stream(dev))
    torch.cuda.synchronize()
    ref = O.project_queries(np64(x), vis.numpy(), (np64(pv), np64(bv)), (np64(pt), np64(bt)), bool(normalize),
                            ODT[dtype])
    got = np64(q)
    abssum = proj_abssum(np64(x), vis.numpy(), np64(pv), np64(pt))
    if normalize:
        raw = O.project_queries(np64(x), vis.numpy(), (np64(pv), np64(bv)), (np64(pt), np64(bt)), False, ODT[dtype])
        abssum = abssum / np.maximum(np.linalg.norm(raw, axis=1, keepdims=True), 1e-6)
    assert_projection_close(got, ref, abssum, dtype, min_exact=0.95 if normalize else 0.97)
    np.testing.assert_allclose(np64(qn), (got * got).sum(1), rtol=2e-6, atol=1e-6)


def _pack_reference(p, dim):
    """The packed layout of a [hidden, dim] matrix as numpy: chunk
    (t*(dim/16) + c)*64 + l holds P[32t + 8(l//16) + e, 16c + l%16], e < 8."""
    hidden = p.shape[0]
    nks = -(-hidden // 32)
    pad = np.zeros((nks * 32, dim), dtype=p.dtype)
    pad[:hidden] = p
    t, c, l, e = np.meshgrid(np.arange(nks), np.arange(dim // 16), np.arange(64), np.arange(8), indexing="ij")
    return pad[32 * t + 8 * (l // 16) + e, 16 * c + l % 16].reshape(-1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hidden,dim,layout", [(2048, 128, "rowmajor"), (1000, 64, "kmajor"), (72, 256, "rowmajor"),
                                               (40, 16, "kmajor")])
def test_project_pack_layout(hip_device, dtype, hidden, dim, layout):
    g = _gen(hidden + dim)
    p = torch.randn(hidden, dim, generator=g).to(dtype)
    dev = hip_device
    src = p.to(dev) if layout == "rowmajor" else p.t().contiguous().to(dev).t()
    nbytes = N.lib().tm_project_packed_size(hidden, dim, N.dtype_tag(dtype))
    assert nbytes == -(-hidden // 32) * 32 * dim * 2
    out = torch.full((nbytes,), 0x7F, dtype=torch.uint8, device=dev)
    N.call("tm_project_pack", N.dtype_tag(dtype), src.data_ptr(), hidden, dim, src.stride(0), src.stride(1),
           out.data_ptr(), nbytes, N.stream(dev))
    torch.cuda.synchronize()
    want = _pack_reference(p.view(torch.int16).numpy(), dim)
    assert np.array_equal(out.cpu().view(torch.int16).numpy(), want)


@pytest.mark.parametrize("n,hidden,dim", [(4096, 2048, 128), (2100, 1000, 64), (40, 2056, 128), (16, 64, 32),
                                          (300, 2048, 256), (1, 2048, 128)])
def test_project_packed_vs_oracle(hip_device, n, hidden, dim):
    """Packed P at the bench shape, a hidden that ends inside a 32-wide k-step,
    small batches and a single row, with a vision block followed by
    interleaved modalities."""
    g = _gen(n + hidden + dim)
    dtype = torch.bfloat16
    x = torch.randn(n, hidden, generator=g).to(dtype)
    pv, pt = _rand_proj(g, hidden, dim).to(dtype), _rand_proj(g, hidden, dim).to(dtype)
    bv, bt = (torch.randn(dim, generator=g) * 0.1).to(dtype), (torch.randn(dim, generator=g) * 0.1).to(dtype)
    vis = torch.zeros(n, dtype=torch.bool)
    vis[: n // 2] = True
    vis[n // 2:] = torch.rand(n - n // 2, generator=g) < 0.3
    dev = hip_device
    xd, visd = x.to(dev), vis.to(dev)
    bvd, btd = bv.to(dev), bt.to(dev)
    Pv, Pt = N.pack_projection(pv.to(dev), bvd), N.pack_projection(pt.to(dev), btd)
    assert Pv is not None and Pt is not None
    q = torch.empty(n, dim, dtype=dtype, device=dev)
    qn = torch.empty(n, dtype=torch.float32, device=dev)
    N.call("tm_project", N.dtype_tag(dtype), xd.data_ptr(), n, hidden, hidden, N.as_u8(visd).data_ptr(),
           Pv.data_ptr(), bvd.data_ptr(), Pt.data_ptr(), btd.data_ptr(), 0, 0, dim, 0, 1e-6,
           q.data_ptr(), dim, qn.data_ptr(), None, 0, N.stream(dev))
    torch.cuda.synchronize()
    ref = O.project_queries(np64(x), vis.numpy(), (np64(pv), np64(bv)), (np64(pt), np64(bt)), False, ODT[dtype])
    got = np64(q)
    assert_projection_close(got, ref, proj_abssum(np64(x), vis.numpy(), np64(pv), np64(pt)), dtype, min_exact=0.97)
    np.testing.assert_allclose(np64(qn), (got * got).sum(1), rtol=2e-6, atol=1e-6)


def test_project_packed_normalized_fp16(hip_device):
    g = _gen(5)
    n, hidden, dim, dtype = 77, 512, 64, torch.float16
    x = torch.randn(n, hidden, generator=g).to(dtype)
    p = _rand_proj(g, hidden, dim).to(dtype)
    b = (torch.randn(dim, generator=g) * 0.1).to(dtype)
    dev = hip_device
    bd, xd = b.to(dev), x.to(dev)
    pk = N.pack_projection(p.to(dev), bd)
    q = torch.empty(n, dim, dtype=dtype, device=dev)
    N.call("tm_project", N.dtype_tag(dtype), xd.data_ptr(), n, hidden, hidden, None, pk.data_ptr(),
           bd.data_ptr(), None, None, 0, 0, dim, 1, 1e-6, q.data_ptr(), dim, None, None, 0, N.stream(dev))
    torch.cuda.synchronize()
    ref = O.project_queries(np64(x), np.ones(n, bool), (np64(p), np64(b)), None, True, ODT[dtype])
    raw = O.project_queries(np64(x), np.ones(n, bool), (np64(p), np64(b)), None, False, ODT[dtype])
    abssum = proj_abssum(np64(x), np.ones(n, bool), np64(p), np64(p))
    abssum = abssum / np.maximum(np.linalg.norm(raw, axis=1, keepdims=True), 1e-6)
    assert_projection_close(np64(q), ref, abssum, dtype, min_exact=0.95)


@pytest.mark.parametrize("n,hidden,dtype,normalize,mix", [
    (4096, 2048, torch.bfloat16, 1, "mixed"), (2048, 2048, torch.bfloat16, 0, "vision"),
    (2100, 2560, torch.float16, 1, "mixed"), (3000, 2048, torch.bfloat16, 1, "text")])
def test_project_packed_d64_pipelined_matches_direct(hip_device, n, hidden, dtype, normalize, mix):
    """From 2048 rows tm_project takes packed d = 64 projections at hidden
    2048 / 2560 through the pipelined column kernel (32-row tiles, one
    64-column group), below that through the direct kernel (16-row tiles).
    Both add the same per-slice MFMA chains in the same order and run the same
    row epilogue, so q and |q|^2 match bit for bit: the whole batch in one
    call against the same rows in calls of 1000 (mixed modalities inside the
    tiles, normalised and not, bf16 and fp16, a ragged last tile), and the
    oracle checks the values (a normalised component within two ulps: one
    from its unnormalised value, one from a norm rounded the other way)."""
    g = _gen(n + hidden)
    dim = 64
    x = torch.randn(n, hidden, generator=g).to(dtype)
    pv, pt = _rand_proj(g, hidden, dim).to(dtype), _rand_proj(g, hidden, dim).to(dtype)
    bv, bt = (torch.randn(dim, generator=g) * 0.1).to(dtype), (torch.randn(dim, generator=g) * 0.1).to(dtype)
    vis = {"mixed": torch.rand(n, generator=g) < 0.5, "vision": torch.ones(n, dtype=torch.bool),
           "text": torch.zeros(n, dtype=torch.bool)}[mix]
    dev = hip_device
    xd, visd = x.to(dev), vis.to(dev)
    bvd, btd = bv.to(dev), bt.to(dev)
    Pv, Pt = N.pack_projection(pv.to(dev), bvd), N.pack_projection(pt.to(dev), btd)

    def project(lo, hi, q, qn):
        N.call("tm_project", N.dtype_tag(dtype), xd[lo:hi].data_ptr(), hi - lo, hidden, hidden,
               N.as_u8(visd[lo:hi]).data_ptr(), Pv.data_ptr(), bvd.data_ptr(), Pt.data_ptr(), btd.data_ptr(), 0, 0,
               dim, normalize, 1e-6, q[lo:hi].data_ptr(), dim, qn[lo:hi].data_ptr(), None, 0, N.stream(dev))

    q_one = torch.empty(n, dim, dtype=dtype, device=dev)
    qn_one = torch.empty(n, dtype=torch.float32, device=dev)
    project(0, n, q_one, qn_one)
    q_parts = torch.empty_like(q_one)
    qn_parts = torch.empty_like(qn_one)
    for lo in range(0, n, 1000):
        project(lo, min(lo + 1000, n), q_parts, qn_parts)
    torch.cuda.synchronize()
    assert torch.equal(q_one.view(torch.int16), q_parts.view(torch.int16))
    assert torch.equal(qn_one, qn_parts)
    ref = O.project_queries(np64(x), vis.numpy(), (np64(pv), np64(bv)), (np64(pt), np64(bt)), bool(normalize),
                            ODT[dtype])
    abssum = proj_abssum(np64(x), vis.numpy(), np64(pv), np64(pt))
    if normalize:
        raw = O.project_queries(np64(x), vis.numpy(), (np64(pv), np64(bv)), (np64(pt), np64(bt)), False, ODT[dtype])
        abssum = abssum / np.maximum(np.linalg.norm(raw, axis=1, keepdims=True), 1e-6)
    got = np64(q_one)
    if normalize:
        # a normalised component: one ulp from the unnormalised one (fp32
        # accumulation order) and one more when the rounded norm it divides by
        # came out on the other side
        tol = 2.0 * ulp(ref, dtype) + 2.0**-18 * abssum
        assert not (np.abs(got - ref) > tol).any()
        assert float(np.mean(got == ref)) >= 0.95
    else:
        assert_projection_close(got, ref, abssum, dtype, min_exact=0.97)
    np.testing.assert_allclose(np64(qn_one), (got * got).sum(1), rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("dtype,dim", [(torch.float32, 2), (torch.float32, 64), (torch.bfloat16, 48)])
def test_project_scalar_path_vs_oracle(hip_device, dtype, dim):
    g = _gen(7)
    n, hidden = 37, 96
    x = torch.randn(n, hidden, generator=g).to(dtype)
    p = _rand_proj(g, hidden, dim).to(dtype).contiguous()  # row-major [hidden, dim]
    b = (torch.randn(dim, generator=g) * 0.1).to(dtype)
    dev = hip_device
    xd, pd, bd = x.to(dev), p.to(dev), b.to(dev)
    assert pd.stride() == (dim, 1)
    q = torch.empty(n, dim, dtype=dtype, device=dev)
    qn = torch.empty(n, dtype=torch.float32, device=dev)
    N.call("tm_project", N.dtype_tag(dtype), xd.data_ptr(), n, hidden, hidden, None, pd.data_ptr(), bd.data_ptr(),
           None, None, dim, 1, dim, 1, 1e-6, q.data_ptr(), dim, qn.data_ptr(), None, 0, N.stream(dev))
    torch.cuda.synchronize()
    ref = O.project_queries(np64(x), np.ones(n, bool), (np64(p), np64(b)), None, True, ODT[dtype])
    if dtype == torch.float32:
        np.testing.assert_allclose(np64(q), ref, rtol=2e-5, atol=2e-6)
    else:
        raw = O.project_queries(np64(x), np.ones(n, bool), (np64(p), np64(b)), None, False, ODT[dtype])
        abssum = proj_abssum(np64(x), np.ones(n, bool), np64(p), np64(p))
        abssum = abssum / np.maximum(np.linalg.norm(raw, axis=1, keepdims=True), 1e-6)
        assert_projection_close(np64(q), ref, abssum, dtype, min_exact=0.95)
    np.testing.assert_allclose(np64(qn), (np64(q) ** 2).sum(1), rtol=2e-6, atol=1e-6)


# ---------------------------------------------------------------- gated search
def _norm_rows(t):
    return t / t.norm(dim=-1, keepdim=True).clamp_min(1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("cmp", [N.TM_CMP_GE, N.TM_CMP_GT])
@pytest.mark.parametrize("col_offset", [0, 3])
def test_search_gated_vs_oracle(hip_device, dtype, cmp, col_offset):
    g = _gen(11)
    E, K, d, n, k = 16, 256, 64, 300, 8
    keys = _norm_rows(torch.randn(E, 2, K, d, generator=g)).to(dtype)
    q = _norm_rows(torch.randn(n, d, generator=g)).to(dtype)
    sel = torch.randint(0, E, (n, k), generator=g)
    bad = torch.rand(n, k, generator=g) < 0.03
    sel[bad] = torch.where(torch.rand(int(bad.sum()), generator=g) < 0.5, -1, E)  # out-of-range ids: never searched
    vis = torch.rand(n, generator=g) < 0.6
    reuse = torch.rand(n, k, generator=g) < 0.6
    thr_v, thr_t = 0.33, 0.36
    dev = hip_device
    qd, kd, seld, visd, rsd = q.to(dev), keys.to(dev), sel.to(dev), vis.to(dev), reuse.to(dev)
    big_hit = torch.full((n, k + 3), 7, dtype=torch.uint8, device=dev)
    big_idx = torch.full((n, k + 3), -7, dtype=torch.long, device=dev)
    hit, idx = big_hit[:, :k], big_idx[:, :k]  # strided outputs
    N.call("tm_search_gated", N.dtype_tag(dtype), qd.data_ptr(), n, d, kd.data_ptr(), E, K, d, kd.stride(0),
           kd.stride(1), kd.stride(2), seld.data_ptr(), k, k, 1, N.as_u8(visd).data_ptr(), N.as_u8(rsd).data_ptr(),
           k, 1, col_offset, thr_v, thr_t, cmp, hit.data_ptr(), idx.data_ptr(), k + 3, 1, N.stream(dev))
    torch.cuda.synchronize()
    assert (big_hit[:, k:] == 7).all() and (big_idx[:, k:] == -7).all()
    want_hit, want_idx, mx, scores = O.search_gated(np64(q), np64(keys), sel.numpy(), vis.numpy(), reuse.numpy(),
                                                    thr_v, thr_t, cmp, col_offset=col_offset)
    got_hit, got_idx = np64(hit).astype(bool), np64(idx)
    assert np.isin(np64(hit), [0, 1]).all()
    n_hits = 0
    for b in range(n):
        thr = float(np.float32(thr_v if vis[b] else thr_t))
        for s in range(k):
            if np.isnan(mx[b, s]):
                assert not got_hit[b, s] and got_idx[b, s] == 0
                continue
            assert O.threshold_ok(mx[b, s], thr, got_hit[b, s], want_hit[b, s]), (b, s, mx[b, s])
            if got_hit[b, s]:
                n_hits += 1
                best = int(np.argmax(scores[b, s]))
                check_pick(scores[b, s], got_idx[b, s], best, True, f"token {b} slot {s}")
            else:
                assert got_idx[b, s] == 0
    assert n_hits > 50  # the thresholds produce both hits and misses


def test_engine_reference_kat_dot(hip_device):
    """table_moe/cache_engine/test_search.py:48-89 on the device: fp32 identity
    PCA, raw keys {[1,0],[-1,0]} and {[0,0],[-1,0]}, query [1,0]."""
    from table_moe.cache_engine import CacheConfig, VectorSearchEngine

    class DummyManager:
        def __init__(self, dev):
            self.device = dev
            self.keys_buffer = torch.zeros((2, 2, 2, 2), dtype=torch.float32, device=dev)
            self.raw_keys_buffer = torch.zeros((2, 2, 2, 2), dtype=torch.float32, device=dev)
            eye = {"proj": torch.eye(2, device=dev), "bias": torch.zeros(2, device=dev)}
            self.pca = {"vision": dict(eye), "text": dict(eye)}
            self.online_expert_ids = None

    dev = hip_device
    m = DummyManager(dev)
    m.raw_keys_buffer[0, 0] = torch.tensor([[1.0, 0.0], [-1.0, 0.0]], device=dev)
    m.raw_keys_buffer[1, 0] = torch.tensor([[0.0, 0.0], [-1.0, 0.0]], device=dev)
    old = float(CacheConfig.OFFLINE_DOT_THRESHOLD)
    CacheConfig.OFFLINE_DOT_THRESHOLD = 0.0
    try:
        eng = VectorSearchEngine(m)
        args = dict(layer_idx=0, hidden_states=torch.tensor([[1.0, 0.0], [1.0, 0.0]], device=dev),
                    selected_experts=torch.tensor([[0], [1]], device=dev),
                    is_vision_mask=torch.tensor([True, True], device=dev),
                    reuse_mask=torch.tensor([[True], [True]], device=dev))
        for fn in (eng.search_prefill_offline_dot, eng.search_decode_offline_dot):
            hit, idx = fn(**args)
            assert bool(hit[0, 0].item()) and int(idx[0, 0].item()) == 0
            assert not bool(hit[1, 0].item())
    finally:
        CacheConfig.OFFLINE_DOT_THRESHOLD = old


# --------------------------------------------------------------- hybrid search
@pytest.mark.parametrize("n_valid", [0, 5, 64])
@pytest.mark.parametrize("keep_k", [0, 4, 8])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_search_hybrid_vs_oracle(hip_device, n_valid, keep_k, dtype):
    g = _gen(21 + n_valid + keep_k)
    E, K, d, H, n, k, W, wk = 24, 256, 64, 512, 20, 8, 64, 8
    keys = _norm_rows(torch.randn(E, 2, K, d, generator=g)).to(dtype)
    pv, pt = _rand_proj(g, H, d).to(dtype), _rand_proj(g, H, d).to(dtype)
    bv, bt = (torch.randn(d, generator=g) * 0.05).to(dtype), (torch.randn(d, generator=g) * 0.05).to(dtype)
    on_keys = torch.randn(W, H, generator=g).to(dtype)
    x = (0.7 * on_keys[torch.randint(0, max(n_valid, 1), (n,), generator=g)].float()
         + torch.randn(n, H, generator=g)).to(dtype)
    x[::5] = -x[::5]  # some tokens with no positive online score
    sel = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(n)])
    on_ids = torch.randint(0, E, (W, wk), generator=g)
    on_ids[torch.rand(W, wk, generator=g) < 0.2] = -1
    vis = torch.rand(n, generator=g) < 0.5
    dev = hip_device
    T = lambda t: t.to(dev)  # noqa: E731
    xd, kd, visd, seld, okd, oid = T(x), T(keys), T(vis), T(sel), T(on_keys), T(on_ids)
    pvt, ptt, bvd, btd = T(pv.t().contiguous()), T(pt.t().contiguous()), T(bv), T(bt)
    on_hit = torch.full((n, k), 9, dtype=torch.uint8, device=dev)
    off_hit = torch.full((n, k), 9, dtype=torch.uint8, device=dev)
    on_idx = torch.full((n,), -9, dtype=torch.long, device=dev)
    off_idx = torch.full((n, k), -9, dtype=torch.long, device=dev)
    on_slot = torch.full((n, k), -9, dtype=torch.long, device=dev)
    ws = torch.zeros(n, d, dtype=dtype, device=dev)  # the projected queries
    nbytes = N.lib().tm_search_hybrid_workspace_size(n, H, d)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    N.call("tm_search_hybrid", N.dtype_tag(dtype), xd.data_ptr(), n, H, H, N.as_u8(visd).data_ptr(), pvt.data_ptr(),
           bvd.data_ptr(), ptt.data_ptr(), btd.data_ptr(), 1, H, d, okd.data_ptr() if n_valid else None, H, n_valid,
           oid.data_ptr() if n_valid else None, wk, wk, kd.data_ptr(), E, K, kd.stride(0), kd.stride(1), kd.stride(2),
           seld.data_ptr(), k, k, 1, keep_k, on_hit.data_ptr(), on_idx.data_ptr(), off_hit.data_ptr(),
           off_idx.data_ptr(), on_slot.data_ptr(), k, 1, ws.data_ptr(), d, scratch.data_ptr(), nbytes, N.stream(dev))
    torch.cuda.synchronize()
    ref = O.search_hybrid(np64(x), vis.numpy(), (np64(pv), np64(bv)), (np64(pt), np64(bt)), ODT[dtype], np64(keys),
                          sel.numpy(), keep_k, np64(on_keys) if n_valid else None, on_ids.numpy() if n_valid else None,
                          n_valid)
    g_on_hit, g_on_idx, g_off_hit = np64(on_hit), np64(on_idx), np64(off_hit)
    g_off_idx, g_on_slot = np64(off_idx), np64(on_slot)
    assert np.isin(g_on_hit, [0, 1]).all() and np.isin(g_off_hit, [0, 1]).all()
    assert (g_on_hit[:, :keep_k] == 0).all() and (g_off_hit[:, :keep_k] == 0).all()
    # online stage
    if n_valid and keep_k < k:
        for b in range(n):
            sc = ref["on_scores"][b]
            best = int(np.argmax(sc))
            if g_on_idx[b] >= 0:
                check_pick(sc, g_on_idx[b], best, True, f"online token {b}")
            assert O.threshold_ok(ref["on_max"][b], 0.0, g_on_idx[b] >= 0, ref["on_idx"][b] >= 0)
        same_online = g_on_idx == ref["on_idx"]
        np.testing.assert_array_equal(g_on_hit[same_online].astype(bool), ref["on_hit"][same_online])
        np.testing.assert_array_equal(g_on_slot[same_online], ref["on_slot"][same_online])
    else:
        assert (g_on_idx == -1).all() and (g_on_hit == 0).all()
    # offline stage, scored on the device's own projected queries
    if keep_k < k:
        rows = np.nonzero(((g_on_hit == 0)[:, keep_k:]).any(1))[0]
        qg = np64(ws)
        abssum = proj_abssum(np64(x), vis.numpy(), np64(pv), np64(pt))
        assert_projection_close(qg[rows], ref["q_low"][rows], abssum[rows], dtype, min_exact=0.9)
        reuse = np.zeros((n, k), bool)
        reuse[:, keep_k:] = g_on_hit[:, keep_k:] == 0
        h, i, mx, scores = O.search_gated(qg, np64(keys), sel.numpy(), vis.numpy(), reuse, 0.0, 0.0, O.CMP_GE)
        for b in range(n):
            for s in range(k):
                if not reuse[b, s]:
                    assert g_off_hit[b, s] == 0 and g_off_idx[b, s] == 0
                    continue
                assert O.threshold_ok(mx[b, s], 0.0, g_off_hit[b, s], h[b, s])
                if g_off_hit[b, s]:
                    check_pick(scores[b, s], g_off_idx[b, s], int(np.argmax(scores[b, s])), True, f"off {b},{s}")
                else:
                    assert g_off_idx[b, s] == 0


# ---------------------------------------------------------- global-table search
GLOBAL_CASES = [
    # n, C, dim, top_k, metric, dtype
    (4096, 8192, 128, 1, "l2", torch.bfloat16),  # config 2 shape
    (1, 16384, 128, 4, "l2", torch.bfloat16),    # config 3 decode shapes
    (8, 16384, 128, 4, "l2", torch.bfloat16),
    (32, 16384, 128, 4, "l2", torch.bfloat16),
    (256, 1024, 64, 1, "l2", torch.bfloat16),    # config 1 shape (bf16 storage)
    (300, 1000, 64, 8, "l2", torch.float16),
    (77, 5000, 256, 2, "dot", torch.bfloat16),
    (33, 129, 128, 3, "l2", torch.float16),
    (130, 77, 128, 1, "dot", torch.float16),
    # wide top-1 kernel (8-wave workgroups, one per CU): dot metric and fp16, d = 64
    (4096, 8192, 128, 1, "dot", torch.float16),
    (4096, 16384, 64, 1, "l2", torch.float16),
]


@pytest.mark.parametrize("n,c,dim,top_k,metric,dtype", GLOBAL_CASES)
def test_search_global_vs_oracle(hip_device, n, c, dim, top_k, metric, dtype):
    g = _gen(31 + n + c)
    cents = torch.randn(c, dim, generator=g)
    near = cents[torch.randint(0, c, (n,), generator=g)] + 0.2 * torch.randn(n, dim, generator=g)
    q = torch.where((torch.rand(n, 1, generator=g) < 0.7), near, torch.randn(n, dim, generator=g) * 1.2).to(dtype)
    cents = cents.to(dtype)
    dev = hip_device
    qd, cd = q.to(dev), cents.to(dev)
    from table_moe.cache_engine.global_table import GlobalTable

    H = 16
    tbl = GlobalTable(cd, torch.zeros(c, H, dtype=dtype, device=dev),
                      (torch.zeros(H, dim, dtype=dtype, device=dev), torch.zeros(dim, dtype=dtype, device=dev)),
                      metric=metric)
    dist, idx = tbl.search(qd, top_k)
    torch.cuda.synchronize()
    vals, want_idx, exact = O.global_search(np64(q), np64(cents), top_k, metric)
    got_idx = np64(idx)
    check_topk_rows(exact, got_idx, want_idx, larger_is_better=(metric == "dot"), what=f"global {metric}")
    got_exact = np.take_along_axis(exact, got_idx, axis=1)
    scale = np.abs(np64(q) ** 2).sum(1, keepdims=True) + (np64(cents) ** 2).sum(1).max()
    np.testing.assert_allclose(np64(dist), got_exact, rtol=0, atol=float(scale.max()) * 2e-6 + 1e-5)
    np.testing.assert_allclose(np64(tbl.c_sqnorm), (np64(cents) ** 2).sum(1), rtol=2e-6)


@pytest.mark.parametrize("n,c,dim,top_k,metric", [
    (777, 3000, 128, 1, "l2"),    # tile kernel, several splits and a partial last stage
    (300, 2100, 64, 1, "l2"),
    (513, 1500, 128, 1, "dot"),
    (300, 1000, 128, 4, "l2"),    # top-k tile kernel
    (40, 3000, 128, 1, "l2"),     # decode-sized stream kernel
    (40, 3000, 128, 4, "l2"),
    (4096, 8192, 128, 1, "l2"),   # wide top-1 kernel: ties across its two block halves and ranges
    (4096, 8192, 128, 1, "dot"),
])
def test_search_global_exact_ties(hip_device, n, c, dim, top_k, metric):
    """Centroid rows repeat (row i equals row i % 97), so every distance is tied
    with at least one other centroid bit for bit: each kernel path must return
    the lowest index among the tied centroids, as the reference's first-minimum
    rule does (search.py argmin / topk order)."""
    g = _gen(53 + n + c + top_k)
    base = torch.randn(97, dim, generator=g).to(torch.bfloat16)
    cents = base[torch.arange(c) % 97]
    q = (base[torch.randint(0, 97, (n,), generator=g)].float() + 0.3 * torch.randn(n, dim, generator=g)).to(torch.bfloat16)
    dev = hip_device
    from table_moe.cache_engine.global_table import GlobalTable

    H = 16
    tbl = GlobalTable(cents.to(dev), torch.zeros(c, H, dtype=torch.bfloat16, device=dev),
                      (torch.zeros(H, dim, dtype=torch.bfloat16, device=dev),
                       torch.zeros(dim, dtype=torch.bfloat16, device=dev)), metric=metric)
    dist, idx = tbl.search(q.to(dev), top_k)
    torch.cuda.synchronize()
    got = np64(idx)
    # distances of the 97 distinct rows; the true answer lists, per distinct
    # row in rank order, its first occurrences (index r, then r + 97, ...)
    _, want_base, exact_base = O.global_search(np64(q), np64(base), 97, metric)
    assert got.min() >= 0 and got.max() < c
    # every returned index must be one of the lowest-indexed copies of a
    # best-ranked distinct row: for top-1, exactly the first copy of the best row
    for r in range(n):
        row_rank = want_base[r]
        if top_k == 1:
            b0 = int(row_rank[0])
            if exact_base[r, b0] == exact_base[r, int(row_rank[1])]:
                continue  # two distinct rows at the same distance: not this test's concern
            assert got[r, 0] == b0, f"row {r}: got {got[r, 0]} want {b0}"
        else:
            # the best distinct row has c // 97 (+1) copies; the top_k list must be
            # its lowest-indexed copies in increasing index order
            b0 = int(row_rank[0])
            copies = np.arange(b0, c, 97)[:top_k]
            if len(copies) == top_k:
                np.testing.assert_array_equal(got[r], copies, err_msg=f"row {r}")


def test_search_global_precomputed_qnorm_and_repeat(hip_device):
    """The q_sqnorm argument changes nothing; a second call reuses the workspace."""
    from table_moe.cache_engine.global_table import GlobalTable

    g = _gen(41)
    dev = hip_device
    c, dim, H = 3000, 128, 256
    cents = torch.randn(c, dim, generator=g).to(torch.bfloat16).to(dev)
    x = torch.randn(500, H, generator=g).to(torch.bfloat16).to(dev)
    p = _rand_proj(g, H, dim).to(torch.bfloat16).to(dev)
    tbl = GlobalTable(cents, torch.zeros(c, H, dtype=torch.bfloat16, device=dev),
                      (p, torch.zeros(dim, dtype=torch.bfloat16, device=dev)))
    q, qn = tbl.project(x)
    d1, i1 = [t.clone() for t in tbl.search(q, 1, qn)]
    d2, i2 = [t.clone() for t in tbl.search(q, 1)]
    q2, _ = tbl.project(x[:100])
    d3, i3 = [t.clone() for t in tbl.search(q2, 1)]
    torch.cuda.synchronize()
    assert torch.equal(i1, i2) and torch.equal(i1[:100], i3)
    torch.testing.assert_close(d1, d2, rtol=0, atol=1e-3)


# ------------------------------------------------------------- keep selection
@pytest.mark.parametrize("n", [1, 2, 5, 1023, 1024, 1025, 4096, 5000, 16384, 16385, 70000])
@pytest.mark.parametrize("pattern", ["random", "ties", "constant", "signed", "clustered"])
def test_keep_select_exact(hip_device, n, pattern):
    g = _gen(51 + n)
    if pattern == "random":
        s = torch.rand(n, generator=g) * 300
    elif pattern == "ties":
        s = torch.randint(0, 7, (n,), generator=g).float() * 0.5
    elif pattern == "constant":
        s = torch.full((n,), 3.25)
    elif pattern == "clustered":  # one exponent, keys differing only in low mantissa bits
        s = 100.0 + torch.randint(0, 50, (n,), generator=g).float() * 2.0 ** -16
    else:
        s = torch.randn(n, generator=g) * 1e3
        s[: n // 3] = -0.0
    dev = hip_device
    col = torch.zeros(n, 4)
    col[:, 0] = s
    sd = col.to(dev)[:, 0]  # strided score column
    keep = torch.empty(n, dtype=torch.bool, device=dev)
    for n_keep in sorted({0, 1, n // 3, O.keep_count(n, 0.6), n - 1, n}):
        keep.fill_(False)
        N.call("tm_keep_select", sd.data_ptr(), n, 4, n_keep, N.as_u8(keep).data_ptr(), None, 0, N.stream(dev))
        torch.cuda.synchronize()
        want = O.keep_select(np64(s), n_keep)
        np.testing.assert_array_equal(np64(keep), want, err_msg=f"n={n} n_keep={n_keep}")
