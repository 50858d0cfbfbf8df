"""GPU parity of the reference-semantics ("mode R") searches at the shapes the
Qwen3-VL-30B-A3B layers use (128 experts x 2 modalities x 256 centroids in
64-d, hidden 2048, top-8, N=4096 prefill / 1 token decode), of the
segment-grouped gated search kernel on its edge cases (duplicate and
out-of-range expert ids, ragged tables, other dims and dtypes, large top_k,
tiny batches), and of the fp32 tiled projection."""

import numpy as np
import pytest
import torch

from oracle import tm_oracle as O
from parity_util import ODT, check_gated_end_to_end, check_pick, np64, proj_abssum, ulp
from table_moe import _native as N

pytestmark = pytest.mark.gpu


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _norm_rows(t):
    return t / t.norm(dim=-1, keepdim=True).clamp_min(1e-6)


def check_gated(q, keys, sel, vis, reuse, hit, idx, thr_v, thr_t, cmp, col_offset=0, rows=None, min_hits=1):
    """Device (hit, idx) against O.search_gated on the device's own queries:
    hit flags exact except within the near-threshold rule, hit indices exact
    except within the near-tie rule, misses and unsearched slots (0, 0)."""
    rows = np.arange(sel.shape[0]) if rows is None else rows
    want_hit, _, mx, scores = O.search_gated(np64(q)[rows], np64(keys), np64(sel)[rows], np64(vis)[rows],
                                             None if reuse is None else np64(reuse)[rows], thr_v, thr_t, cmp,
                                             col_offset=col_offset)
    got_hit, got_idx = np64(hit)[rows].astype(bool), np64(idx)[rows]
    assert np.isin(np64(hit)[rows], [0, 1]).all()
    visn = np64(vis)[rows]
    n_hits = 0
    for i in range(len(rows)):
        thr = float(np.float32(thr_v if visn[i] else thr_t))
        for s in range(sel.shape[1]):
            if np.isnan(mx[i, s]):
                assert not got_hit[i, s] and got_idx[i, s] == 0, (rows[i], s)
                continue
            assert O.threshold_ok(mx[i, s], thr, got_hit[i, s], want_hit[i, s]), (rows[i], s, mx[i, s])
            if got_hit[i, s]:
                n_hits += 1
                check_pick(scores[i, s], got_idx[i, s], int(np.argmax(scores[i, s])), True, f"row {rows[i]} slot {s}")
            else:
                assert got_idx[i, s] == 0
    assert n_hits >= min_hits, n_hits
    return n_hits


def _gated(dtype, q, keys, sel, vis, reuse, thr_v, thr_t, cmp, col_offset=0):
    dev = q.device
    n, k = sel.shape
    hit = torch.full((n, k), 9, dtype=torch.uint8, device=dev)
    idx = torch.full((n, k), -9, dtype=torch.long, device=dev)
    rs = None if reuse is None else N.as_u8(reuse)
    N.call("tm_search_gated", N.dtype_tag(dtype), q.data_ptr(), n, q.stride(0), keys.data_ptr(), keys.shape[0],
           keys.shape[2], keys.shape[3], keys.stride(0), keys.stride(1), keys.stride(2), sel.data_ptr(), k,
           sel.stride(0), sel.stride(1), N.as_u8(vis).data_ptr(), N.ptr(rs), 0 if rs is None else rs.stride(0),
           0 if rs is None else rs.stride(1), col_offset, thr_v, thr_t, cmp, hit.data_ptr(), idx.data_ptr(), k, 1,
           N.stream(dev))
    torch.cuda.synchronize()
    return hit, idx


# ------------------------------------------------------------- Qwen shapes
@pytest.fixture(scope="module")
def qwen(hip_device):
    from synth import make_mode_r_manager

    return make_mode_r_manager(hip_device)


def test_prefill_offline_qwen_shape_vs_oracle(hip_device, qwen):
    """search_prefill_offline at N=4096 (3584 vision + 512 text), top-8 of 128
    experts, reuse from the expert keep mask at keep_rate 0.6, half the
    tokens placed near a key of their first expert: the engine's queries
    against the oracle projection, and the search on those queries against
    the oracle on 512 sampled tokens of each modality mix; the reuse mask's
    complement is (0, 0) on every token."""
    from synth import make_workload
    from table_moe.cache_engine import CacheConfig, VectorSearchEngine
    from table_moe.ops import qwen_topk_softmax
    from table_moe.skip import build_prefill_keep_mask

    dev = hip_device
    mgr = qwen
    eng = VectorSearchEngine(mgr)
    wl = make_workload(2, with_slot_out=False, device=dev, gen_device=dev)
    n, k = wl.x.shape[0], 8
    w, sel = qwen_topk_softmax(wl.logits, k)
    reuse = ~build_prefill_keep_mask(sel, w, torch.rand(n, device=dev), 128, 0.6)
    g = torch.Generator(device=dev).manual_seed(9)
    near = torch.rand(n, device=dev, generator=g) < 0.5
    src = mgr.keys_buffer[sel[:, 0], (~wl.is_vision).long(), torch.randint(0, 256, (n,), device=dev, generator=g)]
    p_v, p_t = mgr.pca["vision"]["proj"].float(), mgr.pca["text"]["proj"].float()
    lift = torch.where(wl.is_vision[:, None], src.float() @ p_v.T, src.float() @ p_t.T) * 4.0
    x = torch.where(near[:, None], wl.x.float() * 0.2 + lift, wl.x.float()).to(torch.bfloat16)
    hit, idx = eng.search_prefill_offline(0, x, sel, wl.is_vision, reuse)
    torch.cuda.synchronize()
    q = eng.prefill_query_workspace[:n]
    pca = mgr.pca
    rows = np.concatenate([np.arange(0, 3584, 9)[:400], np.arange(3584, 4096, 4)[:112]])
    ref_q = O.project_queries(np64(x)[rows], np64(wl.is_vision)[rows],
                              (np64(pca["vision"]["proj"]), np64(pca["vision"]["bias"])),
                              (np64(pca["text"]["proj"]), np64(pca["text"]["bias"])), True, O.BF16)
    got_q = np64(q)[rows]
    raw = O.project_queries(np64(x)[rows], np64(wl.is_vision)[rows],
                            (np64(pca["vision"]["proj"]), np64(pca["vision"]["bias"])),
                            (np64(pca["text"]["proj"]), np64(pca["text"]["bias"])), False, O.BF16)
    abssum = proj_abssum(np64(x)[rows], np64(wl.is_vision)[rows], np64(pca["vision"]["proj"]),
                         np64(pca["text"]["proj"])) / np.maximum(np.linalg.norm(raw, axis=1, keepdims=True), 1e-6)
    # the raw value may round the other way by one ulp, which the normalisation carries
    assert np.all(np.abs(got_q - ref_q) <= 2 * ulp(ref_q, torch.bfloat16) + 2.0**-18 * abssum)
    thr_v, thr_t = CacheConfig.OFFLINE_COSINE_THRESHOLD_VISION, CacheConfig.OFFLINE_COSINE_THRESHOLD_TEXT
    check_gated(q, mgr.keys_buffer, sel, wl.is_vision, reuse, hit, idx, thr_v, thr_t, O.CMP_GE, rows=rows,
                min_hits=50)
    # end to end from x: the oracle's search on its own normalised queries
    check_gated_end_to_end(got_q, ref_q, np64(mgr.keys_buffer), np64(sel)[rows], np64(wl.is_vision)[rows],
                           np64(reuse)[rows], np64(hit)[rows], np64(idx)[rows], thr_v, thr_t, O.CMP_GE,
                           what="prefill offline (Qwen shape)")
    rs = np64(reuse)
    assert not np64(hit)[~rs].any() and (np64(idx)[~rs] == 0).all()
    assert np64(hit).sum() > 200


def test_decode_offline_entry_points_qwen_shape(hip_device, qwen):
    """search_decode_offline (fused projection, hit = max >= 0 on normalised
    keys), search_decode_offline_dot and search_decode_offline_bs1_into (raw
    keys, hit = max > 0) at the Qwen decode shape: the device's decode
    queries (raw projection) against the oracle, then each search against
    O.search_gated on those queries."""
    from table_moe.cache_engine import CacheConfig, VectorSearchEngine

    dev = hip_device
    mgr = qwen
    eng = VectorSearchEngine(mgr)
    g = _gen(77)
    n, k, H = 8, 8, 2048
    x = (torch.randn(n, H, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    sel = torch.stack([torch.randperm(128, generator=g)[:k] for _ in range(n)]).to(dev)
    vis = torch.tensor([True, False] * 4, device=dev)
    reuse = (torch.rand(n, k, generator=g) < 0.6).to(dev)
    pca = mgr.pca
    hit, idx = eng.search_decode_offline(0, x, sel, vis, reuse)
    torch.cuda.synchronize()
    q = eng.decode_query_workspace[:n].clone()
    ref_q = O.project_queries(np64(x), np64(vis), (np64(pca["vision"]["proj"]), np64(pca["vision"]["bias"])),
                              (np64(pca["text"]["proj"]), np64(pca["text"]["bias"])), False, O.BF16)
    abssum = proj_abssum(np64(x), np64(vis), np64(pca["vision"]["proj"]), np64(pca["text"]["proj"]))
    assert np.all(np.abs(np64(q) - ref_q) <= ulp(ref_q, torch.bfloat16) + 2.0**-18 * abssum)
    check_gated(q, mgr.keys_buffer, sel, vis, reuse, hit, idx, 0.0, 0.0, O.CMP_GE, min_hits=5)
    check_gated_end_to_end(np64(q), ref_q, np64(mgr.keys_buffer), np64(sel), np64(vis), np64(reuse), np64(hit),
                           np64(idx), 0.0, 0.0, O.CMP_GE, what="decode offline")
    hit2, idx2 = eng.search_decode_offline_dot(0, x, sel, vis, reuse)
    torch.cuda.synchronize()
    thr = float(CacheConfig.OFFLINE_DOT_THRESHOLD)
    check_gated(q, mgr.raw_keys_buffer, sel, vis, reuse, hit2, idx2, thr, thr, O.CMP_GT, min_hits=5)
    check_gated_end_to_end(np64(q), ref_q, np64(mgr.raw_keys_buffer), np64(sel), np64(vis), np64(reuse),
                           np64(hit2), np64(idx2), thr, thr, O.CMP_GT, what="decode offline dot")
    keep_k = 4
    for b in range(n):
        oh = torch.full((k,), True, device=dev)
        oi = torch.full((k,), -5, dtype=torch.long, device=dev)
        eng.search_decode_offline_bs1_into(x[b], sel[b], vis[b], keep_k, oh, oi)
        torch.cuda.synchronize()
        check_gated(q[b:b + 1], mgr.raw_keys_buffer, sel[b:b + 1], vis[b:b + 1], None, oh.view(1, k),
                    oi.view(1, k), thr, thr, O.CMP_GT, col_offset=keep_k, min_hits=0)


def test_decode_hybrid_bs1_qwen_shape_vs_oracle(hip_device, qwen):
    """search_decode_hybrid_bs1_into with the full 64-entry online window at
    the Qwen decode shape (keep_k 4 of top-8): online index, online hits and
    slots, and the offline search of the rest against O.search_hybrid; one
    token drawn near a window entry so the online path hits."""
    from table_moe.cache_engine import VectorSearchEngine

    dev = hip_device
    mgr = qwen
    eng = VectorSearchEngine(mgr)
    g = _gen(91)
    k, H = 8, 2048
    pca = mgr.pca
    for t, near in enumerate((True, False, True)):
        if near:
            j = 5 + 20 * t
            x = (mgr.online_keys[j].float().cpu() + 0.05 * torch.randn(H, generator=g)).to(torch.bfloat16)
            sel = mgr.online_expert_ids[j].cpu().clone()
            sel[::3] = torch.randperm(128, generator=g)[:3]
        else:
            x = torch.randn(H, generator=g).to(torch.bfloat16)
            sel = torch.randperm(128, generator=g)[:k]
        vis = torch.tensor(t % 2 == 0)
        outs = [torch.empty(k, dtype=torch.bool, device=dev), torch.empty(1, dtype=torch.long, device=dev),
                torch.empty(k, dtype=torch.bool, device=dev), torch.empty(k, dtype=torch.long, device=dev),
                torch.empty(k, dtype=torch.long, device=dev)]
        eng.search_decode_hybrid_bs1_into(x.to(dev), sel.to(dev), vis.to(dev), 4, *outs)
        torch.cuda.synchronize()
        ref = O.search_hybrid(np64(x)[None], np.array([bool(vis)]),
                              (np64(pca["vision"]["proj"]), np64(pca["vision"]["bias"])),
                              (np64(pca["text"]["proj"]), np64(pca["text"]["bias"])), O.BF16,
                              np64(mgr.keys_buffer), np64(sel)[None], 4, np64(mgr.online_keys),
                              np64(mgr.online_expert_ids), 64)
        assert int(outs[1].item()) == int(ref["on_idx"][0])
        np.testing.assert_array_equal(np64(outs[0]), ref["on_hit"][0])
        np.testing.assert_array_equal(np64(outs[4]), ref["on_slot"][0])
        if near:
            assert np64(outs[0]).any()
        # the offline part on the device's own fused projection (checked against the oracle's)
        reuse = np.zeros((1, k), dtype=bool)
        reuse[0, 4:] = ~ref["on_hit"][0, 4:]
        if reuse.any():
            q = eng.decode_query_workspace[:1]
            abssum = proj_abssum(np64(x)[None], np.array([bool(vis)]), np64(pca["vision"]["proj"]),
                                 np64(pca["text"]["proj"]))
            assert np.all(np.abs(np64(q) - ref["q_low"]) <= ulp(ref["q_low"], torch.bfloat16) + 2.0**-18 * abssum)
            check_gated(q, mgr.keys_buffer, sel.view(1, k).to(dev), vis.view(1).to(dev),
                        torch.from_numpy(reuse).to(dev), outs[2].view(1, k), outs[3].view(1, k), 0.0, 0.0,
                        O.CMP_GE, min_hits=0)
        else:
            assert not np64(outs[2]).any()


def test_modality_mask_on_device_ids(hip_device):
    """ModalityContext with the prompt's ids on the device (as the model's
    generate() leaves them): the mask is computed on the device, equals the
    oracle's closed form, is memoised per (device, seq_len), and a decode
    step (seq_len 1) takes the newest token."""
    from table_moe.utils.modality import ModalityContext

    g = _gen(3)
    ids = torch.randint(0, 152000, (1, 700), generator=g)
    ids[0, 5:600:3] = 151655
    ids[0, 10:20] = 151656
    ids[0, -1] = 151655
    dev = hip_device
    ModalityContext.clear()
    try:
        ModalityContext.set_input_ids(ids.to(dev))
        m = ModalityContext.get_modality_mask(dev, 700)
        assert m.device.type == "cuda" and m.dtype == torch.bool and m.shape == (1, 700)
        np.testing.assert_array_equal(np64(m), O.modality_mask(ids.numpy()))
        assert ModalityContext.get_modality_mask(dev, 700) is m
        last = ModalityContext.get_modality_mask(dev, 1)
        assert last.shape == (1, 1) and bool(last.item())
        np.testing.assert_array_equal(np64(ModalityContext.get_modality_mask(dev, 64)),
                                      O.modality_mask(ids.numpy())[:, -64:])
    finally:
        ModalityContext.clear()


# ------------------------------------------------- segment-grouped edge cases
@pytest.mark.parametrize("dtype,E,K,d,n,k,vis_frac,case", [
    (torch.bfloat16, 16, 100, 64, 300, 8, 0.6, "ragged_table"),   # K not a multiple of 32
    (torch.float16, 8, 1000, 128, 77, 6, 0.5, "big_table"),       # several 32-row blocks per wave
    (torch.bfloat16, 4, 256, 16, 513, 2, 0.0, "text_only_d16"),
    (torch.bfloat16, 128, 256, 256, 33, 8, 1.0, "vision_d256"),
    (torch.bfloat16, 3, 64, 32, 40, 64, 0.5, "top64"),            # 128 tokens per chunk at most
    (torch.bfloat16, 6, 256, 64, 1, 8, 1.0, "one_token"),
    (torch.float16, 2, 256, 64, 2000, 8, 0.5, "dups_and_bad_ids"),  # an expert in several slots of a token
])
def test_gated_segmented_edge_cases(hip_device, dtype, E, K, d, n, k, vis_frac, case):
    g = _gen(E * 7 + K + d + n + k)
    keys = _norm_rows(torch.randn(E, 2, K, d, generator=g)).to(dtype)
    sel = torch.randint(0, E, (n, k), generator=g)
    if case == "dups_and_bad_ids":
        sel[:, 1] = sel[:, 0]
        bad = torch.rand(n, k, generator=g) < 0.1
        sel[bad] = torch.where(torch.rand(int(bad.sum()), generator=g) < 0.5, -3, E + 5)
    vis = torch.rand(n, generator=g) < vis_frac
    reuse = torch.rand(n, k, generator=g) < 0.7
    # queries near table rows of their first slot's expert, so both hits and misses occur
    pick = keys[sel[:, 0].clamp(0, E - 1), (~vis).long(), torch.randint(0, K, (n,), generator=g)].float()
    q = _norm_rows(pick + 0.6 * torch.randn(n, d, generator=g) / d ** 0.5).to(dtype)
    dev = hip_device
    qd, kd, seld, visd, rsd = q.to(dev), keys.to(dev), sel.to(dev), vis.to(dev), reuse.to(dev)
    for col_offset, rs, cmp in ((0, rsd, N.TM_CMP_GE), (3 if k > 3 else 1, None, N.TM_CMP_GT)):
        hit, idx = _gated(dtype, qd, kd, seld, visd, rs, 0.5, 0.55, cmp, col_offset)
        check_gated(qd, kd, seld, visd, rs, hit, idx, 0.5, 0.55, cmp, col_offset=col_offset, min_hits=1)


def test_gated_segmented_repeat_and_graph(hip_device):
    """The grouped kernel keeps no state between calls: two calls and a
    captured graph replayed three times give the same bits."""
    g = _gen(5)
    E, K, d, n, k = 32, 256, 64, 1500, 8
    dev = hip_device
    keys = _norm_rows(torch.randn(E, 2, K, d, generator=g)).to(torch.bfloat16).to(dev)
    q = _norm_rows(torch.randn(n, d, generator=g)).to(torch.bfloat16).to(dev)
    sel = torch.randint(0, E, (n, k), generator=g).to(dev)
    vis = (torch.rand(n, generator=g) < 0.5).to(dev)
    reuse = (torch.rand(n, k, generator=g) < 0.5).to(dev)
    h1, i1 = _gated(torch.bfloat16, q, keys, sel, vis, reuse, 0.1, 0.1, N.TM_CMP_GE)
    h2, i2 = _gated(torch.bfloat16, q, keys, sel, vis, reuse, 0.1, 0.1, N.TM_CMP_GE)
    assert torch.equal(h1, h2) and torch.equal(i1, i2)
    hit = torch.empty(n, k, dtype=torch.uint8, device=dev)
    idx = torch.empty(n, k, dtype=torch.long, device=dev)

    def call():
        N.call("tm_search_gated", N.TM_DT_BF16, q.data_ptr(), n, d, keys.data_ptr(), E, K, d, keys.stride(0),
               keys.stride(1), keys.stride(2), sel.data_ptr(), k, k, 1, N.as_u8(vis).data_ptr(),
               N.as_u8(reuse).data_ptr(), k, 1, 0, 0.1, 0.1, N.TM_CMP_GE, hit.data_ptr(), idx.data_ptr(), k, 1,
               N.stream(dev))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for _ in range(3):
        hit.fill_(7)
        idx.fill_(-7)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(hit, h1) and torch.equal(idx, i1)


# ------------------------------------------------------------ fp32 projection
@pytest.mark.parametrize("dim,layout,n,hidden", [(64, "kmajor", 256, 2048), (32, "rowmajor", 300, 1000),
                                                 (128, "kmajor", 70, 520), (256, "rowmajor", 33, 2048)])
def test_project_f32_tiled_vs_oracle(hip_device, dim, layout, n, hidden):
    """The fp32 projection with a workspace (tiled, split over hidden): mixed
    modalities inside the row tiles, both P layouts, ragged row tiles and k
    chunks; within the fp32 summation bound of the exactly rounded value
    (each output is a sum over one k chunk plus the ordered chunk sums)."""
    g = _gen(dim + n)
    x = torch.randn(n, hidden, generator=g)
    pv, pt = (torch.linalg.qr(torch.randn(hidden, dim, generator=g, dtype=torch.float64))[0].float()
              for _ in range(2))
    bv, bt = torch.randn(dim, generator=g) * 0.1, torch.randn(dim, generator=g) * 0.1
    vis = torch.rand(n, generator=g) < 0.5
    dev = hip_device
    if layout == "kmajor":
        pvd, ptd, ps_h, ps_d = pv.t().contiguous().to(dev), pt.t().contiguous().to(dev), 1, hidden
    else:
        pvd, ptd, ps_h, ps_d = pv.contiguous().to(dev), pt.contiguous().to(dev), dim, 1
    xd, visd, bvd, btd = x.to(dev), vis.to(dev), bv.to(dev), bt.to(dev)  # held: their pointers are passed
    q = torch.empty(n, dim, device=dev)
    qn = torch.empty(n, device=dev)
    nbytes = N.lib().tm_project_workspace_size(n, hidden, dim)
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    for normalize in (0, 1):
        N.call("tm_project", N.TM_DT_F32, xd.data_ptr(), n, hidden, hidden, N.as_u8(visd).data_ptr(),
               pvd.data_ptr(), bvd.data_ptr(), ptd.data_ptr(), btd.data_ptr(), ps_h, ps_d, dim,
               normalize, 1e-6, q.data_ptr(), dim, qn.data_ptr(), ws.data_ptr(), nbytes, N.stream(dev))
        torch.cuda.synchronize()
        raw = O.project_queries(np64(x), vis.numpy(), (np64(pv), np64(bv)), (np64(pt), np64(bt)), False, O.F32)
        abssum = proj_abssum(np64(x), vis.numpy(), np64(pv), np64(pt))
        if normalize:
            ref = O.project_queries(np64(x), vis.numpy(), (np64(pv), np64(bv)), (np64(pt), np64(bt)), True, O.F32)
            abssum = abssum / np.maximum(np.linalg.norm(raw, axis=1, keepdims=True), 1e-6)
        else:
            ref = raw
        bad = np.abs(np64(q) - ref) > 2 * ulp(ref, torch.float32) + 2.0**-14 * abssum
        assert not bad.any(), (normalize, bad.sum())
        np.testing.assert_allclose(np64(qn), (np64(q) ** 2).sum(1), rtol=2e-6, atol=1e-6)
