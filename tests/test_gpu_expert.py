"""GPU parity of the recompute path: the SwiGLU expert MLP (tm_expert_swiglu),
the device-side grouping of recomputed slots by expert (tm_group_slots) and
the grouped MLP writing the slot layout (tm_grouped_swiglu), against the
oracle (oracle/tm_oracle.py: swiglu_expert, grouped_swiglu)."""

import numpy as np
import pytest
import torch

from oracle import tm_oracle as O
from parity_util import ODT, np64
from table_moe import _native as N

pytestmark = pytest.mark.gpu


def _weights(g, e, h, inter, dtype, scale=0.02):
    w1 = (torch.randn(e, inter, h, generator=g) * scale).to(dtype)
    w3 = (torch.randn(e, inter, h, generator=g) * scale).to(dtype)
    w2 = (torch.randn(e, h, inter, generator=g) * scale).to(dtype)
    return w1, w3, w2


def assert_mlp_close(got, exact, dtype, min_exact=0.9):
    """North-star tolerance (atol 1e-2, rtol 2e-3) where it exceeds the
    type's own half-ulp, plus a floor on the bit-exact fraction: the device
    accumulates in fp32 (the intermediate can round the other way where an
    exact value sits on a rounding boundary)."""
    got, exact = np.asarray(got), np.asarray(exact)
    small = np.abs(exact) < 8.0
    np.testing.assert_allclose(got[small], exact[small], atol=1e-2, rtol=2e-3)
    frac = float(np.mean(got == exact))
    assert frac >= min_exact, f"only {frac:.4f} bit-exact"


@pytest.mark.parametrize("m,h,inter,dtype", [(1, 2048, 768, torch.bfloat16), (7, 2560, 1536, torch.float16),
                                             (128, 1024, 512, torch.bfloat16), (300, 2560, 1536, torch.bfloat16),
                                             (129, 256, 128, torch.float16)])
def test_expert_swiglu_vs_oracle(hip_device, m, h, inter, dtype):
    from table_moe.ops import expert_swiglu

    g = torch.Generator().manual_seed(m + h + inter)
    x = torch.randn(m, h, generator=g).to(dtype)
    w1, w3, w2 = (w[0] for w in _weights(g, 1, h, inter, dtype))
    y = expert_swiglu(x.to(hip_device), w1.to(hip_device), w3.to(hip_device), w2.to(hip_device))
    torch.cuda.synchronize()
    want, _ = O.swiglu_expert(np64(x), np64(w1), np64(w3), np64(w2), ODT[dtype])
    assert_mlp_close(np64(y), want, dtype)


@pytest.mark.parametrize("n,k", [(1000, 6), (4096, 8), (5000, 8), (300, 10)])
def test_group_slots_buckets_every_pair(hip_device, n, k):
    """Counts, offsets, tiles and the (token, slot) -> row map of the device
    grouping against a host bincount; every selected pair appears once (the
    register path up to 4096 tokens x 8 slots, the looped path beyond)."""
    from table_moe.ops import GroupedExperts

    dev = hip_device
    g = torch.Generator().manual_seed(11 + n + k)
    e, h = 64, 128
    ids = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    ids[5, 2] = -1  # out-of-range ids are skipped
    ids[6, 0] = e
    keep = torch.rand(n, generator=g) < 0.6
    w = torch.zeros(e, 128, h, dtype=torch.bfloat16, device=dev)
    ge = GroupedExperts(w, w.clone(), torch.zeros(e, h, 128, dtype=torch.bfloat16, device=dev))
    slot_out = torch.empty(n, k, h, dtype=torch.bfloat16, device=dev)
    offs, row_token, row_out, tiles = ge.group(ids.to(dev), keep.to(dev), slot_out)
    torch.cuda.synchronize()
    sel = keep[:, None].expand(n, k) & (ids >= 0) & (ids < e)
    counts = np.bincount(ids[sel].numpy(), minlength=e)
    offs = offs.cpu().numpy()
    np.testing.assert_array_equal(np.diff(offs[: e + 1]), counts)
    total = int(counts.sum())
    tiles = tiles.cpu().numpy()
    assert tiles[0] == total
    t_max = N.lib().tm_group_slots_tiles(n * k, e)
    n_tiles = int(tiles[1])
    rows_per_tile = 256  # tile height of the grouped GEMM
    assert n_tiles == int(np.sum((counts + rows_per_tile - 1) // rows_per_tile)) <= t_max
    te, tr = tiles[2: 2 + n_tiles], tiles[2 + t_max: 2 + t_max + n_tiles]
    for ex in range(e):
        rows = tr[te == ex]
        np.testing.assert_array_equal(rows, offs[ex] + rows_per_tile * np.arange(len(rows)))
    rt = row_token[:total].cpu().numpy()
    ro = row_out[:total].cpu().numpy()
    b_of, s_of = ro // slot_out.stride(0), (ro % slot_out.stride(0)) // slot_out.stride(1)
    np.testing.assert_array_equal(b_of, rt)
    pairs = set(zip(b_of.tolist(), s_of.tolist()))
    assert len(pairs) == total
    want = set(zip(*[a.tolist() for a in np.nonzero(sel.numpy())]))
    assert pairs == want
    for ex in range(e):  # each row sits in its expert's range
        bb, ss = b_of[offs[ex]: offs[ex + 1]], s_of[offs[ex]: offs[ex + 1]]
        assert np.all(ids.numpy()[bb, ss] == ex)


@pytest.mark.parametrize("n,k,e,per_slot", [(4096, 6, 64, False), (8192, 8, 256, True), (37, 6, 64, True),
                                             (64, 8, 5, False), (8193, 6, 64, False)])
def test_group_slots_ws_matches_one_workgroup(hip_device, n, k, e, per_slot):
    """tm_group_slots_ws (per-workgroup counts, then placement) against the
    one-workgroup tm_group_slots on the same ids and mask: the same offsets
    and tile list, and the same set of (token, slot) rows in each expert's
    range (the order inside an expert is unspecified), ids out of range
    skipped; 8193 tokens are past the multi-workgroup limit and take the
    one-workgroup kernel."""
    dev = hip_device
    g = torch.Generator().manual_seed(41 + n + e)
    ids = torch.randint(0, e, (n, k), generator=g)
    ids[3 % n, 1] = -1
    ids[5 % n, 0] = e
    mask = (torch.rand(n, k, generator=g) < 0.6) if per_slot else (torch.rand(n, generator=g) < 0.6)
    ids, m = ids.to(dev), mask.to(torch.uint8).to(dev)
    ms_b, ms_s = (k, 1) if per_slot else (1, 0)
    h = 128
    so_b, so_s = k * h, h
    t_max = N.lib().tm_group_slots_tiles(n * k, e)
    nbytes = N.lib().tm_group_slots_workspace_size(n, k, e)
    assert (nbytes > 0) == (n <= 8192)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
    outs = []
    for multi in (False, True):
        offs = torch.full((e + 1,), -7, dtype=torch.int32, device=dev)
        tiles = torch.full((2 + 2 * t_max,), -7, dtype=torch.int32, device=dev)
        rt = torch.full((n * k,), -7, dtype=torch.int32, device=dev)
        ro = torch.full((n * k,), -7, dtype=torch.int64, device=dev)
        args = (N.ptr(ids), n, k, k, N.ptr(m), ms_b, ms_s, e, so_b, so_s, N.ptr(offs), N.ptr(rt), N.ptr(ro),
                N.ptr(tiles))
        if multi:
            N.call("tm_group_slots_ws", *args, N.ptr(ws), ws.numel(), N.stream(dev))
        else:
            N.call("tm_group_slots", *args, N.stream(dev))
        torch.cuda.synchronize()
        outs.append((offs.cpu().numpy(), tiles.cpu().numpy(), rt.cpu().numpy(), ro.cpu().numpy()))
    (o1, t1, rt1, ro1), (o2, t2, rt2, ro2) = outs
    np.testing.assert_array_equal(o1, o2)
    total, n_tiles = int(t1[0]), int(t1[1])
    assert total == int(o1[e]) and total > 0
    np.testing.assert_array_equal(t1[:2 + n_tiles], t2[:2 + n_tiles])
    np.testing.assert_array_equal(t1[2 + t_max:2 + t_max + n_tiles], t2[2 + t_max:2 + t_max + n_tiles])
    np.testing.assert_array_equal(rt2[:total], ro2[:total] // so_b)
    for ex in range(e):
        a, z = int(o1[ex]), int(o1[ex + 1])
        assert sorted(ro1[a:z].tolist()) == sorted(ro2[a:z].tolist()), ex
    # every selected pair once, in its expert's range
    sel = (mask[:, None].expand(n, k) if not per_slot else mask) & (ids.cpu() >= 0) & (ids.cpu() < e)
    assert total == int(sel.sum())


def test_group_slots_empty_batch(hip_device):
    """An empty recompute batch (no tokens, null id/mask pointers) groups
    nothing: zero offsets and a zero row/tile count, and the grouped MLP after
    it is a no-op; the offsets/tiles buffers start non-zero so the kernel's
    writes are what the test sees."""
    from table_moe.ops import GroupedExperts

    dev = hip_device
    e, h, k = 64, 128, 6
    w = torch.zeros(e, 128, h, dtype=torch.bfloat16, device=dev)
    ge = GroupedExperts(w, w.clone(), torch.zeros(e, h, 128, dtype=torch.bfloat16, device=dev))
    ids = torch.empty(0, k, dtype=torch.long, device=dev)
    keep = torch.empty(0, dtype=torch.bool, device=dev)
    slot_out = torch.empty(0, k, h, dtype=torch.bfloat16, device=dev)
    t_max = N.lib().tm_group_slots_tiles(0, e)
    offs = torch.full((e + 1,), 7, dtype=torch.int32, device=dev)
    tiles = torch.full((2 + 2 * t_max,), 7, dtype=torch.int32, device=dev)
    N.call("tm_group_slots", None, 0, k, k, None, 1, 0, e, k * h, h, N.ptr(offs), None, None, N.ptr(tiles),
           N.stream(dev))
    torch.cuda.synchronize()
    assert (offs.cpu() == 0).all()
    assert tiles[0].item() == 0 and tiles[1].item() == 0
    out = ge.forward(torch.empty(0, h, dtype=torch.bfloat16, device=dev), ids, keep, slot_out)
    torch.cuda.synchronize()
    assert out.shape == (0, k, h)


def test_grouped_forward_rejects_misaligned_slot_rows(hip_device):
    """Grouped rows are written in 16-byte pieces: a slot_out view whose rows
    do not start on 16-byte boundaries (stride hidden + 4) is rejected before
    any launch, by GroupedExperts.forward and by tm_group_slots itself."""
    from table_moe.ops import GroupedExperts

    dev = hip_device
    e, h, k, n = 8, 128, 6, 4
    w = torch.zeros(e, 128, h, dtype=torch.bfloat16, device=dev)
    ge = GroupedExperts(w, w.clone(), torch.zeros(e, h, 128, dtype=torch.bfloat16, device=dev))
    ids = torch.zeros(n, k, dtype=torch.long, device=dev)
    keep = torch.ones(n, dtype=torch.bool, device=dev)
    hidden = torch.zeros(n, h, dtype=torch.bfloat16, device=dev)
    wide = torch.zeros(n, k, h + 4, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="16-byte"):
        ge.forward(hidden, ids, keep, wide[..., :h])
    t_max = N.lib().tm_group_slots_tiles(n * k, e)
    offs = torch.zeros(e + 1, dtype=torch.int32, device=dev)
    tiles = torch.zeros(2 + 2 * t_max, dtype=torch.int32, device=dev)
    rows = torch.zeros(n * k, dtype=torch.int32, device=dev)
    outs = torch.zeros(n * k, dtype=torch.long, device=dev)
    st = N.lib().tm_group_slots(N.ptr(ids), n, k, k, N.ptr(keep), 1, 0, e, k * (h + 4), h + 4, N.ptr(offs),
                                N.ptr(rows), N.ptr(outs), N.ptr(tiles), N.stream(dev))
    assert st == N.TM_EINVAL_SHAPE
    out = ge.forward(hidden, ids, keep, wide[..., :h].contiguous())  # aligned copy: accepted
    torch.cuda.synchronize()
    assert out.shape == (n, k, h)


@pytest.mark.parametrize("mask_kind", ["token", "slot"])
def test_grouped_swiglu_vs_oracle_and_single_expert(hip_device, mask_kind):
    """Config-5 shapes (64 experts, top-6, hidden 2560, intermediate 1536) on
    300 tokens: every selected slot row against the oracle; unselected slots
    untouched; and each expert's rows bit-identical to tm_expert_swiglu on the
    same rows (an output row does not depend on where it sits in a tile)."""
    from table_moe.ops import GroupedExperts, expert_swiglu

    dev = hip_device
    g = torch.Generator().manual_seed(17 if mask_kind == "token" else 19)
    n, k, e, h, inter, dtype = 300, 6, 64, 2560, 1536, torch.bfloat16
    x = torch.randn(n, h, generator=g).to(dtype)
    w1, w3, w2 = _weights(g, e, h, inter, dtype)
    ids = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    mask = (torch.rand(n, generator=g) < 0.6) if mask_kind == "token" else (torch.rand(n, k, generator=g) < 0.5)
    ge = GroupedExperts(w1.to(dev), w3.to(dev), w2.to(dev))
    slot_out = torch.full((n, k, h), 7.0, dtype=dtype, device=dev)
    ge.forward(x.to(dev), ids.to(dev), mask.to(dev), slot_out)
    torch.cuda.synchronize()
    got = np64(slot_out)
    want = O.grouped_swiglu(np64(x), ids.numpy(), mask.numpy(), np64(w1), np64(w3), np64(w2), O.BF16)
    m2 = mask.numpy() if mask.dim() == 2 else np.repeat(mask.numpy()[:, None], k, axis=1)
    assert np.all(got[~m2] == 7.0)
    assert_mlp_close(got[m2], want[m2], dtype)
    xd = x.to(dev)
    for ex in (0, 17, 63):
        bb, ss = np.nonzero(m2 & (ids.numpy() == ex))
        if len(bb) == 0:
            continue
        y = expert_swiglu(xd[torch.from_numpy(bb).to(dev)].contiguous(), ge.w1[ex], ge.w3[ex], ge.w2[ex])
        torch.cuda.synchronize()
        assert torch.equal(y, slot_out[torch.from_numpy(bb).to(dev), torch.from_numpy(ss).to(dev)])


def test_maybe_run_fp16_fused_expert_contract(hip_device, monkeypatch):
    """The reference's entry point: None when it does not apply (more rows than
    TABLEMOE_FP16_FUSED_MAX_TOKENS, default 1; disabled by
    TABLEMOE_USE_FP16_FUSED_EXPERT=0; a bias), else the MLP in the owner's
    reused output buffer."""
    from table_moe.ops import expert_swiglu, maybe_run_fp16_fused_expert

    dev = hip_device
    h, inter = 512, 256

    class Wrap:
        def __init__(self, lin):
            self.linear_module = lin

    class Owner:
        pass

    torch.manual_seed(3)
    owner = Owner()
    owner.w1 = Wrap(torch.nn.Linear(h, inter, bias=False).to(dev, torch.float16))
    owner.w3 = Wrap(torch.nn.Linear(h, inter, bias=False).to(dev, torch.float16))
    owner.w2 = Wrap(torch.nn.Linear(inter, h, bias=False).to(dev, torch.float16))
    x1 = torch.randn(1, h, device=dev, dtype=torch.float16)
    y = maybe_run_fp16_fused_expert(owner, x1)
    ref = expert_swiglu(x1, owner.w1.linear_module.weight, owner.w3.linear_module.weight, owner.w2.linear_module.weight)
    torch.cuda.synchronize()
    assert y is not None and torch.equal(y, ref)
    assert maybe_run_fp16_fused_expert(owner, x1) is y  # the owner's buffer is reused
    x3 = torch.randn(3, h, device=dev, dtype=torch.float16)
    assert maybe_run_fp16_fused_expert(owner, x3) is None
    monkeypatch.setenv("TABLEMOE_FP16_FUSED_MAX_TOKENS", "4")
    assert maybe_run_fp16_fused_expert(owner, x3) is not None
    monkeypatch.setenv("TABLEMOE_USE_FP16_FUSED_EXPERT", "0")
    assert maybe_run_fp16_fused_expert(owner, x1) is None
    monkeypatch.delenv("TABLEMOE_USE_FP16_FUSED_EXPERT")
    owner.w2 = Wrap(torch.nn.Linear(inter, h, bias=True).to(dev, torch.float16))
    assert maybe_run_fp16_fused_expert(owner, x1) is None


def _pack_reference(w, bn):
    """The packed layout restated on the host: tile t of bn rows, stage kt of
    32 columns is one block of bn x 32 elements; its 16-byte slot p holds
    row p // 4, 8-column chunk (p % 4) ^ ((row // 4) % 4) of the stage."""
    e, rows, k = w.shape
    src = w.reshape(e * rows // bn, bn, k // 32, 4, 8)  # [tile, row, stage, chunk, 8]
    p = np.arange(bn * 4)
    row, kc = p // 4, (p % 4) ^ ((p // 4 // 4) % 4)
    out = src[:, row, :, kc, :]  # [slot, tile, stage, 8]: the indexed axes come first
    return np.ascontiguousarray(out.transpose(1, 2, 0, 3)).reshape(w.shape)


@pytest.mark.parametrize("h,inter", [(2560, 1536), (384, 256)])
def test_pack_weights_layout(hip_device, h, inter):
    """tm_expert_pack_weights against the host restatement of the layout:
    gate/up weights in 128-row tiles, down weights in 256-row tiles when
    hidden is a multiple of 256 (else 128), each 32-column stage of a tile
    one contiguous block in the GEMM's LDS slot order."""
    dev = hip_device
    g = torch.Generator().manual_seed(23)
    e = 3
    w13 = torch.arange(e * inter * h, dtype=torch.int32).reshape(e, inter, h)
    w2 = torch.randint(-30000, 30000, (e, h, inter), generator=g, dtype=torch.int32)
    for w, role, bn in ((w13, N.TM_PACK_GATE_UP, 128), (w2, N.TM_PACK_DOWN, 256 if h % 256 == 0 else 128)):
        src = w.to(torch.int16).view(torch.bfloat16).to(dev)
        out = torch.empty_like(src)
        N.call("tm_expert_pack_weights", N.TM_DT_BF16, N.ptr(src), e, h, inter, role, N.ptr(out), N.stream(dev))
        torch.cuda.synchronize()
        want = _pack_reference(src.view(torch.int16).cpu().numpy(), bn)
        np.testing.assert_array_equal(out.view(torch.int16).cpu().numpy(), want)


@pytest.mark.parametrize("n,k,e,h,inter,dtype", [(2048, 6, 64, 2560, 1536, torch.bfloat16),
                                                 (700, 8, 16, 384, 256, torch.float16)])
def test_grouped_swiglu_packed_equals_plain(hip_device, n, k, e, h, inter, dtype):
    """Config-5 shapes on 2048 tokens (experts with more than one 256-row
    tile), and fp16 with a hidden size that takes 128-column down tiles: the
    packed-weight GEMMs write the same slot rows, bit for bit, as the
    plain-layout ones."""
    from table_moe.ops import GroupedExperts

    dev = hip_device
    g = torch.Generator().manual_seed(29 + n)
    x = torch.randn(n, h, generator=g).to(dtype).to(dev)
    w1, w3, w2 = (w.to(dev) for w in _weights(g, e, h, inter, dtype))
    ids = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)]).to(dev)
    mask = (torch.rand(n, k, generator=g) < 0.7).to(dev)
    packed, plain = GroupedExperts(w1, w3, w2), GroupedExperts(w1, w3, w2, packed=False)
    assert packed.packed is not None and plain.packed is None
    a = torch.full((n, k, h), 3.0, dtype=dtype, device=dev)
    b = torch.full((n, k, h), 3.0, dtype=dtype, device=dev)
    for _ in range(2):
        packed.forward(x, ids, mask, a)
        plain.forward(x, ids, mask, b)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert float((a != 3.0).float().mean()) > 0.5


@pytest.mark.parametrize("m,addend,dtype", [(300, True, torch.bfloat16), (4096, True, torch.bfloat16),
                                            (129, False, torch.bfloat16), (257, True, torch.float16)])
def test_shared_experts_packed_equals_plain(hip_device, m, addend, dtype):
    """SharedExperts (one expert's packed weights, tm_expert_swiglu_packed)
    against expert_swiglu on the plain weights: the same rows bit for bit, at
    the config-5 shared shape (intermediate 3072, hidden 2560), with and
    without the residual addend, partial last tiles included."""
    from table_moe.ops import SharedExperts, expert_swiglu

    dev = hip_device
    g = torch.Generator().manual_seed(31 + m)
    h, inter = 2560, 3072
    x = torch.randn(m, h, generator=g).to(dtype).to(dev)
    w1, w3, w2 = (w[0].to(dev) for w in _weights(g, 1, h, inter, dtype))
    add = torch.randn(m, h, generator=g).to(dtype).to(dev) if addend else None
    sh = SharedExperts(w1, w3, w2)
    got = sh.forward(x, addend=add)
    want = expert_swiglu(x, w1, w3, w2, addend=add)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
