"""The torch-CPU baseline restatement (oracle/tm_cpu_ref.py) against the numpy
oracle: it is timed as the CPU path beside the GPU, so it must compute the
same layer.  float64 tensors, so the comparison is about the op sequence, not
rounding."""

import numpy as np
import torch

from oracle import tm_cpu_ref as R
from oracle import tm_oracle as O


def _f64(wl):
    return {k: (v.double() if isinstance(v, torch.Tensor) and v.is_floating_point() else v)
            for k, v in wl.__dict__.items()}


def test_layer_forward_g_matches_oracle():
    from synth import make_workload

    for cfg, n, nn in ((1, 64, 1), (3, 32, 4), (2, 300, 1)):
        wl = make_workload(cfg, n=n, n_cent=512, bias_scale=0.2)
        t = _f64(wl)
        got = R.layer_forward_g(t["x"], t["is_vision"], (t["proj_vis"], t["bias_vis"]), (t["proj_txt"], t["bias_txt"]),
                                t["centroids"], t["values"], t["logits"], t["slot_out"], t["residual"],
                                wl.cfg["router_top_k"], nn, 0.6)
        a = lambda v: v.numpy() if isinstance(v, torch.Tensor) else v  # noqa: E731
        ref = O.layer_forward_g(a(t["x"]), a(t["is_vision"]), (a(t["proj_vis"]), a(t["bias_vis"])),
                                (a(t["proj_txt"]), a(t["bias_txt"])), a(t["centroids"]), a(t["values"]),
                                a(t["logits"]), a(t["slot_out"]), a(t["residual"]), wl.cfg["router_top_k"], nn, 0.6,
                                dt=O.F32)
        np.testing.assert_array_equal(got["ids"].numpy(), ref["ids"])
        np.testing.assert_array_equal(got["idx"].numpy(), ref["idx"])
        np.testing.assert_array_equal(got["keep"].numpy(), ref["keep"])
        np.testing.assert_allclose(got["out"].numpy(), ref["out"], rtol=1e-5, atol=1e-5)


def test_recompute_slots_matches_oracle():
    g = torch.Generator().manual_seed(3)
    n, k, e, h, inter = 40, 6, 8, 64, 32
    x = torch.randn(n, h, generator=g, dtype=torch.float64)
    ids = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    keep = torch.rand(n, generator=g) < 0.6
    w1, w3 = (torch.randn(e, inter, h, generator=g, dtype=torch.float64) * 0.1 for _ in range(2))
    w2 = torch.randn(e, h, inter, generator=g, dtype=torch.float64) * 0.1
    slot = torch.full((n, k, h), float("nan"), dtype=torch.float64)
    R.recompute_slots(x, ids, keep, w1, w3, w2, slot)
    for b in range(n):
        for s in range(k):
            if keep[b]:
                want, _ = O.swiglu_expert(x[b:b + 1].numpy(), w1[ids[b, s]].numpy(), w3[ids[b, s]].numpy(),
                                          w2[ids[b, s]].numpy(), O.F32)
                np.testing.assert_allclose(slot[b, s].numpy(), want[0], rtol=1e-5, atol=1e-6)
            else:
                assert torch.isnan(slot[b, s]).all()


def test_prefill_search_r_matches_oracle():
    g = torch.Generator().manual_seed(5)
    n, k, e, kc, d, h = 200, 8, 16, 64, 16, 48
    x = torch.randn(n, h, generator=g, dtype=torch.float64)
    pv, pt = torch.randn(h, d, generator=g, dtype=torch.float64), torch.randn(h, d, generator=g, dtype=torch.float64)
    bv, bt = torch.randn(d, generator=g, dtype=torch.float64), torch.randn(d, generator=g, dtype=torch.float64)
    keys = torch.randn(e, 2, kc, d, generator=g, dtype=torch.float64)
    keys = keys / torch.linalg.vector_norm(keys, dim=-1, keepdim=True)
    sel = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(n)])
    vis = torch.rand(n, generator=g) < 0.7
    reuse = torch.rand(n, k, generator=g) < 0.4
    hit, idx = R.prefill_search_r(x, vis, (pv, bv), (pt, bt), keys, sel, reuse, 0.3, 0.4)
    q = O.project_queries(x.numpy(), vis.numpy(), (pv.numpy(), bv.numpy()), (pt.numpy(), bt.numpy()), False, O.F32)
    q = q / np.linalg.norm(q, axis=1, keepdims=True)
    wh, wi, _, _ = O.search_gated(q, keys.numpy(), sel.numpy(), vis.numpy(), reuse.numpy(), 0.3, 0.4, O.CMP_GE)
    assert 0 < wh.sum() < reuse.sum()
    np.testing.assert_array_equal(hit.numpy(), wh)
    np.testing.assert_array_equal(idx.numpy(), wi)
