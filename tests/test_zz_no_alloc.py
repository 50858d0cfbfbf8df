"""tm_table_forward_noalloc (the layer call on the library's static scratch)
against tm_table_forward (caller workspace): identical bits on calls in a row
that take different plans over the one shared scratch, the second call
smaller than the first; a layer whose workspace exceeds the scratch is
rejected before any launch."""

import ctypes as C

import pytest
import torch

from table_moe import _native as N

KEYS = ("weights", "ids", "q", "qn", "dist", "idx", "keep", "out")


def _tables(d, metric="l2"):
    from table_moe.cache_engine import GlobalTable

    mk = lambda: GlobalTable(d.centroids, d.values, (d.proj_vis, d.bias_vis), (d.proj_txt, d.bias_txt),  # noqa: E731
                             metric=metric)
    return mk(), mk()


@pytest.mark.gpu
def test_noalloc_matches_workspace_call(hip_device):
    from synth import make_workload

    dev = hip_device
    # ranked top-1 plan (n = 4096, arrival counters per query tile), then the
    # decode plan (n = 32, top-4, arrival counters per projection group), then
    # the fused top-1 plan with a keep-select launch, then the ranked plan again
    cases = [(2, 4096, 1), (3, 32, 4), (2, 1000, 1), (2, 4096, 1)]
    for cfg, n, nn in cases:
        print(f"[noalloc] config {cfg} n={n} n_nearest={nn}", flush=True)
        d = make_workload(cfg, n=n).to(dev)
        a, b = _tables(d)
        topk = d.cfg["router_top_k"]
        ra = a.layer_forward(d.x, d.is_vision, d.logits, d.slot_out, d.residual, topk, nn, 0.6)
        rb = b.layer_forward_noalloc(d.x, d.is_vision, d.logits, d.slot_out, d.residual, topk, nn, 0.6)
        torch.cuda.synchronize()
        for key in KEYS:
            assert torch.equal(ra[key], rb[key]), (cfg, n, key)
        assert int(rb["keep"].sum()) == b.keep_count(n, 0.6)
        assert a.wait_errors() == 0, (cfg, n)


@pytest.mark.gpu
def test_noalloc_rejects_oversized_layer(hip_device):
    """n = 4096 with top-8 search lists needs 16.4 MiB of workspace: rejected
    with TM_EWORKSPACE (ValueError), and the scratch is left usable."""
    from synth import make_workload

    dev = hip_device
    d = make_workload(2, n=4096).to(dev)
    a, b = _tables(d)
    need = N.lib().tm_table_forward_workspace_size(C.byref(b._desc), 4096, 8)
    assert need > N.TM_NOALLOC_SCRATCH_BYTES
    with pytest.raises(ValueError, match="TM_EWORKSPACE"):
        b.layer_forward_noalloc(d.x, d.is_vision, d.logits, d.slot_out, d.residual, 8, 8, 0.6)
    ra = a.layer_forward(d.x, d.is_vision, d.logits, d.slot_out, d.residual, 8, 1, 0.6)
    rb = b.layer_forward_noalloc(d.x, d.is_vision, d.logits, d.slot_out, d.residual, 8, 1, 0.6)
    torch.cuda.synchronize()
    for key in KEYS:
        assert torch.equal(ra[key], rb[key]), key
