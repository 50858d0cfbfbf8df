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
