"""Tolerance checks shared by the parity tests.

The bar for fp16 outputs is max-abs error <= 2e-3 against the fp64 oracle; for lse it is the
reference's rule |got - ref| <= 1e-4 + 1e-4 |ref| (01_decode_attention.cu:776 with
common/bench.cuh:197-225), with -inf required exactly where the oracle has -inf.
"""
import numpy as np

OUT_ATOL = 2e-3
LSE_ATOL = 1e-4
LSE_RTOL = 1e-4


def check_out(got, ref, atol=OUT_ATOL, tag=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (tag, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{tag}: non-finite output"
    err = np.abs(got - ref)
    mx = float(err.max()) if err.size else 0.0
    assert mx <= atol, f"{tag}: out max_abs {mx:.3e} > {atol:.1e} at {np.unravel_index(err.argmax(), err.shape)}"
    return mx


def check_lse(got, ref, atol=LSE_ATOL, rtol=LSE_RTOL, tag=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (tag, got.shape, ref.shape)
    ninf_ref = np.isneginf(ref)
    assert np.array_equal(np.isneginf(got), ninf_ref), f"{tag}: -inf pattern differs"
    fin = ~ninf_ref
    if not fin.any():
        return 0.0
    assert np.all(np.isfinite(got[fin])), f"{tag}: non-finite lse"
    err = np.abs(got[fin] - ref[fin])
    lim = atol + rtol * np.abs(ref[fin])
    assert np.all(err <= lim), f"{tag}: lse max_abs {err.max():.3e} (limit {lim[err.argmax()]:.3e})"
    return float(err.max())
