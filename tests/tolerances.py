"""Parity tolerances, stated once (north star: fp32 <= 1e-5 relative,
bf16/f16 outputs <= 2e-2 with fp32 accumulation; the reference's own flash
battery uses rtol 1e-4-1e-5 against its f64 oracle,
conformance/test_fusion_triton.py, conformance/test_triton_tile.py)."""

import numpy as np

FP32_RTOL = 1e-5
FP32_ATOL = 1e-6
BF16_TOL = 2e-2


def assert_fp32(got, want, *, rtol=FP32_RTOL, atol=FP32_ATOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol, err_msg=what)


def assert_lowp(got, want, *, tol=BF16_TOL, what=""):
    """bf16 / f16 outputs: max |got - want| <= tol * max(1, max |want|)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    err = np.max(np.abs(got - want)) if got.size else 0.0
    bound = tol * max(1.0, float(np.max(np.abs(want))) if want.size else 1.0)
    assert err <= bound, f"{what}: max abs err {err:.3e} > {bound:.3e}"


def assert_lse(got, want, *, rtol=FP32_RTOL, what=""):
    """fp32 log-sum-exp rows: |got - want| <= rtol * max(1, |want|) per row
    (an lse near zero is held to rtol absolute)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    err = np.abs(got - want)
    bound = rtol * np.maximum(1.0, np.abs(want))
    bad = err > bound
    assert not bad.any(), f"{what}: lse err {err.max():.3e} > {rtol:g} relative (worst at {np.argmax(err - bound)})"
