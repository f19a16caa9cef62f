"""The certification gate compares draws inside the operators' domains only.

The reference's differential tier (packages/tensorlib/src/pdum/tl/certify.py:
240-282) compares with numpy's default equal_nan=True, so a tile / naive pair
that both produce NaN on a draw "agree" there. Here a family whose draw makes
either side non-finite (or raises an overflow / invalid operation) is refused,
and the contraction families draw the arguments of sqrt and log positive."""

import numpy as np
import pytest

from pdum_dsl_amd.tl import fusion
from pdum_dsl_amd.tl.certify import certify
from pdum_dsl_amd.tl.dialect import OPS
from pdum_dsl_amd.tl.interp import field, run_region
from pdum_dsl_amd.tl.ir import F64, Builder, Region, tensor_type
from pdum_dsl_amd.tl.licenses import GEMM_K_REASSOC


def _sqrt_pair():
    """naive: sqrt(x); tile: sqrt(x) * 1 (another content key, the same values)."""
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t",), (16,)))
    naive = Region(params=(x,), body=(b.emit("core.yield", b.emit("tl.pointwise", x, f="sqrt")),))
    b2 = Builder(OPS)
    x2 = b2.param(0, tensor_type(("t",), (16,)))
    one = b2.emit("core.const", type=F64, value=1.0)
    y = b2.emit("tl.pointwise", b2.emit("tl.pointwise", x2, f="sqrt"), one, f="mul")
    tile = Region(params=(x2,), body=(b2.emit("core.yield", y),))
    return tile, naive


def test_a_pair_that_agrees_only_on_nan_is_refused():
    tile, naive = _sqrt_pair()
    negative = (("negative", lambda: [field(-np.arange(1.0, 17.0), ("t",))]),)
    with pytest.raises(ValueError, match="left the operators' domain"):
        certify(tile, naive, licenses=GEMM_K_REASSOC, families=negative)


def test_the_same_pair_certifies_inside_its_domain():
    tile, naive = _sqrt_pair()
    positive = (("positive", lambda: [field(np.arange(1.0, 17.0), ("t",))]),)
    c = certify(tile, naive, licenses=GEMM_K_REASSOC, families=positive)
    assert c.verdict == "licensed-differential" and c.families == ("positive",)


def test_an_overflowing_draw_is_refused():
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t",), (4,)))
    naive = Region(params=(x,), body=(b.emit("core.yield", b.emit("tl.pointwise", x, f="exp")),))
    b2 = Builder(OPS)
    x2 = b2.param(0, tensor_type(("t",), (4,)))
    y = b2.emit("tl.pointwise", b2.emit("tl.pointwise", x2, f="exp"), b2.emit("core.const", type=F64, value=1.0),
                f="mul")
    tile = Region(params=(x2,), body=(b2.emit("core.yield", y),))
    wide = (("wide", lambda: [field(np.array([1.0, 2.0, 800.0, 3.0]), ("t",))]),)  # exp(800) overflows
    with pytest.raises(ValueError, match="left the operators' domain"):
        certify(tile, naive, licenses=GEMM_K_REASSOC, families=wide)


def _rms_region():
    """y[t] = sqrt(sum_e x[t, e] * w[e]) + b[t]: x and w reach the sqrt, b does not."""
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "e"), (3, 5)))
    w = b.param(1, tensor_type(("e",), (5,)))
    bias = b.param(2, tensor_type(("t",), (3,)))
    prod = b.emit("tl.pointwise", x, b.emit("tl.repeat_like", w, x), f="mul")
    s = b.emit("tl.reduce", prod, dims=("e",), f="sum")
    y = b.emit("tl.pointwise", b.emit("tl.pointwise", s, f="sqrt"), bias, f="add")
    return Region(params=(x, w, bias), body=(b.emit("core.yield", y),))


def test_the_params_reaching_sqrt_are_found():
    assert fusion.domain_restricted_params(_rms_region()) == frozenset({0, 1})


def test_contraction_families_stay_inside_the_domain():
    region = _rms_region()
    for name, factory in fusion.contraction_families(region):
        vals = factory()
        assert (vals[0].arr > 0).all() and (vals[1].arr > 0).all(), name
        assert (vals[2].arr < 0).any(), f"{name}: a param that reaches no sqrt keeps its sign"
        with np.errstate(over="raise", invalid="raise", divide="raise"):
            out = run_region(region, vals)
        assert np.isfinite(out.arr).all()


def _rmsnorm_region():
    """y[t] = sum_e x[t, e] w[e] / sqrt(sum_e x[t, e]^2 + 1): x reaches the sqrt,
    but through a square: its argument is positive whatever x's sign."""
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "e"), (3, 5)))
    w = b.param(1, tensor_type(("e",), (5,)))
    prod = b.emit("tl.pointwise", x, b.emit("tl.repeat_like", w, x), f="mul")
    s = b.emit("tl.reduce", prod, dims=("e",), f="sum")
    sq = b.emit("tl.reduce", b.emit("tl.pointwise", x, x, f="mul"), dims=("e",), f="sum")
    one = b.emit("core.const", type=F64, value=1.0)
    den = b.emit("tl.pointwise", b.emit("tl.pointwise", sq, one, f="add"), f="sqrt")
    y = b.emit("tl.pointwise", s, den, f="div")
    return Region(params=(x, w), body=(b.emit("core.yield", y),))


def test_params_reaching_a_sqrt_of_squares_keep_signed_draws():
    """Signed first: a param is drawn positive only when a signed draw leaves
    the domain, so an RMS-norm input keeps its sign cancellations."""
    region = _rmsnorm_region()
    assert fusion.domain_restricted_params(region) == frozenset({0})
    for name, factory in fusion.contraction_families(region):
        vals = factory()
        assert (vals[0].arr < 0).any() and (vals[1].arr < 0).any(), name
