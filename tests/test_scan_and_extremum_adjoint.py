"""tl.scan and the first-occurrence max / min adjoint (CPU).

tl.scan is the reference's inclusive prefix reduce along one dim
(packages/tensorlib/src/pdum/tl/compute.py:318-350: ufunc accumulate; a mean
divides by the running count). ``grad`` sends a max / min reduction's
cotangent to the FIRST position attaining the extremum along each reduced dim,
through a prefix count of the hits (autodiff.py:635-665); a scan sum's adjoint
is the suffix sum of the cotangent (autodiff.py:667-677).

Pins, each independent of the rule's own formula:
  * both interpreters (the planner's numpy one, the oracle's torch-f64 one)
    against numpy's ufunc.accumulate, NaN included;
  * the tie-broken gradient against a brute-force first-index loop and
    against torch's max(dim) / min(dim) backward (which scatters into the
    first index its forward returns), on inputs drawn with many ties;
  * a multi-dim max against the brute-force flat first index in C order of
    the reduced dims, as the dim-by-dim rule implies;
  * the scan-sum adjoint against central finite differences."""

import numpy as np
import pytest
import torch

from oracle import region_eval as rev
from pdum_dsl_amd.tl import interp
from pdum_dsl_amd.tl.autodiff import grad, region_names
from pdum_dsl_amd.tl.dialect import OPS
from pdum_dsl_amd.tl.ir import Builder, Region, tensor_type

_ACC = {"sum": np.add, "prod": np.multiply, "max": np.maximum, "min": np.minimum}


def _scan_region(shape, names, dim, f, reverse=False):
    b = Builder(OPS)
    x = b.param(0, tensor_type(names, shape))
    extra = {"reverse": True} if reverse else {}
    y = b.emit("tl.scan", x, dim=dim, f=f, **extra)
    return Region(params=(x,), body=(b.emit("core.yield", y),))


def _numpy_scan(arr, axis, f, reverse):
    a = np.flip(arr, axis) if reverse else arr
    out = (np.add if f == "mean" else _ACC[f]).accumulate(a, axis=axis)
    if f == "mean":
        shape = [1] * a.ndim
        shape[axis] = a.shape[axis]
        out = out / np.arange(1, a.shape[axis] + 1).reshape(shape)
    return np.flip(out, axis) if reverse else out


@pytest.mark.parametrize("f", ["sum", "prod", "max", "min", "mean"])
@pytest.mark.parametrize("dim,reverse", [("s", False), ("t", False), ("s", True)])
def test_scan_on_both_interpreters_is_ufunc_accumulate(f, dim, reverse):
    rng = np.random.default_rng(1)
    arr = rng.standard_normal((4, 7))
    arr[2, 3] = np.nan  # a NaN poisons the rest of its prefix (suffix) for every reducer
    region = _scan_region(arr.shape, ("t", "s"), dim, f, reverse)
    want = _numpy_scan(arr, ("t", "s").index(dim), f, reverse)
    got = interp.run_region(region, [interp.field(arr, ("t", "s"))]).to_numpy(("t", "s"))
    np.testing.assert_allclose(got, want, rtol=1e-12, equal_nan=True)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    got2 = rev.evaluate(region, [rev.value(arr, region.params[0].type)]).numpy(("t", "s"))
    np.testing.assert_allclose(got2, want, rtol=1e-12, equal_nan=True)
    assert np.array_equal(np.isnan(got2), np.isnan(want))


def _extremum_joint(shape, names, dims, f):
    b = Builder(OPS)
    x = b.param(0, tensor_type(names, shape))
    y = b.emit("tl.reduce", x, dims=dims, f=f)
    region = Region(params=(x,), body=(b.emit("core.yield", y),))
    rg = grad(region, "out", seed="dy", wrt=("x",), names=region_names(region, ("x",), ("out",)))
    return region, y, rg


def _eval_joint(rg, y, xv, dy, names):
    """The joint's dx on both interpreters (x in ``names`` order, dy in y's)."""
    res = interp.run_region(rg.region, [interp.field(xv, names), interp.field(dy, y.type.names)])
    g1 = res[1].to_numpy(names)
    vals = [rev.value(xv, rg.region.params[0].type), rev.value(dy, rg.region.params[1].type)]
    g2 = rev.evaluate(rg.region, vals)[1].numpy(names)
    return g1, g2


@pytest.mark.parametrize("f", ["max", "min"])
def test_a_tied_extremum_sends_its_cotangent_to_the_first_position(f):
    rng = np.random.default_rng(5)
    xv = rng.integers(0, 3, size=(6, 9)).astype(np.float64)  # values 0..2: ties in almost every row
    region, y, rg = _extremum_joint(xv.shape, ("t", "s"), ("s",), f)
    dy = rng.standard_normal(6)
    g1, g2 = _eval_joint(rg, y, xv, dy, ("t", "s"))
    # brute force: the first index attaining the row's extremum takes dy
    want = np.zeros_like(xv)
    for t in range(6):
        ext = xv[t].max() if f == "max" else xv[t].min()
        want[t, int(np.flatnonzero(xv[t] == ext)[0])] = dy[t]
    assert (np.sum(xv == (xv.max(1) if f == "max" else xv.min(1))[:, None], axis=1) > 1).any(), "no ties drawn"
    np.testing.assert_array_equal(g1, want)
    np.testing.assert_array_equal(g2, want)
    # torch's max(dim) / min(dim) backward scatters into the first index its forward returns
    xt = torch.tensor(xv, requires_grad=True)
    (xt.max(dim=1) if f == "max" else xt.min(dim=1)).values.backward(torch.tensor(dy))
    np.testing.assert_array_equal(g1, xt.grad.numpy())


def test_a_multi_dim_max_picks_the_first_position_dim_by_dim():
    rng = np.random.default_rng(8)
    xv = rng.integers(0, 2, size=(3, 4, 5)).astype(np.float64)
    region, y, rg = _extremum_joint(xv.shape, ("a", "b", "c"), ("b", "c"), "max")
    dy = rng.standard_normal(3)
    g1, g2 = _eval_joint(rg, y, xv, dy, ("a", "b", "c"))
    want = np.zeros_like(xv)
    for a in range(3):
        # reduce over b first (the first b attaining each c's max), then over c
        mb = xv[a].max(axis=0)
        c = int(np.flatnonzero(mb == mb.max())[0])
        b = int(np.flatnonzero(xv[a, :, c] == mb[c])[0])
        want[a, b, c] = dy[a]
    np.testing.assert_array_equal(g1, want)
    np.testing.assert_array_equal(g2, want)


def test_an_extremum_attained_once_matches_torch_autograd():
    rng = np.random.default_rng(2)
    xv = rng.standard_normal((5, 11))
    region, y, rg = _extremum_joint(xv.shape, ("t", "s"), ("s",), "max")
    dy = rng.standard_normal(5)
    g1, g2 = _eval_joint(rg, y, xv, dy, ("t", "s"))
    xt = torch.tensor(xv, requires_grad=True)
    xt.amax(dim=1).backward(torch.tensor(dy))
    np.testing.assert_allclose(g1, xt.grad.numpy(), rtol=0, atol=0)
    np.testing.assert_allclose(g2, xt.grad.numpy(), rtol=0, atol=0)


@pytest.mark.parametrize("reverse", [False, True])
def test_the_scan_sum_adjoint_matches_finite_differences(reverse):
    rng = np.random.default_rng(3)
    xv = rng.standard_normal((3, 6))
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "s"), xv.shape))
    extra = {"reverse": True} if reverse else {}
    s = b.emit("tl.scan", x, dim="s", f="sum", **extra)
    y = b.emit("tl.pointwise", s, s, f="mul")  # a nonlinear function of the scan
    region = Region(params=(x,), body=(b.emit("core.yield", y),))
    rg = grad(region, "out", seed="dy", wrt=("x",), names=region_names(region, ("x",), ("out",)))
    dy = rng.standard_normal(xv.shape)
    g1, g2 = _eval_joint(rg, y, xv, dy, ("t", "s"))

    def loss(arr):
        sc = _numpy_scan(arr, 1, "sum", reverse)
        return float(np.sum(sc * sc * dy))

    fd = np.zeros_like(xv)
    h = 1e-6
    for i in np.ndindex(xv.shape):
        e = np.zeros_like(xv)
        e[i] = h
        fd[i] = (loss(xv + e) - loss(xv - e)) / (2 * h)
    np.testing.assert_allclose(g1, fd, rtol=1e-6, atol=1e-8)
    np.testing.assert_allclose(g2, fd, rtol=1e-6, atol=1e-8)


def test_the_executor_splits_a_red_carve_at_its_scan():
    """Host side only (no device): a red carve in which a scan meets a
    reduction (a row max over a prefix sum) builds as one split step whose
    remainder runs as a nested plan (the bare max)."""
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl.partition import plan_model

    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "s"), (19, 333)))
    s1 = b.emit("tl.scan", x, dim="s", f="sum")
    y = b.emit("tl.reduce", b.emit("tl.pointwise", s1, s1, f="mul"), dims=("s",), f="max")
    region = Region(params=(x,), body=(b.emit("core.yield", y),))
    ex = PlanExecutor(plan_model(region), region, "f32")
    (step,) = ex.steps
    assert step.source == "split at scan sum along s (rest by nested plans)"
    (rest,) = ex.nested
    assert [st.source.split()[0] for st in rest.steps] == ["reduce_rows"]
