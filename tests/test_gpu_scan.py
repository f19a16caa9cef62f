"""tl.scan on the device: pdh_scan against numpy's ufunc.accumulate (the
reference's scan, compute.py:318-350), and the carved-plan executor running
a max / min joint's first-occurrence adjoint (autodiff.py:635-665) with ties.

Tolerances: max / min / the 0-1 counts are exact; fp32 sums and products of
up to 5000 terms within 1e-5 of scale (the wave-tree order differs from
numpy's sequential one); bf16 storage within 2e-2 of scale."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

_ACC = {"sum": np.add, "prod": np.multiply, "max": np.maximum, "min": np.minimum}


def _want(arr, axis, f, reverse):
    a = np.flip(arr, axis) if reverse else arr
    out = (np.add if f == "mean" else _ACC[f]).accumulate(a, axis=axis)
    if f == "mean":
        shape = [1] * a.ndim
        shape[axis] = a.shape[axis]
        out = out / np.arange(1, a.shape[axis] + 1).reshape(shape)
    return np.flip(out, axis) if reverse else out


@pytest.mark.parametrize("f", ["sum", "max", "min", "prod", "mean"])
@pytest.mark.parametrize("shape,dim", [((37, 5000), 1), ((6, 130, 9), 1), ((300, 4), 0), ((3, 1), 1)])
@pytest.mark.parametrize("reverse", [False, True])
def test_scan_matches_ufunc_accumulate(f, shape, dim, reverse):
    from pdum_dsl_amd import kernels as K

    rng = np.random.default_rng(sum(shape) + dim)
    arr = rng.standard_normal(shape)
    if f == "prod":  # keep products finite and away from 0: factors near 1
        arr = 1.0 + 0.001 * arr
    arr.flat[len(arr.flat) // 3] = np.nan  # poisons its prefix's remainder
    x = torch.as_tensor(arr, dtype=torch.float32, device="cuda")
    got = K.scan(x, dim, f, reverse=reverse).cpu().numpy().astype(np.float64)
    want = _want(arr.astype(np.float32).astype(np.float64), dim, f, reverse)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    if f in ("max", "min"):
        np.testing.assert_array_equal(got[ok], want[ok])
    else:
        assert np.abs(got[ok] - want[ok]).max() <= 1e-5 * max(1.0, np.abs(want[ok]).max())


def test_scan_in_bf16_storage_and_in_place():
    from pdum_dsl_amd import kernels as K

    arr = np.random.default_rng(2).standard_normal((64, 700))
    x = torch.as_tensor(arr, dtype=torch.bfloat16, device="cuda")
    want = np.add.accumulate(x.float().cpu().numpy().astype(np.float64), axis=1)
    got = K.scan(x, 1, "sum", out=x).float().cpu().numpy()  # y may be x
    assert np.abs(got - want).max() <= 2e-2 * max(1.0, np.abs(want).max())
    counts = torch.as_tensor((arr > 0).astype(np.float32), dtype=torch.bfloat16, device="cuda")
    want_c = np.add.accumulate(arr > 0, axis=1)  # integer counts below 256 are exact in bf16
    got_c = K.scan(counts[:, :255].contiguous(), 1, "sum").float().cpu().numpy()
    np.testing.assert_array_equal(got_c, want_c[:, :255])


def test_an_empty_scan_launches_nothing():
    from pdum_dsl_amd import kernels as K

    x = torch.empty((0, 5), device="cuda")
    assert K.scan(x, 1, "sum").shape == (0, 5)


@pytest.mark.parametrize("f", ["max", "min"])
def test_the_executor_runs_a_tied_extremum_joint(f):
    """grad of a row max / min plans into a bare-reduce carve and a red carve
    around the prefix count (a tl.scan); the device joint must send each
    row's cotangent to the first position attaining the extremum."""
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl.autodiff import grad, region_names
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import Builder, Region, tensor_type, walk
    from pdum_dsl_amd.tl.partition import plan_model

    T, S = 37, 700
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "s"), (T, S)))
    y = b.emit("tl.reduce", x, dims=("s",), f=f)
    region = Region(params=(x,), body=(b.emit("core.yield", y),))
    rg = grad(region, "out", seed="dy", wrt=("x",), names=region_names(region, ("x",), ("out",)))
    assert any(n.op == "tl.scan" for n in walk(rg.region))
    ex = PlanExecutor(plan_model(rg.region), rg.region, "f32")
    assert any("scan" in st.source for st in ex.steps)
    rng = np.random.default_rng(9)
    xv = rng.integers(0, 4, size=(T, S)).astype(np.float64)  # many ties per row
    dy = rng.standard_normal(T)
    ex.bind([xv, dy])
    out, dx = ex.run()
    torch.cuda.synchronize()
    want = np.zeros((T, S))
    for t in range(T):
        ext = xv[t].max() if f == "max" else xv[t].min()
        want[t, int(np.flatnonzero(xv[t] == ext)[0])] = np.float32(dy[t])
    got = np.transpose(dx.cpu().numpy(), [rg.nodes["dx"].type.names.index(n) for n in ("t", "s")])
    np.testing.assert_array_equal(got, want)


def _scan_then(kind):
    """Regions whose red carve holds a scan beside other work a map chain
    cannot hold: a row max over a prefix sum, and a scan of a scan."""
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import Builder, Region, tensor_type

    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "s"), (19, 333)))
    s1 = b.emit("tl.scan", x, dim="s", f="sum")
    if kind == "max-of-scan":
        y = b.emit("tl.reduce", b.emit("tl.pointwise", s1, s1, f="mul"), dims=("s",), f="max")
    else:  # scan of a scan, reversed, then elementwise
        s2 = b.emit("tl.scan", b.emit("tl.pointwise", s1, f="tanh"), dim="s", f="sum", reverse=True)
        y = b.emit("tl.pointwise", s2, x, f="mul")
    return Region(params=(x,), body=(b.emit("core.yield", y),))


@pytest.mark.parametrize("kind", ["max-of-scan", "scan-of-scan"])
def test_a_red_carve_splits_at_its_scan(kind):
    from oracle import region_eval as rev
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl.partition import plan_model

    region = _scan_then(kind)
    ex = PlanExecutor(plan_model(region), region, "f32")
    assert any("split at scan" in st.source for st in ex.steps)
    xv = np.random.default_rng(12).standard_normal((19, 333)) * 0.3
    ex.bind([xv])
    got = ex.run().cpu().numpy().astype(np.float64)
    torch.cuda.synchronize()
    y = region.body[-1].args[0]
    want = rev.evaluate(region, [rev.value(xv, region.params[0].type)]).numpy(y.type.names)
    assert np.abs(got - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
