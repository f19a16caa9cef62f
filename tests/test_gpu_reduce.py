"""The ROWSUM and PLAIN shapes of the contraction-epilogue row on silicon
(fusion.py:158-252: same-space operands multiplied and summed, e.g. the
backward's D = rowsum(dO * O); one operand summed, e.g. a bias gradient),
bound by the seat and by the carved-plan executor to pdh_reduce_rows, against
the float64 oracle evaluation of the naive region.

Tolerances: fp32 1e-5 of scale (fp32 sums of up to 4096 terms); bf16 2e-2."""

import numpy as np
import pytest

from oracle import region_eval as rev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _subject(shape, T=37, S=300, epi=None, f="sum", seed=0, dims=None):
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import Builder, Region, tensor_type

    rng = np.random.default_rng(seed)
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "s"), (T, S)))
    params, vals = [x], [rng.standard_normal((T, S))]
    if shape == "rowsum":
        z = b.param(1, tensor_type(("t", "s"), (T, S)))
        params.append(z)
        vals.append(rng.standard_normal((T, S)))
        summand = b.emit("tl.pointwise", x, z, f="mul")
    else:
        summand = x
    red = b.emit("tl.reduce", summand, dims=dims or ("s",), f=f)
    y = red
    if epi == "scale_bias":
        bias = b.param(len(params), red.type)
        params.append(bias)
        vals.append(rng.standard_normal(red.type.shape))
        y = b.emit("tl.pointwise", b.emit("tl.pointwise", red, _const(b, 0.5), f="mul"), bias, f="add")
    return Region(params=tuple(params), body=(b.emit("core.yield", y),)), vals


def _const(b, v):
    from pdum_dsl_amd.tl.ir import F64

    return b.emit("core.const", type=F64, value=float(v))


def _oracle(region, vals):
    got = rev.evaluate(region, [rev.value(v, p.type) for v, p in zip(vals, region.params)])
    y = region.body[-1].args[0]
    return got.numpy(y.type.names)


CASES = [("rowsum", ("s",), None, "sum"), ("rowsum", ("s",), "scale_bias", "sum"), ("plain", ("t",), None, "sum"),
         ("plain", ("t",), "scale_bias", "sum"), ("plain", ("s",), None, "mean"), ("plain", ("t", "s"), None, "sum")]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape,dims,epi,f", CASES)
def test_the_seat_binds_rowsum_and_plain_to_the_row_reduce_kernel(dtype, shape, dims, epi, f):
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion

    region, vals = _subject(shape, epi=epi, f=f, dims=dims)
    (g,) = fusion.plan_region(region).groups
    assert g.template == "contraction-epilogue" and dict(g.params)["shape"] == shape
    run = compile_tile_hip(g.kernel, dtype=dtype)
    assert run.source.startswith(f"hip:reduce_rows shape={shape}")
    if dtype == "bf16":
        vals = [torch.as_tensor(v).to(torch.bfloat16).double().numpy() for v in vals]
    got = np.asarray(run(vals), dtype=np.float64)
    want = _oracle(region, vals)
    tol = 1e-5 if dtype == "f32" else 2e-2
    assert np.abs(got - want).max() <= tol * max(1.0, np.abs(want).max())


def test_the_executor_runs_a_rowsum_carve():
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl.partition import plan_model

    region, vals = _subject("rowsum", T=512, S=4096, epi="scale_bias", seed=3)
    plan = plan_model(region)
    assert [c.group.template for c in plan.carves] == ["contraction-epilogue"]
    ex = PlanExecutor(plan, region, "f32")
    assert "reduce_rows rowsum" in ex.sources()[0]
    ex.bind(vals)
    got = ex.run().cpu().numpy()
    want = _oracle(region, vals)
    assert np.abs(got - want).max() <= 1e-5 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("f", ["sum", "max", "min"])
@pytest.mark.parametrize("T,S", [(1024, 3072), (37, 307)])
def test_a_reduction_over_the_strided_dim_runs_by_columns(f, T, S):
    """x[t, s] reduced over t (s contiguous: a bias gradient's shape) takes the
    column variant of pdh_reduce_rows_ex (16 consecutive outputs per
    workgroup, coalesced loads); against numpy, NaN positions included."""
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import Builder, Region, tensor_type
    from pdum_dsl_amd.tl.partition import plan_model

    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "s"), (T, S)))
    y = b.emit("tl.reduce", x, dims=("t",), f=f)
    region = Region(params=(x,), body=(b.emit("core.yield", y),))
    ex = PlanExecutor(plan_model(region), region, "f32")
    xv = np.random.default_rng(T + S).standard_normal((T, S))
    xv[T // 2, 5] = np.nan
    ex.bind([xv])
    got = ex.run().cpu().numpy().astype(np.float64)
    torch.cuda.synchronize()
    want = {"sum": np.sum, "max": np.max, "min": np.min}[f](xv.astype(np.float32).astype(np.float64), axis=0)
    assert np.array_equal(np.isnan(got), np.isnan(want)) and np.isnan(want).sum() == 1
    ok = ~np.isnan(want)
    if f == "sum":
        assert np.abs(got[ok] - want[ok]).max() <= 1e-5 * max(1.0, np.abs(want[ok]).max()) * (T / 64) ** 0.5
    else:
        np.testing.assert_array_equal(got[ok], want[ok])
