"""The tile flagships on silicon (the reference's
conformance/test_triton_tile.py:20-32 and :106-119 restated): the gemm,
stencil and flash tile programs bound by compile_tile_hip against their numpy
oracles; the gridded stencil is bit-equal to the ungridded one; a stencil
planned by plan_model runs through the device executor.

Tolerances: fp32 1e-5 relative (the reference's 1e-5 / 1e-6 for its fp32
Triton column); bf16 2e-2 of scale."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.mark.parametrize("name", ["gemm", "stencil", "flash"])
def test_translated_flagships_run_on_hip(name):
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import zoo

    f = {"gemm": zoo.gemm_tile, "stencil": zoo.stencil_tile, "flash": zoo.flash_tile}[name]()
    run = compile_tile_hip(f.tile if name == "flash" else f.region)  # the flash subject carries its tile apart
    vals = [v.arr for v in f.inputs]
    got = run(vals)
    got = got[0] if isinstance(got, tuple) else got
    np.testing.assert_allclose(got, f.oracle(vals), rtol=1e-5, atol=1e-6)


def test_the_grid_partition_is_bit_exact_without_reductions():
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import zoo

    s = zoo.stencil_tile(MI=30, NI=46)
    u = [s.inputs[0].arr]
    one = compile_tile_hip(s.region)(u)
    g = compile_tile_hip(s.region, launch=(("x", 16), ("y", 16)))
    assert g.grid == 6
    assert "shifted_reads=4" in g.source  # the centre reads at offset 0 too, four move
    np.testing.assert_array_equal(one, g(u))


@pytest.mark.parametrize("dtype,tol", [("f32", 1e-5), ("bf16", 2e-2)])
def test_a_large_stencil_matches_the_closed_form(dtype, tol):
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import zoo

    s = zoo.stencil_tile(MI=1000, NI=1534, alpha=0.2, seed=4)
    u = s.inputs[0].arr
    got = compile_tile_hip(s.region, dtype=dtype)([u])
    uu = torch.as_tensor(u).to(torch.bfloat16).double().numpy() if dtype == "bf16" else u
    want = s.oracle([uu])
    assert np.abs(got - want).max() <= tol * max(1.0, np.abs(want).max())


def test_a_planned_stencil_runs_through_the_executor():
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.partition import plan_model

    s = zoo.stencil_tile(MI=256, NI=512, seed=8)
    plan = plan_model(s.naive)
    assert [c.group.template for c in plan.carves] == ["stencil"]
    ex = PlanExecutor(plan, s.naive, "f32")
    ex.bind([s.inputs[0].arr])
    got = ex.run().cpu().numpy()
    np.testing.assert_allclose(got, s.oracle([s.inputs[0].arr]), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("MI,NI", [(64, 64), (30, 46)])
def test_the_stencil_joint_runs_on_the_device(MI, NI):
    """grad of the 5-point update w.r.t. its halo (each tap's cotangent shifted
    back and zero-padded to the halo frame, summed) planned by plan_model and
    run by the executor: the pads materialized into fill-valued buffers, then
    one map chain over their offset views. Against the float64 oracle's
    evaluation of the same joint, and the forward against the numpy model."""
    from oracle import region_eval as rev
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.autodiff import grad, region_names
    from pdum_dsl_amd.tl.partition import plan_model

    s = zoo.stencil_tile(MI=MI, NI=NI, alpha=0.1, seed=17)
    reg = s.naive
    rg = grad(reg, "out", seed="dout", names=region_names(reg, ("u",)))
    ex = PlanExecutor(plan_model(rg.region), rg.region, "f32")
    assert any(st.source.startswith("padded pads=") for st in ex.steps), [st.source for st in ex.steps]
    u = s.inputs[0].arr
    dout = np.random.default_rng(5).standard_normal(tuple(rg.region.params[-1].type.shape))
    vals = [u, dout]
    ex.bind(vals)
    outs = ex.run()
    torch.cuda.synchronize()
    want = rev.evaluate(rg.region, [rev.value(v, p.type) for v, p in zip(vals, rg.region.params)])
    assert len(outs) == len(want) == 2
    np.testing.assert_allclose(outs[0].cpu().numpy(), s.oracle([u]), rtol=1e-5, atol=1e-6)
    for g, w in zip(outs, want):
        w = w.numpy()
        assert np.abs(g.cpu().numpy() - w).max() <= 1e-5 * max(1.0, np.abs(w).max())
