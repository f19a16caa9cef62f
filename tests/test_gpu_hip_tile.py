"""The HIP seat on silicon: compile_tile_hip(g.kernel, g.launch, g.prune)
runs the groups plan_region produced, against the float64 oracles — the
restated battery of conformance/test_fusion_triton.py and
conformance/test_triton_tile.py, at the reference's own tolerances (f32
column: rtol 1e-4 / atol 1e-6 for flash, 1e-5 / 1e-6 elsewhere)."""

import numpy as np
import pytest

from oracle import closed_forms as cf
from oracle import region_eval as re_
from tests.tolerances import assert_lowp

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SHARED_4090 = None


def _machine():
    from pdum_dsl_amd.tl.launch import TileLevel, TileMachine

    return TileMachine((TileLevel("shared", 128, 101376),))


def _oracle_out(subject):
    vals = [re_.value(f.arr, p.type) for f, p in zip(subject.inputs, subject.region.params)]
    res = re_.evaluate(subject.region, vals)
    return tuple(r.numpy() for r in res) if isinstance(res, tuple) else res.numpy()


def test_the_fused_flash_composition_runs_on_hip():
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo

    f = zoo.flash_tile()
    (g,) = fusion.plan_region(f.region).groups
    assert g.template == "flash"
    run = compile_tile_hip(g.kernel)
    got = run(f.numpy_inputs())
    np.testing.assert_allclose(got, _oracle_out(f), rtol=1e-4, atol=1e-6)
    assert "sweeps=1" in run.source and "stores=1" in run.source and run.grid == 1


def test_the_flashsm_reducer_runs_as_the_flash_row():
    """Attention spelled with the flashsm composite reducer plans as the
    flash row and runs on the same kernel."""
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo

    f = zoo.flash_attention(T=96, E=16, OD=8, seed=4)
    (g,) = fusion.plan_region(f.region).groups
    assert g.template == "flash"
    got = compile_tile_hip(g.kernel)(f.numpy_inputs())
    np.testing.assert_allclose(got, f.oracle(f.numpy_inputs()), rtol=1e-4, atol=1e-6)


def test_affine_views_run_on_the_map_chain_seat():
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, interp
    from tests.test_views_reducers import _affine_region

    r = _affine_region()
    (g,) = fusion.plan_region(r).groups
    rng = np.random.default_rng(15)
    X, Y = rng.standard_normal((3, 30)), rng.standard_normal((12, 3, 14))
    run = compile_tile_hip(g.kernel)
    want = interp.run_region(r, [interp.Field(X, r.params[0].type.dims), interp.Field(Y, r.params[1].type.dims)])
    np.testing.assert_allclose(run([X, Y]), want.to_numpy(r.body[-1].args[0].type.names), rtol=1e-5, atol=1e-6)
    assert "shifted_reads=3" in run.source


def test_the_hand_written_flash_tile_runs_on_hip():
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import zoo

    f = zoo.flash_tile(T=64, E=8, OD=4, SI=8)
    got = compile_tile_hip(f.tile)(f.numpy_inputs())
    np.testing.assert_allclose(got, _oracle_out(f), rtol=1e-4, atol=1e-6)


def test_the_planned_launch_runs_gridded():
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo

    f = zoo.flash_tile(T=512, E=64, OD=64, SI=2)
    (g,) = fusion.plan_region(f.region, machine=_machine()).groups
    assert g.template == "flash" and g.launch
    run = compile_tile_hip(g.kernel, g.launch)
    assert run.grid > 1
    want = cf.attention(*f.numpy_inputs(), band=(None, 0))[0]
    np.testing.assert_allclose(run(f.numpy_inputs()), want, rtol=1e-4, atol=1e-5)


def test_mask_derived_bounds_prune_the_sweep_bit_exactly():
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo

    f = zoo.flash_tile(T=128, E=32, OD=32, SI=2)
    (g,) = fusion.plan_region(f.region, machine=_machine()).groups
    assert g.prune == (("so", (0, 0, 1), (1, 1, 1)),)
    vals = f.numpy_inputs()
    full = compile_tile_hip(g.kernel, g.launch)
    pruned = compile_tile_hip(g.kernel, g.launch, g.prune)
    assert "prune=on" in pruned.source and "prune=off" in full.source
    np.testing.assert_array_equal(full(vals), pruned(vals))


def test_the_flash_artifacts_store_from_one_sweep():
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo

    a = zoo.attention(T=40, S=40, E=6, OD=5, mask="causal", artifacts=True, seed=31)
    (g,) = fusion.plan_region(a.region).groups
    run = compile_tile_hip(g.kernel)
    assert "stores=3" in run.source and "sweeps=1" in run.source
    got = run(a.numpy_inputs())
    assert isinstance(got, tuple) and len(got) == 3
    for x, w in zip(got, _oracle_out(a)):
        np.testing.assert_allclose(x, w, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("mask", ["all", "strict", ("window", 5)])
def test_other_closed_masks_bind_as_bands(mask):
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo

    a = zoo.attention(T=70, S=70, E=16, OD=8, mask=mask, seed=5)
    (g,) = fusion.plan_region(a.region).groups
    got = compile_tile_hip(g.kernel)(a.numpy_inputs())
    np.testing.assert_allclose(got, _oracle_out(a), rtol=1e-4, atol=1e-6)


def test_config_c1_single_head_noncausal_template_attention():
    """The CPU-runnable headline config C1: B=H=1, S=256, D=64, fp32, scale 1/sqrt(64) = 1/8
    applied to q (exact: a power of two), non-causal via an always-true
    closed mask, through the fusion template."""
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo

    a = zoo.attention(T=256, S=256, E=64, OD=64, mask="all", seed=0, scale=0.125)
    (g,) = fusion.plan_region(a.region).groups
    assert g.template == "flash" and dict(g.params)["si"] == 32
    got = compile_tile_hip(g.kernel)(a.numpy_inputs())
    q, k, v = a.numpy_inputs()
    want = cf.attention(q, k, v)[0]
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err <= 1e-5, f"C1 max-abs-err relative {err:.3e}"


def test_the_bf16_column_binds_the_mfma_kernel():
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo

    a = zoo.attention(T=192, S=192, E=64, OD=64, mask="causal", seed=2, scale=0.125)
    (g,) = fusion.plan_region(a.region).groups
    run = compile_tile_hip(g.kernel, dtype="bf16")
    assert "flash_fwd_m16<bf16,64>" in run.source
    q, k, v = (torch.as_tensor(x).to(torch.bfloat16).double().numpy() for x in a.numpy_inputs())
    assert_lowp(run(a.numpy_inputs()), cf.attention(q, k, v, band=(None, 0))[0])


@pytest.mark.parametrize("rows,cols", [(4, 6), (300, 1024), (33, 5000)])
def test_the_row_normalization_group_runs_on_hip(rows, cols):
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo

    s = zoo.row_softmax(rows, cols)
    (g,) = fusion.plan_region(s.region).groups
    run = compile_tile_hip(g.kernel)
    x = s.numpy_inputs()[0].astype(np.float32).astype(np.float64)
    np.testing.assert_allclose(run(s.numpy_inputs()), cf.np_softmax(x, axis=1), rtol=1e-5, atol=1e-6)


def test_softmax_over_a_leading_dim_is_transposed_by_name():
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo

    s = zoo.row_softmax(6, 5, names=("s", "t"))  # reduce over "t", the trailing name
    (g,) = fusion.plan_region(s.region).groups
    got = compile_tile_hip(g.kernel)(s.numpy_inputs())
    np.testing.assert_allclose(got, _oracle_out(s), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("affine", [False, True])
def test_the_rowstat_layernorm_runs_on_hip(affine):
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo

    ln = zoo.layernorm(rows=6, feat=768, affine=affine)
    (g,) = fusion.plan_region(ln.region).groups
    run = compile_tile_hip(g.kernel)
    assert "/ 768" in run.source  # the mean's divide-by-N, N static
    np.testing.assert_allclose(run(ln.numpy_inputs()), _oracle_out(ln), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_the_row_templates_run_on_16_bit_storage(dtype):
    """The row groups at the seat's 16-bit columns (fp32 arithmetic, storage
    rounded): within 2e-2 of the oracle on the rounded inputs."""
    import torch

    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo

    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    for subj in (zoo.row_softmax(33, 1024), zoo.layernorm(rows=9, feat=768, affine=True)):
        (g,) = fusion.plan_region(subj.region).groups
        run = compile_tile_hip(g.kernel, dtype=dtype)
        assert f"dtype={dtype}" in run.source
        vals = [torch.as_tensor(v).to(tdt).double().numpy() for v in subj.numpy_inputs()]
        got = run(vals)
        want = subj.oracle(vals)
        assert np.abs(got - want).max() <= 2e-2 * max(1.0, np.abs(want).max())


def test_run_dev_takes_device_tensors_and_matches_run():
    """The device-resident form of the seat (run.run_dev): torch tensors in,
    device tensors out, no host copies or synchronization; bit-equal to the
    numpy contract ``run``."""
    import torch

    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion, zoo
    from tests.test_contraction_mapchain import gemm_subject

    f = zoo.flash_tile(T=64, E=16, OD=16, SI=8)
    ln = zoo.layernorm(rows=7, feat=512)
    gm, gvals = gemm_subject(M=70, K=96, N=50, epilogue="gelu_tanh", seed=2)
    st = zoo.stencil_tile(MI=40, NI=60)
    for region, vals in ((f.tile, f.numpy_inputs()), (fusion.plan_region(ln.region).groups[0].kernel, ln.numpy_inputs()),
                         (fusion.plan_region(gm).groups[0].kernel, gvals), (st.region, [st.inputs[0].arr])):
        run = compile_tile_hip(region, dtype="f32")
        host = run(vals)
        dev = run.run_dev([torch.as_tensor(np.asarray(v), dtype=torch.float32, device="cuda") for v in vals])
        torch.cuda.synchronize()
        dev = dev if isinstance(dev, tuple) else (dev,)
        host = host if isinstance(host, tuple) else (host,)
        assert all(d.is_cuda for d in dev)
        for d, h in zip(dev, host):
            np.testing.assert_array_equal(d.cpu().numpy(), h)
    # the stencil's runner on a side stream the caller names: the same bits once it is synchronized
    side = torch.cuda.Stream()
    x = torch.as_tensor(np.asarray(st.inputs[0].arr), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    got = run.run_dev([x], stream=side)
    side.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), run([st.inputs[0].arr]))
