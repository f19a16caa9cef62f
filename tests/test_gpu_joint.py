"""The flash joint on silicon: autodiff.grad -> partition.plan_model ->
compile_tile_hip(carve) runs (out, *grads) through the forward-with-artifacts
and backward kernels, against the joint's float64 evaluation by the oracle
(oracle.region_eval over the very region the carve holds) and the closed-form
gradients. This is the restated test_partition.py:124-193 battery (the flash
joint executes to the naive joint) with the HIP seat as the executor; plus
the fp32 backward column directly through the C ABI at ragged shapes."""

import numpy as np
import pytest

from oracle import closed_forms as cf
from oracle import region_eval as rev
from tests.tolerances import assert_fp32, assert_lowp

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

MASKS = [("causal", (None, 0)), ("all", None), ("strict", (None, -1)), (("window", 5), (-4, 0))]


def _plan_joint(T, S, E, OD, mask, wrt=("q", "k", "v"), seed=3, qscale=1.0):
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.autodiff import grad, region_names
    from pdum_dsl_amd.tl.launch import TileLevel, TileMachine
    from pdum_dsl_amd.tl.partition import plan_model

    subj = zoo.attention(T=T, S=S, E=E, OD=OD, mask=mask, seed=seed, scale=qscale)
    rg = grad(subj.region, "out", seed="dO", wrt=wrt, names=region_names(subj.region, ("q", "k", "v")))
    mp = plan_model(rg.region, machine=TileMachine((TileLevel("shared", 128, 101376),)))
    (carve,) = mp.carves
    assert carve.group.template == "flash-joint"
    dO = np.random.default_rng(seed + 1).standard_normal((T, OD))
    return subj, rg, carve, dO


def _yield_names(rg):
    return [n.type.names for n in rg.region.body[-1].args[0].args]


def _oracle_joint(rg, values):
    """The joint's outputs in each yielded node's type-dim order (the seat's contract)."""
    vals = [rev.value(a, p.type) for a, p in zip(values, rg.region.params)]
    return [r.numpy(names) for r, names in zip(rev.evaluate(rg.region, vals), _yield_names(rg))]


def _as(arr, canon, names):
    return np.transpose(arr, [canon.index(n) for n in names])


@pytest.mark.parametrize("mask,band", MASKS)
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_the_flash_joint_runs_on_hip(mask, band, dtype):
    from pdum_dsl_amd.hip_tile import compile_tile_hip

    T = S = 96
    E, OD = (64, 64) if dtype == "bf16" else (24, 40)
    # the template carries no score scale: q is drawn at 1/sqrt(E) (attention's usual statistics),
    # so bf16's input rounding is measured against scores of unit spread
    subj, rg, carve, dO = _plan_joint(T, S, E, OD, mask, qscale=E**-0.5)
    run = compile_tile_hip(carve.kernel, carve.group.launch, carve.group.prune, dtype=dtype)
    assert run.template == "flash-joint" and "launches=fwd+bwd" in run.source
    values = subj.numpy_inputs() + [dO]
    got = run(values)
    want = _oracle_joint(rg, values)
    q, k, v = subj.numpy_inputs()
    closed = (cf.attention(q, k, v, scale=1.0, band=band)[0],) + cf.attention_bwd(q, k, v, dO, scale=1.0, band=band)
    canon = (("t", "o"), ("t", "e"), ("s", "e"), ("s", "o"))
    closed = [_as(c, cn, names) for c, cn, names in zip(closed, canon, _yield_names(rg))]
    for name, g, w, c in zip(rg.outputs, got, want, closed):
        np.testing.assert_allclose(w, c, rtol=1e-9, atol=1e-9, err_msg=f"oracle joint vs closed form: {name}")
        if dtype == "f32":
            assert_fp32(g, w, rtol=0.0, atol=1e-5 * max(1.0, np.abs(w).max()), what=f"{name} {mask}")
        else:
            assert_lowp(g, w, what=f"{name} {mask}")


def test_a_partial_joint_yields_its_grads_in_order():
    from pdum_dsl_amd.hip_tile import compile_tile_hip

    subj, rg, carve, dO = _plan_joint(64, 64, 64, 64, "causal", wrt=("v", "q"), qscale=0.125)
    run = compile_tile_hip(carve.kernel, carve.group.launch, carve.group.prune, dtype="bf16")
    values = subj.numpy_inputs() + [dO]
    got = run(values)
    want = _oracle_joint(rg, values)
    assert len(got) == 3 and rg.outputs == ("out", "dv", "dq")
    for g, w in zip(got, want):
        assert_lowp(g, w)


@pytest.mark.parametrize(
    "T,S,E,OD,band",
    [(70, 130, 33, 17, (None, 0)), (129, 64, 8, 200, None), (65, 65, 64, 64, (None, -1)), (200, 200, 96, 96, (-31, 0))],
)
def test_fp32_backward_matches_the_closed_form(T, S, E, OD, band):
    from pdum_dsl_amd import kernels as K

    rng = np.random.default_rng(T * 7 + S)
    dev = "cuda"
    q, k, v = (torch.as_tensor(rng.standard_normal(sh), dtype=torch.float32, device=dev).view(1, 1, *sh)
               for sh in ((T, E), (S, E), (S, OD)))
    do = torch.as_tensor(rng.standard_normal((T, OD)), dtype=torch.float32, device=dev).view(1, 1, T, OD)
    kb = K.Band(*band) if band is not None else None
    fw = K.flash_fwd(q, k, v, scale=0.25, band=kb, want_artifacts=True)
    dq, dk, dv = K.flash_bwd(q, k, v, fw.o, do, fw.lse, m=fw.m, den=fw.den, scale=0.25, band=kb)
    torch.cuda.synchronize()
    h = lambda t: t.detach().cpu().numpy().astype(np.float64)[0, 0]  # noqa: E731
    wq, wk, wv = cf.attention_bwd(h(q), h(k), h(v), h(do), scale=0.25, band=band)
    for name, g, w in (("dq", dq, wq), ("dk", dk, wk), ("dv", dv, wv)):
        assert_fp32(h(g), w, rtol=0.0, atol=1e-5 * max(1.0, np.abs(w).max()), what=name)
