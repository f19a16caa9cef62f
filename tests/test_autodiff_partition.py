"""autodiff.grad and partition.plan_model (CPU).

The reference's own batteries for these layers are CPU tests against the
oracle (packages/tensorlib/tests/test_partition.py:124-193: the flash joint
executes to the naive joint at 1e-9; autodiff tests against numpy / finite
differences). Here the joint region ``grad`` builds is evaluated by BOTH
interpreters (the planner's numpy one and the oracle's torch-f64 one) and
checked against the closed-form gradients (oracle.closed_forms.attention_bwd,
itself pinned by torch.autograd and finite differences in test_oracle.py),
and row templates' joints against torch.autograd in float64."""

import numpy as np
import pytest
import torch

from oracle import closed_forms as cf
from oracle import region_eval as rev
from pdum_dsl_amd.tl import interp, zoo
from pdum_dsl_amd.tl.autodiff import grad, region_names
from pdum_dsl_amd.tl.launch import TileLevel, TileMachine
from pdum_dsl_amd.tl.partition import match_flash_joint, plan_model

RTX4090 = TileMachine((TileLevel("shared", 128, 101376),))
MASKS = [("causal", (None, 0)), ("all", None), ("strict", (None, -1)), (("window", 3), (-2, 0))]


def _joint(subj, wrt=("q", "k", "v")):
    names = region_names(subj.region, ("q", "k", "v"), ("out",))
    return grad(subj.region, "out", seed="dO", wrt=wrt, names=names)


@pytest.mark.parametrize("mask,band", MASKS)
def test_attention_joint_equals_the_closed_form_on_both_interpreters(mask, band):
    subj = zoo.attention(T=9, S=9, E=5, OD=4, mask=mask, seed=3)
    rg = _joint(subj)
    assert rg.outputs == ("out", "dq", "dk", "dv")
    assert rg.grads == {"q": "dq", "k": "dk", "v": "dv"}
    dO = np.random.default_rng(0).standard_normal((9, 4))
    q, k, v = subj.numpy_inputs()
    wq, wk, wv = cf.attention_bwd(q, k, v, dO, scale=1.0, band=band)
    wo = cf.attention(q, k, v, scale=1.0, band=band)[0]
    # planner's numpy interpreter
    res = interp.run_region(rg.region, subj.inputs + [interp.field(dO, ("t", "o"))])
    got = [res[0].to_numpy(("t", "o")), res[1].to_numpy(("t", "e")), res[2].to_numpy(("s", "e")),
           res[3].to_numpy(("s", "o"))]
    for g, w in zip(got, (wo, wq, wk, wv)):
        np.testing.assert_allclose(g, w, rtol=1e-9, atol=1e-12)
    # the oracle's torch-f64 evaluator, independently
    vals = [rev.value(a, p.type) for a, p in zip([q, k, v, dO], rg.region.params)]
    res2 = rev.evaluate(rg.region, vals)
    got2 = [res2[0].numpy(("t", "o")), res2[1].numpy(("t", "e")), res2[2].numpy(("s", "e")), res2[3].numpy(("s", "o"))]
    for g, w in zip(got2, (wo, wq, wk, wv)):
        np.testing.assert_allclose(g, w, rtol=1e-9, atol=1e-12)


def test_a_partial_wrt_yields_only_those_grads_in_order():
    subj = zoo.attention(T=6, E=3, OD=2, mask="causal", seed=7)
    rg = _joint(subj, wrt=("v", "q"))
    assert rg.outputs == ("out", "dv", "dq")
    assert len(rg.region.params) == 4 and rg.names[id(rg.region.params[-1])] == "dO"


def _autograd_rows(fn, x, extra, seed):
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    ex = [torch.tensor(e, dtype=torch.float64, requires_grad=True) for e in extra]
    y = fn(xt, *ex)
    y.backward(torch.tensor(seed, dtype=torch.float64))
    return [xt.grad.numpy()] + [e.grad.numpy() for e in ex]


def test_row_softmax_joint_matches_torch_autograd():
    subj = zoo.row_softmax(rows=5, cols=7, seed=4)
    names = region_names(subj.region, ("x",), ("y",))
    rg = grad(subj.region, "y", seed="dy", names=names)
    dy = np.random.default_rng(1).standard_normal((5, 7))
    res = interp.run_region(rg.region, subj.inputs + [interp.field(dy, ("t", "s"))])
    (want,) = _autograd_rows(lambda x: torch.softmax(x, dim=1), subj.numpy_inputs()[0], [], dy)
    np.testing.assert_allclose(res[1].to_numpy(("t", "s")), want, rtol=1e-9, atol=1e-12)


def test_layernorm_joint_matches_torch_autograd():
    subj = zoo.layernorm(rows=4, feat=6, seed=2)
    names = region_names(subj.region, ("x", "g", "b"), ("y",))
    rg = grad(subj.region, "y", seed="dy", names=names)
    dy = np.random.default_rng(2).standard_normal((4, 6))
    res = interp.run_region(rg.region, subj.inputs + [interp.field(dy, ("t", "d"))])
    x, g, b = subj.numpy_inputs()
    want = _autograd_rows(
        lambda x, g, b: torch.nn.functional.layer_norm(x, (6,), g, b, eps=1e-5), x, [g, b], dy
    )
    got = [res[1].to_numpy(("t", "d")), res[2].to_numpy(("d",)), res[3].to_numpy(("d",))]
    for a, w in zip(got, want):
        np.testing.assert_allclose(a, w, rtol=1e-8, atol=1e-10)


def test_grad_refuses_what_it_cannot_linearize():
    # folds differentiate, read at their final state or emitting
    # (tests/test_fold_adjoint.py, tests/test_views_reducers.py); a top-k
    # selection has no linearization here
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import Builder, Region, tensor_type

    b = Builder(OPS)
    x = b.param(0, tensor_type(("r", "c"), (3, 5)))
    top = b.emit("tl.argtopk", x, dim="c", k=2, k_name="j")
    r2 = Region(params=(x,), body=(b.emit("core.yield", top),))
    with pytest.raises(NotImplementedError, match="tl.argtopk"):
        grad(r2, "out", seed="w", names=region_names(r2, ("x",)))
    subj = zoo.attention(T=6, E=3, OD=2, seed=7)
    with pytest.raises(ValueError, match="not a scalar"):
        grad(subj.region, "out", names=region_names(subj.region, ("q", "k", "v")))
    with pytest.raises(ValueError, match="collides"):
        grad(subj.region, "out", seed="q", names=region_names(subj.region, ("q", "k", "v")))
    with pytest.raises(KeyError, match="not defined"):
        grad(subj.region, "nope", seed="dO", names=region_names(subj.region, ("q", "k", "v")))


# ------------------------------------------------------------ plan_model


@pytest.mark.parametrize("wrt", [("q", "k", "v"), ("v", "q"), ("k",)])
def test_plan_model_claims_the_flash_joint_whole(wrt):
    subj = zoo.attention(T=128, S=128, E=32, OD=32, mask="causal", seed=3)
    rg = _joint(subj, wrt)
    mp = plan_model(rg.region, machine=RTX4090)
    assert len(mp.carves) == 1 and mp.coverage() == 1.0 and mp.distinct_kernels() == 1
    g = mp.carves[0].group
    assert (g.template, g.confidence) == ("flash-joint", "yellow")
    assert dict(g.params)["wrt"] == wrt and dict(g.params)["forward"] == "flash"
    assert dict(g.params)["si"] == 32
    assert g.certificate.verdict == "proved-exact" and g.certificate.licenses == ("flash.online-softmax",)
    # the forward's launch and mask-derived prune ride along (test_launch.py:114-117's answer)
    assert g.launch == (("t", 32),)  # smallest t-tile at or above the 1024-element floor
    assert g.prune == (("so", (0, 0, 1), (1, 1, 1)),)
    assert g.artifacts == ("m", "den")
    assert mp.carves[0].root_op == "tl.reduce"


def test_a_tampered_joint_is_not_a_flash_joint():
    subj = zoo.attention(T=8, E=4, OD=4, mask="causal", seed=3)
    rg = _joint(subj)
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import F64, Builder, Region

    b = Builder(OPS)
    y = rg.region.body[-1].args[0]
    dq2 = b.emit("tl.pointwise", y.args[1], b.emit("core.const", type=F64, value=2.0), f="mul")
    bad = Region(params=rg.region.params, body=(b.emit("core.yield", b.emit("core.tuple", y.args[0], dq2, *y.args[2:])),))
    assert match_flash_joint(bad) is None
    mp = plan_model(bad)
    assert mp.carves[0].group.template != "flash-joint"


def test_plan_model_of_a_single_template_region_is_its_plan_region():
    for subj, tmpl in ((zoo.row_softmax(), "row-normalization"), (zoo.layernorm(), "row-statistics"),
                       (zoo.attention(T=8, E=4, OD=4), "flash")):
        mp = plan_model(subj.region)
        assert [c.group.template for c in mp.carves] == [tmpl]
        assert mp.coverage() == 1.0


def test_the_gelu_marker_differentiates_through_its_derived_partial():
    """grad of zoo.gelu (the composite marker, zoo_common.py:20) emits the
    derived partial marker zoo.gelu.d0, as autodiff.py:303-309 derives f.d{i}.
    Pinned by torch's own tanh-approximate gelu and its autograd (a separate
    implementation), on the planner's interpreter, the float64 oracle and the
    lowered elementwise program."""
    from pdum_dsl_amd import ewprog
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import Builder, Dim, Region, TensorType
    from tests.test_contraction_mapchain import emulate

    b = Builder(OPS)
    x = b.param(0, TensorType((Dim("i", 0, 9), Dim("j", 0, 11))))
    y = b.emit("tl.pointwise", x, f="zoo.gelu")
    region = Region(params=(x,), body=(b.emit("core.yield", y),))
    names = region_names(region, ("x",), ("y",))
    rg = grad(region, "y", seed="dy", names=names)
    rng = np.random.default_rng(5)
    xv, dy = rng.standard_normal((9, 11)) * 3, rng.standard_normal((9, 11))
    xt = torch.tensor(xv, requires_grad=True)
    torch.nn.functional.gelu(xt, approximate="tanh").backward(torch.tensor(dy))
    res = interp.run_region(rg.region, [interp.field(xv, ("i", "j")), interp.field(dy, ("i", "j"))])
    np.testing.assert_allclose(res[1].to_numpy(("i", "j")), xt.grad.numpy(), rtol=1e-12, atol=1e-14)
    got = rev.evaluate(rg.region, [rev.value(xv, x.type), rev.value(dy, rg.region.params[1].type)])
    np.testing.assert_allclose(got[1].numpy(), xt.grad.numpy(), rtol=1e-12, atol=1e-14)
    from pdum_dsl_amd.tl.ir import walk

    assert any(n.op == "tl.pointwise" and n.attr("f") == "zoo.gelu.d0" for n in walk(rg.region))
    bb = Builder(OPS)
    xp = bb.param(0, x.type)
    dn = bb.emit("tl.pointwise", xp, f="zoo.gelu.d0")
    low = ewprog.lower(dn, dn.type.dims, {id(xp): xp})
    want = xt.grad.numpy() / dy
    np.testing.assert_allclose(emulate(low, [xv]), want, rtol=1e-9, atol=1e-12)


def test_rename_adjoint_and_wrt_pruning():
    """A rename's cotangent takes the operand's names back; nodes with no wrt
    param among their ancestors are not differentiated (the joint of gpt2's
    weights without its embedding tables then needs no adjoint for the
    gather). Against torch autograd."""
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import Builder, Dim, Region, TensorType, walk

    b = Builder(OPS)
    x = b.param(0, TensorType((Dim("t", 0, 5), Dim("d", 0, 3))))
    w = b.param(1, TensorType((Dim("d", 0, 3),)))
    r = b.emit("tl.rename", x, mapping=(("t", "s"),))
    y = b.emit("tl.pointwise", b.emit("tl.pointwise", r, f="tanh"), b.emit("tl.repeat_like", w, r), f="mul")
    region = Region(params=(x, w), body=(b.emit("core.yield", y),))
    names = region_names(region, ("x", "w"), ("y",))
    rng = np.random.default_rng(8)
    xv, wv, dy = rng.standard_normal((5, 3)), rng.standard_normal(3), rng.standard_normal((5, 3))
    xt, wt = torch.tensor(xv, requires_grad=True), torch.tensor(wv, requires_grad=True)
    (torch.tanh(xt) * wt).backward(torch.tensor(dy))
    full = grad(region, "y", seed="dy", names=names)
    res = interp.run_region(full.region, [interp.field(xv, ("t", "d")), interp.field(wv, ("d",)),
                                          interp.field(dy, ("s", "d"))])
    np.testing.assert_allclose(res[1].to_numpy(("t", "d")), xt.grad.numpy(), rtol=1e-12)
    np.testing.assert_allclose(res[2].to_numpy(("d",)), wt.grad.numpy(), rtol=1e-12)
    only_w = grad(region, "y", seed="dy", wrt=("w",), names=names)
    assert len(list(walk(only_w.region))) < len(list(walk(full.region)))  # no tanh' or rename back for x
    res_w = interp.run_region(only_w.region, [interp.field(xv, ("t", "d")), interp.field(wv, ("d",)),
                                              interp.field(dy, ("s", "d"))])
    np.testing.assert_allclose(res_w[1].to_numpy(("d",)), wt.grad.numpy(), rtol=1e-12)


@pytest.mark.parametrize("with_tables", [False, True])
def test_the_gpt2_weight_joint_builds_and_plans(with_tables):
    """grad of the gpt2 zoo model's logits w.r.t. every weight (with or
    without the embedding tables, whose gradient comes through the take's
    adjoint, a scatter-add, plus the tied head's product): the joint plans
    into contraction, map-chain and row-statistics carves (the residue: the
    forward gather, the scatter-add and the softmax's bare row max), and its
    values equal torch autograd of the same forward in float64."""
    from collections import Counter

    from pdum_dsl_amd.tl.ir import walk

    m = zoo.gpt2(zoo.GPT2Config(t=16, d=64, nh=2, hk=32, m=128, layers=1, v=32), seed=3)
    pn = tuple(m.names[id(p)] for p in m.region.params)
    names = region_names(m.region, pn, ("logits",))
    wrt = tuple(n for n in pn if n not in (("ids",) if with_tables else ("ids", "wte", "wpe")))
    rg = grad(m.region, "logits", seed="dlogits", wrt=wrt, names=names)
    assert set(rg.grads) == set(wrt) and all(rg.grads[n] for n in wrt)
    assert any(n.op == "tl.scatter_add" for n in walk(rg.region)) == with_tables
    counts = Counter(c.group.template for c in plan_model(rg.region).carves)
    assert counts["contraction-epilogue"] > 0 and counts["map-chain"] > 0
    # the joint's values against torch autograd of the same forward (zoo.gpt2's ref, float64)
    inp = {k: torch.tensor(v) for k, v in m.inputs.items()}
    for nm in wrt:
        inp[nm].requires_grad_(True)
    T, K = 16, 32

    def ln(x, g, b_):
        mu = x.mean(-1, keepdim=True)
        xc = x - mu
        return xc / torch.sqrt((xc * xc).mean(-1, keepdim=True) + 1e-5) * g + b_

    hh = inp["wte"][inp["ids"]] + inp["wpe"]
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))
    p = "h.0."
    a = ln(hh, inp[p + "attn.ln1g"], inp[p + "attn.ln1b"])
    q = torch.einsum("td,dhk->thk", a, inp[p + "attn.wq"]) / np.sqrt(K)
    kk = torch.einsum("sd,dhk->shk", a, inp[p + "attn.wk"])
    vv = torch.einsum("sd,dhk->shk", a, inp[p + "attn.wv"])
    sc = torch.where(mask[:, :, None], torch.einsum("thk,shk->tsh", q, kk), torch.tensor(-1e9, dtype=torch.float64))
    ctx = torch.einsum("tsh,shk->thk", torch.softmax(sc, dim=1), vv)
    hh = hh + torch.einsum("thk,hkd->td", ctx, inp[p + "attn.wo"])
    a2 = ln(hh, inp[p + "mlp.ln2g"], inp[p + "mlp.ln2b"])
    mm = torch.nn.functional.gelu(a2 @ inp[p + "mlp.w1"] + inp[p + "mlp.b1"], approximate="tanh")
    hh = hh + mm @ inp[p + "mlp.w2"] + inp[p + "mlp.b2"]
    logits = ln(hh, inp["lnfg"], inp["lnfb"]) @ inp["wte"].T
    y = m.region.body[-1].args[0]
    dl = np.random.default_rng(2).standard_normal(tuple(y.type.shape))
    dl_tv = np.transpose(dl, [y.type.names.index(n) for n in ("t", "v")])
    logits.backward(torch.tensor(dl_tv))
    vals = [rev.value(m.inputs[m.names[id(p_)]], p_.type) for p_ in m.region.params]
    res = rev.evaluate(rg.region, vals + [rev.value(dl, rg.region.params[-1].type)])
    by = dict(zip(rg.outputs, res))
    for nm in wrt:
        pt = next(p_ for p_ in m.region.params if m.names[id(p_)] == nm).type
        got = by[rg.grads[nm]].numpy()
        g_names = rg.nodes[rg.grads[nm]].type.names
        got = np.transpose(got, [g_names.index(d) for d in pt.names])
        want = inp[nm].grad.numpy()
        np.testing.assert_allclose(got, want, rtol=1e-7, atol=1e-9 * max(1.0, np.abs(want).max()), err_msg=nm)
