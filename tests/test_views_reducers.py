"""Window, stencil, decimate and diagonal views, round_to, composite reducers
and the emitting fold's adjoint (CPU).

The reference's ops (layout.py:669-771 window / decimate / diagonal,
guarded.py:463-520 stencil, compute.py:368-375 round_to, mdsl.py:221-261
composite reducers) and their adjoints (autodiff.py:335-400 composite
sweeps, :680-763 taps / decimate / diagonal, :843-845 round_to).

Pins, independent of the rules' own formulas: both interpreters against
numpy indexing written out per op; round_to against numpy's float16 /
float32 conversions and torch's bfloat16 conversion of float32 values; every
adjoint against torch autograd (float64) of the same computation written
with torch indexing; the flashsm reduce against causal softmax attention
and its gradient against torch autograd of that attention; a linear
recurrence reducer against its loop."""

import numpy as np
import pytest
import torch

from oracle import region_eval as rev
from pdum_dsl_amd.tl import interp, zoo
from pdum_dsl_amd.tl.autodiff import grad, region_names
from pdum_dsl_amd.tl.dialect import OPS, check_tier
from pdum_dsl_amd.tl.ir import Builder, Dim, Region, TensorType, tensor_type, walk
from pdum_dsl_amd.tl.reducers import defreducer

linrec = defreducer("test.linrec", state=2, element=2, lift=lambda a, b: (a, b),
                    combine=lambda l, r: (l[0] * r[0], r[0] * l[1] + r[1]), init=(1.0, 0.0),
                    project=lambda A, B: B)


def _both(region, vals):
    p = region.params
    a = interp.run_region(region, [interp.Field(np.asarray(v, dtype=np.float64), q.type.dims) for v, q in zip(vals, p)])
    b = rev.evaluate(region, [rev.value(v, q.type) for v, q in zip(vals, p)])
    return a, b


def _arr(v, names):
    return v.to_numpy(names) if isinstance(v, interp.Field) else v.numpy(names)


def _one(op_builder, shape, names, frames=None):
    b = Builder(OPS)
    tt = tensor_type(names, shape)
    if frames:
        tt = TensorType(tuple(Dim(n, lo, lo + s) for n, s, lo in zip(names, shape, frames)))
    px = b.param(0, tt)
    out = op_builder(b, px)
    return Region(params=(px,), body=(b.emit("core.yield", out),)), out


# ------------------------------------------------------------------ types


def test_view_types():
    b = Builder(OPS)
    x = b.param(0, tensor_type(("r", "x"), (2, 9)))
    w = b.emit("tl.window", x, name="x", k_name="j", k=(-1, 2), dilation=2)
    assert [(d.name, d.start, d.stop) for d in w.type.dims] == [("r", 0, 2), ("x", 2, 7), ("j", -1, 2)]
    st = b.emit("tl.stencil", x, name="x", k=(-2, 1))
    assert [(d.name, d.start, d.stop) for d in st.type.dims] == [("r", 0, 2), ("x", 0, 9), ("x_k", -2, 2)]
    dc = b.emit("tl.decimate", b.emit("tl.shift", x, deltas=(("x", 2),)), name="x", factor=3, phase=1)
    assert dc.type.dim("x").start == 1 and dc.type.dim("x").stop == 4  # cells 4, 7, 10 of [2, 11)
    y = b.param(1, tensor_type(("a", "r", "b"), (4, 2, 6)))
    dg = b.emit("tl.diagonal", b.emit("tl.shift", y, deltas=(("b", 1),)), parts=("b", "a"), name="z")
    assert [(d.name, d.start, d.stop) for d in dg.type.dims] == [("z", 1, 4), ("r", 0, 2)]
    with pytest.raises(TypeError, match="wider than"):
        b.emit("tl.window", x, name="x", k_name="j", k=11)
    with pytest.raises(TypeError, match="already exists"):
        b.emit("tl.window", x, name="x", k_name="r", k=2)
    with pytest.raises(TypeError, match="two or more"):
        b.emit("tl.diagonal", y, parts=("a",), name="z")
    with pytest.raises(TypeError, match="unknown encoding"):
        b.emit("tl.round_to", x, encoding="fp8")
    # the views are tile vocabulary (the reference's LAYOUT family); round_to is not
    check_tier(Region(params=(x,), body=(b.emit("core.yield", w),)))
    with pytest.raises(ValueError, match="host citizen"):
        check_tier(Region(params=(x,), body=(b.emit("core.yield", b.emit("tl.round_to", x, encoding="bf16")),)))


# ------------------------------------------------------------- evaluation


def test_views_on_both_interpreters_are_numpy_indexing():
    rng = np.random.default_rng(4)
    X = rng.standard_normal((2, 9))
    # window: x' in [2, 7), taps j in [-1, 2), reads x' + 2 j
    r, _ = _one(lambda b, p: b.emit("tl.window", p, name="x", k_name="j", k=(-1, 2), dilation=2), X.shape, ("r", "x"))
    want = np.stack([X[:, np.arange(2, 7) + 2 * j] for j in range(-1, 2)], axis=-1)
    for v in _both(r, [X]):
        np.testing.assert_array_equal(_arr(v, ("r", "x", "j")), want)
    # stencil: every x of [0, 9), taps -2..1 inclusive, -3.5 outside
    r, _ = _one(lambda b, p: b.emit("tl.stencil", p, name="x", k=(-2, 1), fill=-3.5), X.shape, ("r", "x"))
    want = np.full((2, 9, 4), -3.5)
    for xi in range(9):
        for jj, j in enumerate(range(-2, 2)):
            if 0 <= xi + j < 9:
                want[:, xi, jj] = X[:, xi + j]
    for v in _both(r, [X]):
        np.testing.assert_array_equal(_arr(v, ("r", "x", "x_k")), want)
    # decimate over x in [2, 11): cells 4, 7, 10 (phase 1 mod 3) -> j = 1, 2, 3
    r, _ = _one(lambda b, p: b.emit("tl.decimate", p, name="x", factor=3, phase=1), X.shape, ("r", "x"), (0, 2))
    for v in _both(r, [X]):
        np.testing.assert_array_equal(_arr(v, ("r", "x")), X[:, [2, 5, 8]])
    # diagonal of three parts with different frames, placed where the first sits
    Y = rng.standard_normal((4, 2, 6, 5))
    r, out = _one(lambda b, p: b.emit("tl.diagonal", p, parts=("c", "a", "b"), name="z"), Y.shape,
                  ("a", "r", "b", "c"), (0, 0, 1, 2))
    assert out.type.names == ("z", "r") and (out.type.dim("z").start, out.type.dim("z").stop) == (2, 4)
    want = np.stack([Y[z, :, z - 1, z - 2] for z in (2, 3)], axis=0)
    for v in _both(r, [Y]):
        np.testing.assert_array_equal(_arr(v, ("z", "r")), want)


def _bf16_via_torch(x):
    return torch.tensor(x, dtype=torch.float32).to(torch.bfloat16).to(torch.float64).numpy()


@pytest.mark.parametrize("enc", ["f32", "f16", "bf16"])
def test_round_to_is_the_format_conversion(enc):
    rng = np.random.default_rng(11)
    if enc == "f32":
        x = rng.standard_normal(4000) * np.exp2(rng.integers(-160, 120, 4000))
        x = np.concatenate([x, [0.0, -0.0, 1 + 2.0 ** -24, 1 + 3 * 2.0 ** -24, 2.0 ** -149 * 2.5, 2.0 ** -150]])
        want = x.astype(np.float32).astype(np.float64)
    elif enc == "f16":
        x = rng.standard_normal(4000) * np.exp2(rng.integers(-30, 15, 4000))
        x = np.concatenate([x, [1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 2.0 ** -24 * 0.5, 2.0 ** -24 * 1.5, 65519.0]])
        want = x.astype(np.float16).astype(np.float64)
    else:  # float32 values, where one rounding from float32 is the direct rounding
        x = (rng.standard_normal(4000) * np.exp2(rng.integers(-140, 120, 4000))).astype(np.float32).astype(np.float64)
        x = np.concatenate([x, [1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8, 2.0 ** -133 * 1.5, 2.0 ** -134]])
        want = _bf16_via_torch(x)
    r, _ = _one(lambda b, p: b.emit("tl.round_to", p, encoding=enc), x.shape, ("i",))
    for v in _both(r, [x]):
        np.testing.assert_array_equal(_arr(v, ("i",)), want)
    top = {"f32": 3.5e38, "f16": 65520.0, "bf16": 3.4e38}[enc]
    for bad in (np.array([top]), np.array([np.nan])):
        r, _ = _one(lambda b, p: b.emit("tl.round_to", p, encoding=enc), bad.shape, ("i",))
        with pytest.raises(ValueError, match="finite"):
            interp.run_region(r, [interp.field(bad, ("i",))])
        with pytest.raises(ValueError, match="finite"):
            rev.evaluate(r, [rev.value(bad, r.params[0].type)])


# --------------------------------------------------------------- adjoints


def _grad_check(region, arrays, names, torch_fn, tol=1e-12, **kw):
    """grad of <seed, out> on the numpy interpreter against torch autograd."""
    rng = np.random.default_rng(5)
    out_t = region.body[-1].args[0].type
    seed = rng.standard_normal(out_t.shape)
    g = grad(region, "out", seed="seed", names=region_names(region, names), **kw)
    vals = [interp.Field(np.asarray(a, dtype=np.float64), p.type.dims) for a, p in zip(arrays, region.params)]
    res = interp.run_region(g.region, vals + [interp.Field(seed, out_t.dims)])
    ts = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in arrays]
    (torch_fn(*ts) * torch.tensor(seed)).sum().backward()
    for nm, t, p in zip(names, ts, region.params):
        gn = g.grads[nm]
        got = np.zeros(t.shape) if gn is None else res[g.outputs.index(gn)].to_numpy(p.type.names)
        np.testing.assert_allclose(got, t.grad.numpy(), rtol=tol, atol=tol, err_msg=nm)
    return g


def test_window_and_stencil_adjoints_match_torch():
    rng = np.random.default_rng(6)
    X = rng.standard_normal((3, 11))
    r, _ = _one(lambda b, p: b.emit("tl.pointwise", b.emit("tl.window", p, name="x", k_name="j", k=(-1, 3),
                                                           dilation=2), f="sin"), X.shape, ("r", "x"))
    _grad_check(r, [X], ("x",), lambda x: torch.sin(torch.stack([x[:, torch.arange(2, 7) + 2 * j]
                                                                 for j in range(-1, 3)], dim=-1)))
    # stencil with dilation 3: taps past the domain read the fill and carry nothing back
    def tstencil(x):
        cols = []
        for j in range(-2, 3):
            idx = torch.arange(11) + 3 * j
            live = (idx >= 0) & (idx < 11)
            cols.append(torch.where(live, x[:, idx.clamp(0, 10)], torch.tensor(0.25, dtype=torch.float64)))
        return torch.exp(torch.stack(cols, dim=-1))
    r, _ = _one(lambda b, p: b.emit("tl.pointwise", b.emit("tl.stencil", p, name="x", k=(-2, 2), fill=0.25,
                                                            dilation=3), f="exp"), X.shape, ("r", "x"))
    _grad_check(r, [X], ("x",), tstencil)


def test_decimate_and_diagonal_adjoints_match_torch():
    rng = np.random.default_rng(7)
    X = rng.standard_normal((3, 11))  # x over [2, 13): phase 1 of 3 keeps 4, 7, 10 (domain not divisible)
    r, _ = _one(lambda b, p: b.emit("tl.pointwise", b.emit("tl.decimate", p, name="x", factor=3, phase=1), f="cos"),
                X.shape, ("r", "x"), (0, 2))
    _grad_check(r, [X], ("x",), lambda x: torch.cos(x[:, [2, 5, 8]]))
    r, _ = _one(lambda b, p: b.emit("tl.pointwise", b.emit("tl.decimate", p, name="x", factor=4), f="sin"),
                X.shape, ("r", "x"))
    _grad_check(r, [X], ("x",), lambda x: torch.sin(x[:, [0, 4, 8]]))
    Y = rng.standard_normal((4, 2, 6, 5))
    r, _ = _one(lambda b, p: b.emit("tl.pointwise", b.emit("tl.diagonal", p, parts=("c", "a", "b"), name="z"),
                                    f="tanh"), Y.shape, ("a", "r", "b", "c"), (0, 0, 1, 2))
    _grad_check(r, [Y], ("y",), lambda y: torch.tanh(torch.stack([y[z, :, z - 1, z - 2] for z in (2, 3)])))


@pytest.mark.parametrize("mode", ["straight_through", "zero"])
def test_round_to_gradient(mode):
    X = np.random.default_rng(8).standard_normal((3, 4))
    r, _ = _one(lambda b, p: b.emit("tl.pointwise", b.emit("tl.round_to", p, encoding="bf16", grad=mode), p,
                                    f="mul"), X.shape, ("r", "x"))
    rx = _bf16_via_torch(X)
    # d/dx [round(x) * x] = (1 or 0) * x + round(x)
    want = (X if mode == "straight_through" else 0.0) + rx
    g = grad(r, "out", seed="seed", names=region_names(r, ("x",)))
    res = interp.run_region(g.region, [interp.field(X, ("r", "x")), interp.field(np.ones((3, 4)), ("r", "x"))])
    np.testing.assert_allclose(res[1].to_numpy(("r", "x")), want, rtol=1e-15, atol=0)


# ------------------------------------------------------- composite reducers


def test_flashsm_reduce_is_causal_attention_on_both_interpreters():
    sj = zoo.flash_attention(T=7, E=3, OD=2, seed=2)
    want = sj.oracle(sj.numpy_inputs())
    for v in _both(sj.region, sj.numpy_inputs()):
        np.testing.assert_allclose(_arr(v, ("t", "o")), want, rtol=1e-13, atol=1e-14)


def _linrec_region(T=6, reduce=False):
    b = Builder(OPS)
    pa = b.param(0, tensor_type(("r", "t"), (3, T)))
    pb = b.param(1, tensor_type(("r", "t"), (3, T)))
    if reduce:
        out = b.emit("tl.reduce", pa, pb, dims=("t",), f=linrec.name)
    else:
        out = b.emit("tl.scan", pa, pb, dim="t", f=linrec.name)
    return Region(params=(pa, pb), body=(b.emit("core.yield", out),))


def _linrec_loop(a, b):
    h = [b[:, 0]]
    for t in range(1, a.shape[1]):
        h.append(a[:, t] * h[-1] + b[:, t])
    return h


def test_composite_scan_and_reduce_follow_the_sweep():
    rng = np.random.default_rng(9)
    A, B = rng.standard_normal((3, 6)), rng.standard_normal((3, 6))
    h = np.stack(_linrec_loop(A, B), axis=1)
    for v in _both(_linrec_region(), [A, B]):
        np.testing.assert_allclose(_arr(v, ("r", "t")), h, rtol=1e-14, atol=1e-14)
    for v in _both(_linrec_region(reduce=True), [A, B]):
        np.testing.assert_allclose(_arr(v, ("r",)), h[:, -1], rtol=1e-14, atol=1e-14)
    # an empty dim reduces to the projected identity state (B = 0)
    E = np.zeros((3, 0))
    for v in _both(_linrec_region(T=0, reduce=True), [E, E]):
        np.testing.assert_array_equal(_arr(v, ("r",)), np.zeros(3))


def test_composite_refusals():
    b = Builder(OPS)
    x = b.param(0, tensor_type(("r", "t"), (2, 3)))
    with pytest.raises(TypeError, match="consumes 2"):
        b.emit("tl.reduce", x, dims=("t",), f=linrec.name)
    with pytest.raises(TypeError, match="one dim at a time"):
        b.emit("tl.reduce", x, x, dims=("r", "t"), f=linrec.name)
    with pytest.raises(TypeError, match="scans forward"):
        b.emit("tl.scan", x, x, dim="t", f=linrec.name, reverse=True)
    with pytest.raises(TypeError, match="unknown reducer"):
        b.emit("tl.reduce", x, dims=("t",), f="no.such")


@pytest.mark.parametrize("sched", [{}, {"fold_slots": 2}, {"fold_segments": 3}])
def test_flashsm_gradient_is_attentions(sched):
    T = 7
    sj = zoo.flash_attention(T=T, E=3, OD=2, seed=3)
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))

    def attn(q, k, v):
        sc = torch.where(mask, q @ k.T, torch.tensor(-1e9, dtype=torch.float64))
        return torch.softmax(sc, dim=1) @ v

    g = _grad_check(sj.region, sj.numpy_inputs(), ("q", "k", "v"), attn, tol=1e-12, **sched)
    ops = {n.op for n in walk(g.region)}
    assert "tl.fold" in ops  # the reduce differentiated as its lowering


def test_composite_scan_gradient_is_the_loops():
    rng = np.random.default_rng(10)
    A, B = rng.standard_normal((3, 6)), rng.standard_normal((3, 6))
    _grad_check(_linrec_region(), [A, B], ("a", "b"), lambda a, b: torch.stack(_linrec_loop(a, b), dim=1))


def test_emitting_fold_adjoint():
    """A fold emitting each step's state, s' = s cos(x) + x^2 s0-free: the
    reverse sweep takes every emission's cotangent."""
    rng = np.random.default_rng(12)
    X, S0 = rng.standard_normal((2, 5)), rng.standard_normal(2)
    b = Builder(OPS)
    px = b.param(0, tensor_type(("r", "t"), X.shape))
    ps = b.param(1, tensor_type(("r",), S0.shape))
    sb = Builder(OPS)
    s_ = sb.param(("s", 0), ps.type)
    e_ = sb.param(("e", 0), ps.type)
    nxt = sb.emit("tl.pointwise", sb.emit("tl.pointwise", s_, sb.emit("tl.pointwise", e_, f="cos"), f="mul"),
                  sb.emit("tl.pointwise", e_, e_, f="mul"), f="add")
    em = sb.emit("tl.pointwise", nxt, f="tanh")
    step = Region(params=(s_, e_), body=(sb.emit("core.yield", sb.emit("core.tuple", nxt, em)),))
    out = b.emit("tl.fold", ps, px, regions=(step,), dim="t", state=("s",), element=("x",), out=("emit",))
    region = Region(params=(px, ps), body=(b.emit("core.yield", out),))

    def loop(x, s0):
        s, outs = s0, []
        for t in range(x.shape[1]):
            s = s * torch.cos(x[:, t]) + x[:, t] ** 2
            outs.append(torch.tanh(s))
        return torch.stack(outs, dim=1)

    for sched in ({}, {"fold_slots": 2}, {"fold_segments": 5}):
        _grad_check(region, [X, S0], ("x", "s0"), loop, **sched)


def test_the_flashsm_program_is_claimed_by_the_flash_row():
    """reduce(flashsm, ...) denotes causal attention, so the flash row claims
    it (the reference leaves this region to its reference runtime): one flash
    carve, certified like the softmax composition, whose generated tile
    program evaluates to the same values."""
    from pdum_dsl_amd.tl.fusion import match_flash, plan_region
    from pdum_dsl_amd.tl.partition import plan_model

    sj = zoo.flash_attention(T=16, E=4, OD=3, seed=5)
    fm = match_flash(sj.region)
    assert fm is not None and (fm["t"], fm["s"], fm["e"], fm["o"], fm["fill"]) == ("t", "s", "e", "o", -1e9)
    (g,) = plan_region(sj.region).groups
    assert (g.template, g.confidence) == ("flash", "yellow") and g.certificate.licenses == ("flash.online-softmax",)
    got = interp.run_region(g.kernel, sj.inputs)
    np.testing.assert_allclose(got.to_numpy(("t", "o")), sj.oracle(sj.numpy_inputs()), rtol=1e-12, atol=1e-13)
    assert [c.group.template for c in plan_model(sj.region).carves] == ["flash"]
    # a reducer of another name (even with the same parts) is not the flash row's
    other = defreducer("test.notflash", state=3, element=2, lift=lambda s, v: (s, 1.0, v),
                       combine=zoo._flash_combine, init=(-1e30, 0.0, 0.0), project=lambda m, d, o: o / d)
    b = Builder(OPS)
    y = sj.region.body[-1].args[0]
    alt = b.emit("tl.reduce", *y.args, dims=("s",), f=other.name)
    assert match_flash(Region(params=sj.region.params, body=(b.emit("core.yield", alt),))) is None


def _affine_region():
    """sin(window(x)) * decimate(shift(x)) + diagonal(y), over one lattice."""
    b = Builder(OPS)
    px = b.param(0, tensor_type(("r", "x"), (3, 30)))
    py = b.param(1, tensor_type(("p", "r", "q"), (12, 3, 14)))
    w = b.emit("tl.window", px, name="x", k_name="j", k=(-1, 3), dilation=2)  # x in [2, 26), j in [-1, 3)
    w = b.emit("tl.slice", w, ranges=(("x", (4, 12)),))
    d = b.emit("tl.decimate", b.emit("tl.shift", px, deltas=(("x", 5),)), name="x", factor=3, phase=2)  # x in [1, 11)
    d = b.emit("tl.slice", d, ranges=(("x", (4, 10)),))
    d = b.emit("tl.shift", d, deltas=(("x", 2),))  # [6, 12)
    d = b.emit("tl.slice", d, ranges=(("x", (6, 12)),))
    dg = b.emit("tl.diagonal", b.emit("tl.shift", py, deltas=(("q", -2),)), parts=("q", "p"), name="x")  # [0, 12)
    dg = b.emit("tl.rename", b.emit("tl.slice", dg, ranges=(("x", (6, 12)),)), mapping=(("r", "r"),))
    sw = b.emit("tl.slice", w, ranges=(("x", (6, 12)),))
    y = b.emit("tl.pointwise", b.emit("tl.pointwise", sw, f="sin"), b.emit("tl.repeat_like", d, sw), f="mul")
    y = b.emit("tl.pointwise", y, b.emit("tl.repeat_like", dg, sw), f="add")
    return Region(params=(px, py), body=(b.emit("core.yield", y),))


def test_affine_views_lower_to_strided_reads():
    """The elementwise program reads window / decimate / diagonal views in
    place: each slot's (strides, offset) over the stored tensor, applied as
    an as_strided view, gives the interpreter's values of that slot."""
    from numpy.lib.stride_tricks import as_strided

    from pdum_dsl_amd import ewprog
    from pdum_dsl_amd.tl.fusion import plan_region

    r = _affine_region()
    rng = np.random.default_rng(13)
    X, Y = rng.standard_normal((3, 30)), rng.standard_normal((12, 3, 14))
    y = r.body[-1].args[0]
    low = ewprog.lower(y, y.type.dims, {id(p): p for p in r.params}, allow_views=True)
    assert low.offset_reads() == len(low.operands) == 3
    store = {id(r.params[0]): X, id(r.params[1]): Y}
    for j, (slot, base) in enumerate(zip(low.operands, low.bases)):
        arr = store[id(base)]
        st, off = low.operand_view(j, dict(zip(base.type.names, (s // 8 for s in arr.strides))))
        assert off >= 0
        flat = np.ascontiguousarray(arr).reshape(-1)
        got = as_strided(flat[off:], shape=y.type.shape, strides=[8 * s for s in st])
        sub = Region(params=r.params, body=(Builder(OPS).emit("core.yield", slot),))
        want = interp.run_region(sub, [interp.Field(X, r.params[0].type.dims), interp.Field(Y, r.params[1].type.dims)])
        want = np.broadcast_to(want.to_numpy(tuple(n for n in y.type.names if n in want.names)).reshape(
            [y.type.dim(n).size if n in want.names else 1 for n in y.type.names]), y.type.shape)
        np.testing.assert_array_equal(got, want)
    (g,) = plan_region(r).groups
    assert (g.template, g.confidence) == ("map-chain", "yellow")


def _stencil_region(k, dil, fill=0.5):
    b = Builder(OPS)
    x = b.param(0, tensor_type(("r", "x"), (3, 40)))
    st = b.emit("tl.stencil", x, name="x", k=k, fill=fill, dilation=dil)
    return Region(params=(x,), body=(b.emit("core.yield", b.emit("tl.pointwise", st, f="exp")),))


@pytest.mark.parametrize("k,dil", [((-2, 1), 1), ((1, 3), 2), ((-3, -1), 3), ((0, 0), 1)])
def test_a_stencil_is_a_window_over_a_pad(k, dil):
    """The executor's device form of tl.stencil: a window over a pad of the
    fill, cut back to the domain. Bit-equal on the interpreter."""
    from pdum_dsl_amd.executor import _stencils_as_windows

    r = _stencil_region(k, dil)
    X = np.random.default_rng(16).standard_normal((3, 40))
    r2 = _stencils_as_windows(r)
    assert not any(n.op == "tl.stencil" for n in walk(r2))
    a = interp.run_region(r, [interp.field(X, ("r", "x"))]).to_numpy(("r", "x", "x_k"))
    b2 = interp.run_region(r2, [interp.field(X, ("r", "x"))]).to_numpy(("r", "x", "x_k"))
    np.testing.assert_array_equal(a, b2)


def _round_region(enc):
    b = Builder(OPS)
    x = b.param(0, tensor_type(("r", "c"), (64, 96)))
    y = b.emit("tl.pointwise", b.emit("tl.round_to", b.emit("tl.pointwise", x, x, f="mul"), encoding=enc), x, f="add")
    return Region(params=(x,), body=(b.emit("core.yield", y),))


def test_round_to_lowers_to_its_round_trip_instruction():
    from pdum_dsl_amd import ewprog

    for enc, opc in (("bf16", "RBF16"), ("f16", "RF16"), ("f32", "MAX")):
        r = _round_region(enc)
        y = r.body[-1].args[0]
        low = ewprog.lower(y, y.type.dims, {id(r.params[0]): r.params[0]}, allow_views=True)
        assert [i[0] for i in low.insns] == ["LOAD", "MUL", opc, "ADD"]
