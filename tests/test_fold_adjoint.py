"""The adjoint of tl.fold (autodiff.py:411-605) on the CPU.

Pinned by closed forms that do not restate the rule: a linear recurrence's
gradient (powers of its coefficient), the logsumexp fold's gradient (the
softmax), and the hand-written flash tile (a fold over key blocks carrying
(m, den, o)) whose gradient must be plain causal attention's, taken by torch
autograd in float64; plus central differences. Both evaluators (the planner's
interpreter and the float64 oracle) run every joint, and the emitting fold
the adjoint is built from is checked against an explicit loop."""

import numpy as np
import pytest

torch = pytest.importorskip("torch")


def _eval_both(region, vals):
    from oracle import region_eval as rev
    from pdum_dsl_amd.tl.interp import run_region

    got_i = run_region(region, [v for v in vals])
    got_o = rev.evaluate(region, [rev.value(v.arr if hasattr(v, "arr") else v, p.type)
                                  for v, p in zip(vals, region.params)])
    return got_i, got_o


def _recurrence(T=7, I=3):
    """out = fold over t of s <- a * s + x[t], from s0: params a[i], s0[i], x[t, i]."""
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import Builder, Region, tensor_type

    b = Builder(OPS)
    pa = b.param(0, tensor_type(("i",), (I,)))
    ps0 = b.param(1, tensor_type(("i",), (I,)))
    px = b.param(2, tensor_type(("t", "i"), (T, I)))
    sb = Builder(OPS)
    s = sb.param(0, tensor_type(("i",), (I,)))
    a_ = sb.param(1, tensor_type(("i",), (I,)))
    x_ = sb.param(2, tensor_type(("i",), (I,)))
    nxt = sb.emit("tl.pointwise", sb.emit("tl.pointwise", a_, s, f="mul"), x_, f="add")
    step = Region(params=(s, a_, x_), body=(sb.emit("core.yield", nxt),))
    ar = b.emit("tl.repeat", pa, name="t", extent=T)
    out = b.emit("tl.fold", ps0, ar, px, regions=(step,), dim="t", state=("s",), element=("a", "x"),
                 out=("final", 0))
    return Region(params=(pa, ps0, px), body=(b.emit("core.yield", out),))


def test_the_emitting_fold_stacks_each_steps_extra_yield():
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.interp import Field, run_region
    from pdum_dsl_amd.tl.ir import Builder, Dim, Region

    T, I = 5, 2
    reg = _recurrence(T, I)
    fold = reg.body[-1].args[0]
    step = fold.regions[0]
    y = step.body[-1].args[0]
    sb = Builder(OPS)
    st2 = Region(params=step.params, body=(sb.emit("core.yield", sb.emit("core.tuple", y, y)),))
    b = Builder(OPS)
    em = b.emit("tl.fold", *fold.args, regions=(st2,), out=("emit",), dim="t", state=("s",), element=("a", "x"))
    assert em.type.names == ("i", "t") and em.type.dim("t") == Dim("t", 0, T)
    r2 = Region(params=reg.params, body=(b.emit("core.yield", em),))
    rng = np.random.default_rng(1)
    a, s0, x = rng.standard_normal(I), rng.standard_normal(I), rng.standard_normal((T, I))
    vals = [Field(a, reg.params[0].type.dims), Field(s0, reg.params[1].type.dims), Field(x, reg.params[2].type.dims)]
    got_i, got_o = _eval_both(r2, vals)
    want, s = np.zeros((I, T)), s0.copy()
    for t in range(T):
        s = a * s + x[t]
        want[:, t] = s
    np.testing.assert_allclose(got_i.to_numpy(("i", "t")), want, rtol=1e-14)
    np.testing.assert_allclose(got_o.t.numpy(), want, rtol=1e-14)
    assert run_region(reg, vals).to_numpy(("i",)) == pytest.approx(want[:, -1])


def test_a_linear_recurrences_gradient_is_its_closed_form():
    """L = <w, s_T>, s_t = a s_{t-1} + x_t (elementwise): dL/dx_t =
    w a^(T-1-t), dL/ds0 = w a^T, dL/da = w sum_t a^(T-1-t) s_{t-1}."""
    from pdum_dsl_amd.tl.autodiff import grad, region_names
    from pdum_dsl_amd.tl.interp import Field

    T, I = 7, 3
    reg = _recurrence(T, I)
    rg = grad(reg, "out", seed="w", names=region_names(reg, ("a", "s0", "x")))
    rng = np.random.default_rng(2)
    a, s0, x, w = (rng.uniform(0.5, 1.2, I), rng.standard_normal(I), rng.standard_normal((T, I)),
                   rng.standard_normal(I))
    vals = [Field(a, reg.params[0].type.dims), Field(s0, reg.params[1].type.dims), Field(x, reg.params[2].type.dims),
            Field(w, rg.region.params[-1].type.dims)]
    got_i, got_o = _eval_both(rg.region, vals)
    s = [s0]
    for t in range(T):
        s.append(a * s[-1] + x[t])
    dx = np.stack([w * a ** (T - 1 - t) for t in range(T)])
    ds0 = w * a ** T
    da = sum(w * a ** (T - 1 - t) * s[t] for t in range(T))
    out = dict(zip(rg.outputs, got_i))
    np.testing.assert_allclose(out["dx"].to_numpy(("t", "i")), dx, rtol=1e-12)
    np.testing.assert_allclose(out["ds0"].to_numpy(("i",)), ds0, rtol=1e-12)
    np.testing.assert_allclose(out["da"].to_numpy(("i",)), da, rtol=1e-12)
    out = dict(zip(rg.outputs, got_o))
    np.testing.assert_allclose(out["dx"].order(("t", "i")).numpy(), dx, rtol=1e-12)
    np.testing.assert_allclose(out["da"].order(("i",)).numpy(), da, rtol=1e-12)


def _logsumexp_fold(T=9, I=4):
    """(m, l) <- (max(m, x_t), l exp(m - max) + exp(x_t - max)); out = m + log l."""
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import Builder, Region, tensor_type

    b = Builder(OPS)
    px = b.param(0, tensor_type(("t", "i"), (T, I)))
    sb = Builder(OPS)
    m = sb.param(0, tensor_type(("i",), (I,)))
    ll = sb.param(1, tensor_type(("i",), (I,)))
    x_ = sb.param(2, tensor_type(("i",), (I,)))
    pw = lambda f, *xs: sb.emit("tl.pointwise", *xs, f=f)  # noqa: E731
    mn = pw("maximum", m, x_)
    ln = pw("add", pw("mul", ll, pw("exp", pw("sub", m, mn))), pw("exp", pw("sub", x_, mn)))
    step = Region(params=(m, ll, x_), body=(sb.emit("core.yield", sb.emit("core.tuple", mn, ln)),))
    m0 = b.emit("tl.const", value=-1e30, dims=(("i", I),))
    l0 = b.emit("tl.const", value=0.0, dims=(("i", I),))
    kw = dict(dim="t", state=("m", "l"), element=("x",))
    fm = b.emit("tl.fold", m0, l0, px, regions=(step,), out=("final", 0), **kw)
    fl = b.emit("tl.fold", m0, l0, px, regions=(step,), out=("final", 1), **kw)
    out = b.emit("tl.pointwise", fm, b.emit("tl.pointwise", fl, f="log"), f="add")
    return Region(params=(px,), body=(b.emit("core.yield", out),))


def test_the_logsumexp_folds_gradient_is_the_softmax():
    from pdum_dsl_amd.tl.autodiff import grad, region_names
    from pdum_dsl_amd.tl.interp import Field

    T, I = 9, 4
    reg = _logsumexp_fold(T, I)
    rg = grad(reg, "out", seed="w", names=region_names(reg, ("x",)))
    rng = np.random.default_rng(3)
    x, w = rng.standard_normal((T, I)) * 3, rng.standard_normal(I)
    vals = [Field(x, reg.params[0].type.dims), Field(w, rg.region.params[-1].type.dims)]
    got_i, got_o = _eval_both(rg.region, vals)
    sm = np.exp(x - x.max(0)) / np.exp(x - x.max(0)).sum(0)
    np.testing.assert_allclose(dict(zip(rg.outputs, got_i))["dx"].to_numpy(("t", "i")), w * sm, rtol=1e-12,
                               atol=1e-14)
    np.testing.assert_allclose(dict(zip(rg.outputs, got_o))["dx"].order(("t", "i")).numpy(), w * sm, rtol=1e-12,
                               atol=1e-14)


def test_the_flash_tiles_gradient_is_causal_attentions():
    """The flash tile (a fold over key blocks carrying (m, den, o), the max
    through its first-occurrence rule) differentiated by the fold adjoint
    equals torch autograd of softmax(q k^T + causal mask) v in float64, and
    central differences of the tile itself."""
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.autodiff import grad, region_names
    from pdum_dsl_amd.tl.interp import Field, run_region

    subj = zoo.flash_tile(T=6, E=3, OD=2, SI=2, seed=7)
    tile = subj.tile
    rg = grad(tile, "out", seed="dout", names=region_names(tile, ("q", "k", "v")))
    rng = np.random.default_rng(4)
    q, k, v = (f.arr for f in subj.inputs)
    dout = rng.standard_normal(tuple(tile.body[-1].args[0].type.shape))
    vals = [Field(q, tile.params[0].type.dims), Field(k, tile.params[1].type.dims),
            Field(v, tile.params[2].type.dims), Field(dout, rg.region.params[-1].type.dims)]
    got_i, got_o = _eval_both(rg.region, vals)
    gi, go = dict(zip(rg.outputs, got_i)), dict(zip(rg.outputs, got_o))

    qt, kt, vt = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (q, k, v))
    sc = qt @ kt.T
    causal = torch.ones(sc.shape, dtype=torch.bool).tril()
    o = torch.softmax(sc.masked_fill(~causal, -1e9), dim=-1) @ vt
    yn = tile.body[-1].args[0].type.names
    d_t = torch.tensor(Field(dout, rg.region.params[-1].type.dims).to_numpy(("t", "o")))
    o.backward(d_t)
    for nm, t_, names in (("dq", qt, ("t", "e")), ("dk", kt, ("s", "e")), ("dv", vt, ("s", "o"))):
        want = t_.grad.numpy()
        np.testing.assert_allclose(gi[nm].to_numpy(names), want, rtol=1e-10, atol=1e-12, err_msg=nm)
        np.testing.assert_allclose(go[nm].order(names).numpy(), want, rtol=1e-10, atol=1e-12, err_msg=nm)
    # central differences of the tile program itself, one coordinate of each input
    fwd = lambda qq, kk, vv: (run_region(tile, [Field(qq, tile.params[0].type.dims), Field(kk, tile.params[1].type.dims),  # noqa: E731
                                                Field(vv, tile.params[2].type.dims)]).to_numpy(yn) * dout).sum()
    h = 1e-6
    for nm, arr, idx, names in (("dq", q, (3, 1), ("t", "e")), ("dk", k, (2, 2), ("s", "e")),
                                ("dv", v, (4, 1), ("s", "o"))):
        up, dn = arr.copy(), arr.copy()
        up[idx] += h
        dn[idx] -= h
        args_up = [up if a is arr else a for a in (q, k, v)]
        args_dn = [dn if a is arr else a for a in (q, k, v)]
        fd = (fwd(*args_up) - fwd(*args_dn)) / (2 * h)
        assert gi[nm].to_numpy(names)[idx] == pytest.approx(fd, rel=1e-6, abs=1e-9), nm
