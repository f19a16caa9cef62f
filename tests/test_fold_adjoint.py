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


# ------------------------------------------------ checkpointed schedules


def test_revolve_costs_closed_forms():
    """One slot re-advances L - 1, L - 2, ... steps: L (L - 1) / 2 in all; a
    range that fits its slots is reversed as stored."""
    from pdum_dsl_amd.tl.autodiff import revolve_cost, revolve_split

    for L in range(1, 12):
        assert revolve_cost(1, L) == L * (L - 1) // 2
        for s in range(L, L + 3):
            assert revolve_cost(s, L) == 0
    assert revolve_cost(0, 3) == float("inf")
    for s, L in ((1, 5), (2, 6), (3, 10), (2, 9)):
        m = revolve_split(s, L)
        assert 1 <= m < L
        assert m + revolve_cost(s - 1, L - m) + revolve_cost(s, m) == revolve_cost(s, L)
    # more slots never cost more; more steps never cost less
    for s in range(1, 5):
        for L in range(2, 14):
            assert revolve_cost(s + 1, L) <= revolve_cost(s, L) <= revolve_cost(s, L + 1)


def _readvanced(region, dim, full):
    """Forward steps re-advanced in a joint: the extents of the folds that read
    their final state over a strict sub-range of the scan dim (checkpoint
    advances), counted once per distinct fold."""
    from pdum_dsl_amd.tl.ir import walk

    seen, total = set(), 0
    for nd in walk(region):
        if nd.op != "tl.fold" or nd.attr("dim") != dim or tuple(nd.attr("out"))[0] != "final":
            continue
        if tuple(nd.attr("state"))[0].startswith("fold.ct"):
            continue  # a reverse fold
        k = len(nd.attr("state"))
        ext = nd.args[k].type.dim(dim)
        if (ext.start, ext.stop) == (0, full):
            continue  # the forward fold itself
        key = (tuple(id(a) for a in nd.args), ext.start, ext.stop)
        if key in seen:
            continue
        seen.add(key)
        total += ext.size
    return total


@pytest.mark.parametrize("sched", [{"fold_segments": 7}, {"fold_segments": 2}, {"fold_slots": 1},
                                   {"fold_slots": 2}, {"fold_slots": 3}, {"fold_slots": 14}])
def test_checkpointed_schedules_give_the_one_segment_gradient(sched):
    """The linear recurrence and the logsumexp fold (two states) under every
    schedule: the same gradients as the one-segment adjoint to 1e-12, and the
    closed forms; revolve re-advances exactly revolve_cost steps."""
    from pdum_dsl_amd.tl.autodiff import grad, region_names, revolve_cost
    from pdum_dsl_amd.tl.interp import Field

    T, I = 14, 3
    reg = _recurrence(T, I)
    names = region_names(reg, ("a", "s0", "x"))
    one = grad(reg, "out", seed="w", names=names)
    chk = grad(reg, "out", None, "w", None, None, sched.get("fold_segments"), sched.get("fold_slots"), names=names)
    rng = np.random.default_rng(5)
    a, s0, x, w = (rng.uniform(0.5, 1.1, I), rng.standard_normal(I), rng.standard_normal((T, I)),
                   rng.standard_normal(I))
    vals = [Field(a, reg.params[0].type.dims), Field(s0, reg.params[1].type.dims), Field(x, reg.params[2].type.dims),
            Field(w, one.region.params[-1].type.dims)]
    got1, _ = _eval_both(one.region, vals)
    gotc_i, gotc_o = _eval_both(chk.region, vals)
    d1, dci, dco = dict(zip(one.outputs, got1)), dict(zip(chk.outputs, gotc_i)), dict(zip(chk.outputs, gotc_o))
    dx = np.stack([w * a ** (T - 1 - t) for t in range(T)])
    for nm, names_ in (("dx", ("t", "i")), ("da", ("i",)), ("ds0", ("i",))):
        np.testing.assert_allclose(dci[nm].to_numpy(names_), d1[nm].to_numpy(names_), rtol=1e-12, atol=1e-13)
        np.testing.assert_allclose(dco[nm].order(names_).numpy(), d1[nm].to_numpy(names_), rtol=1e-12, atol=1e-13)
    np.testing.assert_allclose(dci["dx"].to_numpy(("t", "i")), dx, rtol=1e-12)
    if "fold_slots" in sched:
        assert _readvanced(chk.region, "t", T) == revolve_cost(sched["fold_slots"], T)
    if sched.get("fold_slots") == 14:  # enough slots: the stored trajectory, as one segment
        assert chk.region.key == one.region.key

    reg2 = _logsumexp_fold(12, 4)
    n2 = region_names(reg2, ("x",))
    segs = sched.get("fold_segments")
    segs = None if segs is not None and 12 % segs else segs
    r1 = grad(reg2, "out", seed="w", names=n2)
    rc = grad(reg2, "out", None, "w", None, None, segs, sched.get("fold_slots"), names=n2)
    x2, w2 = rng.standard_normal((12, 4)) * 3, rng.standard_normal(4)
    v2 = [Field(x2, reg2.params[0].type.dims), Field(w2, r1.region.params[-1].type.dims)]
    sm = np.exp(x2 - x2.max(0)) / np.exp(x2 - x2.max(0)).sum(0)
    g_i, g_o = _eval_both(rc.region, v2)
    np.testing.assert_allclose(dict(zip(rc.outputs, g_i))["dx"].to_numpy(("t", "i")), w2 * sm, rtol=1e-12,
                               atol=1e-14)
    np.testing.assert_allclose(dict(zip(rc.outputs, g_o))["dx"].order(("t", "i")).numpy(), w2 * sm, rtol=1e-12,
                               atol=1e-14)


def test_uniform_segments_must_divide_the_extent():
    from pdum_dsl_amd.tl.autodiff import grad, region_names

    reg = _recurrence(7, 2)
    with pytest.raises(ValueError, match="must divide the fold extent"):
        grad(reg, "out", None, "w", None, None, 3, None, names=region_names(reg, ("a", "s0", "x")))


def test_the_flash_tile_under_revolve_matches_one_segment():
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.autodiff import grad, region_names
    from pdum_dsl_amd.tl.interp import Field

    subj = zoo.flash_tile(T=8, E=3, OD=2, SI=2, seed=9)
    tile = subj.tile
    nm = region_names(tile, ("q", "k", "v"))
    one = grad(tile, "out", seed="dout", names=nm)
    rev = grad(tile, "out", None, "dout", None, None, None, 2, names=nm)
    rng = np.random.default_rng(6)
    q, k, v = (f.arr for f in subj.inputs)
    dout = rng.standard_normal(tuple(tile.body[-1].args[0].type.shape))
    vals = [Field(q, tile.params[0].type.dims), Field(k, tile.params[1].type.dims),
            Field(v, tile.params[2].type.dims), Field(dout, one.region.params[-1].type.dims)]
    g1, _ = _eval_both(one.region, vals)
    gr, _ = _eval_both(rev.region, vals)
    d1, dr = dict(zip(one.outputs, g1)), dict(zip(rev.outputs, gr))
    for nm_, names in (("dq", ("t", "e")), ("dk", ("s", "e")), ("dv", ("s", "o"))):
        np.testing.assert_allclose(dr[nm_].to_numpy(names), d1[nm_].to_numpy(names), rtol=1e-11, atol=1e-13)
