"""Adjoints of the layout views (CPU): tl.shift, tl.slice, tl.pad, tl.flip,
tl.select, tl.split and tl.merge.

The reference's rules (autodiff.py:765-806): a shift's cotangent shifts
back, a slice's is padded with zeros to the operand's frames (and a pad's is
sliced), a flip's is flipped, a select's is repeated at the point and
padded, and split and merge exchange. tl.pad, tl.flip and tl.merge join the
dialect for them (layout.py's pad / flip / merge).

Pins, independent of the rules' own formulas: both interpreters against
numpy for the three new ops; every adjoint against torch autograd of the
same computation written with torch indexing (float64), including the zoo's
5-point stencil differentiated w.r.t. its halo."""

import numpy as np
import pytest
import torch

from oracle import region_eval as rev
from pdum_dsl_amd.tl import interp, zoo
from pdum_dsl_amd.tl.autodiff import grad, region_names
from pdum_dsl_amd.tl.dialect import OPS
from pdum_dsl_amd.tl.ir import Builder, Region, tensor_type, walk


def _both(region, vals):
    """The region on both interpreters (inputs in each param's dim order)."""
    p = region.params
    a = interp.run_region(region, [interp.field(v, q.type.names) for v, q in zip(vals, p)])
    b = rev.evaluate(region, [rev.value(v, q.type) for v, q in zip(vals, p)])
    return a, b


def test_pad_flip_merge_on_both_interpreters_are_numpy():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 4, 5))
    b = Builder(OPS)
    px = b.param(0, tensor_type(("a", "c", "d"), x.shape))
    sh = b.emit("tl.shift", px, deltas=(("c", 2),))  # c's frame [2, 6)
    pad = b.emit("tl.pad", sh, extents=(("c", (0, 9)), ("a", (-1, 3))), fill=1.5)
    flip = b.emit("tl.flip", px, name="c")
    merge = b.emit("tl.merge", px, parts=("d", "a"), name="m")  # parts apart and out of order
    region = Region(params=(px,), body=(b.emit("core.yield", b.emit("core.tuple", pad, flip, merge)),))
    assert tuple((d.name, d.start, d.stop) for d in pad.type.dims) == (("a", -1, 3), ("c", 0, 9), ("d", 0, 5))
    assert merge.type.names == ("c", "m") and merge.type.shape == (4, 15)
    want_pad = np.pad(x, ((1, 0), (2, 3), (0, 0)), constant_values=1.5)
    want_flip = x[:, ::-1, :]
    want_merge = np.transpose(x, (1, 2, 0)).reshape(4, 15)
    (a_pad, a_flip, a_merge), (b_pad, b_flip, b_merge) = _both(region, [x])
    for got, want in ((a_pad.to_numpy(), want_pad), (b_pad.numpy(), want_pad), (a_flip.to_numpy(), want_flip),
                      (b_flip.numpy(), want_flip), (a_merge.to_numpy(), want_merge), (b_merge.numpy(), want_merge)):
        np.testing.assert_array_equal(got, want)


def test_pad_and_merge_refuse_bad_frames():
    b = Builder(OPS)
    x = b.param(0, tensor_type(("a", "c"), (3, 4)))
    with pytest.raises(TypeError, match="does not contain"):
        b.emit("tl.pad", x, extents=(("c", (1, 9)),))
    with pytest.raises(TypeError, match="must start at 0"):
        b.emit("tl.merge", b.emit("tl.shift", x, deltas=(("a", 1),)), parts=("a", "c"), name="m")


def _joint_vs_torch(region, wrt, vals, torch_fn):
    """grad(region) seeded by a random cotangent on both interpreters, against
    torch autograd of ``torch_fn`` (float64 tensors in the params' dim order)."""
    names = region_names(region, tuple(f"p{i}" for i in range(len(region.params))), ("out",))
    rg = grad(region, "out", seed="dy", wrt=wrt, names=names)
    y = region.body[-1].args[0]
    dy = np.random.default_rng(9).standard_normal(tuple(y.type.shape))
    ts = [torch.tensor(v, requires_grad=True) for v in vals]
    out = torch_fn(*ts)
    assert tuple(out.shape) == tuple(y.type.shape)
    out.backward(torch.tensor(dy))
    a, b = _both(rg.region, list(vals) + [dy])
    by_a, by_b = dict(zip(rg.outputs, a)), dict(zip(rg.outputs, b))
    for nm in wrt:
        i = int(nm[1:])
        order = region.params[i].type.names
        want = ts[i].grad.numpy()
        np.testing.assert_allclose(by_a[rg.grads[nm]].to_numpy(order), want, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(by_b[rg.grads[nm]].numpy(order), want, rtol=1e-12, atol=1e-12)
    return rg


def test_the_stencil_adjoint_is_the_transposed_stencil():
    """grad of the zoo's 5-point update w.r.t. the halo: each tap's cotangent
    shifted back and zero-padded to the halo frame, summed."""
    s = zoo.stencil_tile(MI=6, NI=8, alpha=0.1, seed=17)
    u = s.inputs[0].arr

    def torch_stencil(t):
        lap = t[:-2, 1:-1] + t[2:, 1:-1] + t[1:-1, :-2] + t[1:-1, 2:] - 4 * t[1:-1, 1:-1]
        return t[1:-1, 1:-1] + 0.1 * lap

    rg = _joint_vs_torch(s.naive, ("p0",), [u], torch_stencil)
    ops = {n.op for n in walk(rg.region)}
    assert {"tl.pad", "tl.shift"} <= ops


def test_select_flip_pad_adjoints():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 6))
    w = rng.standard_normal((6,))
    b = Builder(OPS)
    px = b.param(0, tensor_type(("a", "c"), x.shape))
    pw = b.param(1, tensor_type(("c",), w.shape))
    sel = b.emit("tl.select", b.emit("tl.flip", px, name="c"), coords=(("a", 3),))
    padded = b.emit("tl.pad", b.emit("tl.slice", px, ranges=(("c", (1, 5)),)), extents=(("c", (0, 6)),), fill=2.0)
    y = b.emit("tl.pointwise", b.emit("tl.pointwise", sel, pw, f="mul"),
               b.emit("tl.reduce", b.emit("tl.pointwise", padded, padded, f="mul"), dims=("a",), f="sum"), f="add")
    region = Region(params=(px, pw), body=(b.emit("core.yield", y),))

    def torch_fn(tx, tw):
        inner = torch.nn.functional.pad(tx[:, 1:5], (1, 1), value=2.0)
        return torch.flip(tx, dims=(1,))[3] * tw + (inner * inner).sum(0)

    _joint_vs_torch(region, ("p0", "p1"), [x, w], torch_fn)


def test_split_merge_adjoints():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((12, 3))
    w = rng.standard_normal((4, 3, 3))
    b = Builder(OPS)
    px = b.param(0, tensor_type(("k", "r"), x.shape))
    pw = b.param(1, tensor_type(("ko", "ki", "r"), w.shape))
    sp = b.emit("tl.split", px, name="k", parts=(("ko", 4), ("ki", 3)))
    prod = b.emit("tl.pointwise", sp, pw, f="mul")
    mg = b.emit("tl.merge", prod, parts=("ki", "ko"), name="m")  # the transposed blocking
    y = b.emit("tl.pointwise", mg, mg, f="mul")
    region = Region(params=(px, pw), body=(b.emit("core.yield", y),))
    assert y.type.names == ("m", "r")

    def torch_fn(tx, tw):
        p = tx.reshape(4, 3, 3) * tw  # (ko, ki, r)
        m = p.permute(1, 0, 2).reshape(12, 3)
        return m * m

    _joint_vs_torch(region, ("p0", "p1"), [x, w], torch_fn)


def test_a_shift_with_offset_frames_sends_the_cotangent_back():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((7,))
    b = Builder(OPS)
    px = b.param(0, tensor_type(("t",), x.shape))
    a = b.emit("tl.slice", b.emit("tl.shift", px, deltas=(("t", 1),)), ranges=(("t", (1, 7)),))  # x[t - 1]
    c = b.emit("tl.slice", px, ranges=(("t", (1, 7)),))  # x[t]
    y = b.emit("tl.pointwise", a, c, f="mul")  # x[t - 1] x[t], t = 1..6
    region = Region(params=(px,), body=(b.emit("core.yield", y),))
    _joint_vs_torch(region, ("p0",), [x], lambda t: t[:-1] * t[1:])
