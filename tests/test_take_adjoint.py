"""tl.scatter_add and the gather's adjoint (CPU).

tl.scatter_add is the reference's take adjoint (packages/tensorlib/src/pdum/
tl/indexing.py:153-190, 223-259): the consumed idx dims are replaced by the
declared dim, every position p adds values[p] into row idx[p], duplicates
sum, rows nothing lands in are zero. ``grad`` sends a take's cotangent
through a scatter-add at the same indices and a scatter-add's through a take
(autodiff.py:846-856); indices carry no gradient.

Pins, each independent of the rules' own formulas: both interpreters against
numpy's add.at with duplicates and an offset frame; the take adjoint against
torch's embedding backward and a brute-force loop; the scatter-add adjoint
against finite differences."""

import numpy as np
import pytest
import torch

from oracle import region_eval as rev
from pdum_dsl_amd.tl import interp
from pdum_dsl_amd.tl.autodiff import grad, region_names
from pdum_dsl_amd.tl.dialect import OPS
from pdum_dsl_amd.tl.ir import Builder, Dim, Region, TensorType, tensor_type, walk


def _scatter_region(vshape, vnames, ishape, inames, dim, extent, over=None):
    b = Builder(OPS)
    v = b.param(0, tensor_type(vnames, vshape))
    i = b.param(1, tensor_type(inames, ishape))
    extra = {} if over is None else {"over": over}
    y = b.emit("tl.scatter_add", v, i, dim=dim, extent=extent, **extra)
    return Region(params=(v, i), body=(b.emit("core.yield", y),)), y


@pytest.mark.parametrize("layout", ["rows", "rest_first", "two_consumed"])
def test_scatter_add_on_both_interpreters_is_numpy_add_at(layout):
    rng = np.random.default_rng(4)
    if layout == "rows":  # values (t, d), idx (t) -> (v, d)
        vals, idx = rng.standard_normal((9, 5)), rng.integers(3, 10, size=9)
        region, y = _scatter_region((9, 5), ("t", "d"), (9,), ("t",), "v", (3, 10))
        want = np.zeros((7, 5))
        np.add.at(want, idx - 3, vals)
        order = ("v", "d")
    elif layout == "rest_first":  # values (d, t): the declared dim lands where t was
        vals, idx = rng.standard_normal((4, 11)), rng.integers(0, 6, size=11)
        region, y = _scatter_region((4, 11), ("d", "t"), (11,), ("t",), "v", 6)
        want = np.zeros((4, 6))
        for t in range(11):
            want[:, idx[t]] += vals[:, t]
        order = ("d", "v")
    else:  # idx (a, t) both consumed
        vals, idx = rng.standard_normal((3, 4, 2)), rng.integers(0, 5, size=(3, 4))
        region, y = _scatter_region((3, 4, 2), ("a", "t", "d"), (3, 4), ("a", "t"), "v", 5)
        want = np.zeros((5, 2))
        np.add.at(want, idx.reshape(-1), vals.reshape(12, 2))
        order = ("v", "d")
    assert y.type.names == order
    assert len(np.unique(idx)) < idx.size, "no duplicate indices drawn"
    p0, p1 = region.params
    got = interp.run_region(region, [interp.field(vals, p0.type.names), interp.field(idx, p1.type.names)])
    np.testing.assert_allclose(got.to_numpy(order), want, rtol=1e-14, atol=1e-14)
    got2 = rev.evaluate(region, [rev.value(vals, p0.type), rev.value(idx, p1.type)])
    np.testing.assert_allclose(got2.numpy(order), want, rtol=1e-14, atol=1e-14)


def test_scatter_add_refuses_misaligned_or_foreign_dims():
    b = Builder(OPS)
    v = b.param(0, tensor_type(("t", "d"), (9, 5)))
    with pytest.raises(TypeError, match="not a values dim"):
        b.emit("tl.scatter_add", v, b.param(1, tensor_type(("s",), (9,))), dim="v", extent=4)
    with pytest.raises(TypeError, match="does not align"):
        b.emit("tl.scatter_add", v, b.param(2, TensorType((Dim("t", 1, 10),))), dim="v", extent=4)
    with pytest.raises(TypeError, match="already a values dim"):
        b.emit("tl.scatter_add", v, b.param(3, tensor_type(("t",), (9,))), dim="d", extent=4)


def _gather_joint(V, D, T, seed):
    """loss-free joint of y = take(table, ids) * w (a weighted gather)."""
    b = Builder(OPS)
    table = b.param(0, tensor_type(("v", "d"), (V, D)))
    ids = b.param(1, tensor_type(("t",), (T,)))
    w = b.param(2, tensor_type(("t", "d"), (T, D)))
    y = b.emit("tl.pointwise", b.emit("tl.take", table, ids, dim="v"), w, f="mul")
    region = Region(params=(table, ids, w), body=(b.emit("core.yield", y),))
    rg = grad(region, "out", seed="dy", wrt=("table", "w"), names=region_names(region, ("table", "ids", "w")))
    rng = np.random.default_rng(seed)
    vals = [rng.standard_normal((V, D)), rng.integers(0, V - 2, size=T), rng.standard_normal((T, D)),
            rng.standard_normal((T, D))]
    return rg, vals


def test_the_take_adjoint_is_the_embedding_backward():
    V, D, T = 7, 4, 15
    rg, (tab, ids, w, dy) = _gather_joint(V, D, T, 5)
    assert len(np.unique(ids)) < T and len(np.unique(ids)) < V  # duplicates and never-gathered rows
    p = rg.region.params
    res = interp.run_region(rg.region, [interp.field(x, q.type.names) for x, q in zip((tab, ids, w, dy), p)])
    dtab = res[1].to_numpy(("v", "d"))
    want = np.zeros((V, D))
    for t in range(T):  # brute force: row ids[t] collects dy[t] * w[t]
        want[ids[t]] += dy[t] * w[t]
    np.testing.assert_allclose(dtab, want, rtol=1e-14, atol=1e-14)
    tt = torch.tensor(tab, requires_grad=True)
    (torch.nn.functional.embedding(torch.tensor(ids), tt) * torch.tensor(w)).backward(torch.tensor(dy))
    np.testing.assert_allclose(dtab, tt.grad.numpy(), rtol=1e-14, atol=1e-14)
    res2 = rev.evaluate(rg.region, [rev.value(x, q.type) for x, q in zip((tab, ids, w, dy), p)])
    np.testing.assert_allclose(res2[1].numpy(("v", "d")), want, rtol=1e-14, atol=1e-14)


def test_the_scatter_add_adjoint_matches_finite_differences():
    rng = np.random.default_rng(6)
    T, D, V = 8, 3, 5
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "d"), (T, D)))
    ids = b.param(1, tensor_type(("t",), (T,)))
    s = b.emit("tl.scatter_add", x, ids, dim="v", extent=V)
    y = b.emit("tl.pointwise", s, s, f="mul")  # nonlinear in the scatter's result
    region = Region(params=(x, ids), body=(b.emit("core.yield", y),))
    rg = grad(region, "out", seed="dy", wrt=("x",), names=region_names(region, ("x", "ids")))
    assert any(n.op == "tl.take" for n in walk(rg.region))
    xv, iv, dy = rng.standard_normal((T, D)), rng.integers(0, V, size=T), rng.standard_normal((V, D))
    p = rg.region.params
    got = interp.run_region(rg.region, [interp.field(a, q.type.names) for a, q in zip((xv, iv, dy), p)])[1]
    got = got.to_numpy(("t", "d"))

    def loss(arr):
        acc = np.zeros((V, D))
        np.add.at(acc, iv, arr)
        return float(np.sum(acc * acc * dy))

    fd = np.zeros_like(xv)
    for i in np.ndindex(xv.shape):
        e = np.zeros_like(xv)
        e[i] = 1e-6
        fd[i] = (loss(xv + e) - loss(xv - e)) / 2e-6
    np.testing.assert_allclose(got, fd, rtol=1e-6, atol=1e-8)
