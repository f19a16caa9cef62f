"""The stencil row (CPU): the reference's fusion.py:846-851 and
tests/test_fusion.py:73-99 restated. A map chain reading one param at two or
more distinct shifts has neighborhood reuse, so the planner stages that halo
once (proved-exact: erasing the stage gives the twin's key); a single shifted
read stays a map chain. Plus the layout views themselves and the element
program's offset reads."""

import numpy as np
import pytest

from oracle import region_eval as rev
from pdum_dsl_amd import ewprog
from pdum_dsl_amd.tl import fusion, interp, zoo
from pdum_dsl_amd.tl.dialect import OPS
from pdum_dsl_amd.tl.ir import Builder, Region, tensor_type, walk


def test_stencils_are_recognized_and_staged():
    st = zoo.stencil_tile()
    (g,) = fusion.plan_region(st.naive).groups
    assert g.template == "stencil"
    assert g.certificate.verdict == "proved-exact"
    assert dict(g.params)["staged"] == (0,)
    assert any(n.op == "tl.stage" for n in walk(g.kernel))
    got = interp.run_region(g.kernel, st.inputs).arr
    want = interp.run_region(st.naive, st.inputs).arr
    np.testing.assert_array_equal(got, want)
    np.testing.assert_allclose(want, st.oracle([st.inputs[0].arr]), rtol=0, atol=1e-14)
    # and the oracle's evaluator agrees with the closed form
    o = rev.evaluate(st.naive, [rev.value(st.inputs[0].arr, st.naive.params[0].type)])
    np.testing.assert_allclose(o.numpy(("x", "y")), st.oracle([st.inputs[0].arr]), rtol=0, atol=1e-14)


def test_reuse_free_chains_stay_map_chains():
    b = Builder(OPS)
    x = b.param(0, tensor_type(("x", "y"), (4, 6)))
    sh = b.emit("tl.shift", x, deltas=(("x", 1),))
    sl = b.emit("tl.slice", sh, ranges=(("x", (1, 5)),))
    region = Region(params=(x,), body=(b.emit("core.yield", b.emit("tl.pointwise", sl, f="exp")),))
    (g,) = fusion.plan_region(region).groups
    assert g.template == "map-chain"
    assert g.certificate.verdict == "proved-exact"


def test_shift_and_slice_types_and_values():
    b = Builder(OPS)
    x = b.param(0, tensor_type(("x", "y"), (4, 6)))
    sh = b.emit("tl.shift", x, deltas=(("x", -1), ("y", 2)))
    assert [(d.name, d.start, d.stop) for d in sh.type.dims] == [("x", -1, 3), ("y", 2, 8)]
    sl = b.emit("tl.slice", sh, ranges=(("x", (0, 2)), ("y", (3, 5))))
    assert [(d.name, d.start, d.stop) for d in sl.type.dims] == [("x", 0, 2), ("y", 3, 5)]
    with pytest.raises(TypeError, match="outside"):
        b.emit("tl.slice", sh, ranges=(("x", (3, 4)),))
    arr = np.arange(24.0).reshape(4, 6)
    region = Region(params=(x,), body=(b.emit("core.yield", sl),))
    got = interp.run_region(region, [interp.field(arr, ("x", "y"))]).arr
    # value at new coordinate c is the input's at c - delta: x in [0, 2) reads rows 1..2, y in [3, 5) reads cols 1..2
    np.testing.assert_array_equal(got, arr[1:3, 1:3])
    o = rev.evaluate(region, [rev.value(arr, x.type)])
    np.testing.assert_array_equal(o.numpy(("x", "y")), arr[1:3, 1:3])


def test_shifted_reads_lower_to_offset_views():
    """Each neighbor is one LOAD slot of the same param at its own element
    offset; applying those offsets by hand to the flat array reproduces the
    stencil (the arithmetic the kernels do, checked on the CPU)."""
    st = zoo.stencil_tile(MI=5, NI=7)
    y = st.naive.body[-1].args[0]
    p = st.naive.params[0]
    low = ewprog.lower(y, y.type.dims, {id(p): p}, allow_views=True)
    assert len(low.operands) == 5 and all(b is p for b in low.bases)
    u = st.inputs[0].arr
    flat = u.reshape(-1)
    offs = set()
    for j in range(5):
        strides, off = low.operand_view(j, {"x": u.shape[1], "y": 1})
        offs.add(off)
        ii, jj = np.meshgrid(np.arange(5), np.arange(7), indexing="ij")
        got = flat[off + ii * strides[0] + jj * strides[1]]
        node = low.operands[j]
        region = Region(params=(p,), body=(Builder(OPS).emit("core.yield", node),))
        np.testing.assert_array_equal(got, interp.run_region(region, st.inputs).arr)
    assert len(offs) == 5  # five distinct neighbors
    with pytest.raises(ewprog.Unlowerable):  # without the offset-aware caller, shifted reads refuse
        ewprog.lower(y, y.type.dims, {id(p): p})


def test_the_gemm_flagship_binds_to_the_contraction_kernel():
    from pdum_dsl_amd.hip_tile import recognize_contraction

    gt = zoo.gemm_tile()
    cb = recognize_contraction(gt.region)
    assert cb is not None and cb["K"] == 8 and (cb["m"], cb["n"], cb["rider"]) == ("mi", "ni", None)
    np.testing.assert_allclose(interp.run_region(gt.region, gt.inputs).to_numpy(("mi", "ni")),
                               gt.oracle([f.arr for f in gt.inputs]), rtol=1e-12)
