"""The planning interface on the CPU: the reference's known-answer battery
for the template rows this backend serves, restated against
pdum_dsl_amd.tl (packages/tensorlib/tests/test_fusion.py:45-173,
test_launch.py:13-117, test_tile_tier.py) plus the HIP seat's recognizers
and refusal law (conformance/triton_tile.py:216-226, :617-621)."""

import numpy as np
import pytest

from pdum_dsl_amd import hip_tile as H
from pdum_dsl_amd.tl import fusion, zoo
from pdum_dsl_amd.tl.dialect import OPS
from pdum_dsl_amd.tl.interp import run_region
from pdum_dsl_amd.tl.ir import Builder, Region, tensor_type, walk_deep
from pdum_dsl_amd.tl.launch import TileLevel, TileMachine, feasible, fit_affine, propose, tri_eval

# the 4090's opt-in shared-memory limit, the reference's machine-table row (test_launch.py:10)
SHARED_4090 = TileMachine((TileLevel("shared", 128, 101376),))


def _folds(region):
    return sum(1 for n in walk_deep(region) if n.op == "tl.fold")


def test_pick_ki():
    assert fusion.pick_ki(8) == 4 and fusion.pick_ki(6) == 3 and fusion.pick_ki(4096) == 32
    assert fusion.pick_ki(2048) == 32 and fusion.pick_ki(256) == 32 and fusion.pick_ki(1) == 1


def test_the_flash_composition_is_recognized_and_licensed():
    f = zoo.flash_tile()
    (g,) = fusion.plan_region(f.region).groups
    assert g.template == "flash"
    assert g.certificate.verdict == "licensed-differential"
    assert g.certificate.licenses == ("flash.online-softmax",)
    assert g.certificate.families == ("gaussian", "wide-scores", "dominant-key")
    assert _folds(g.kernel) == 2  # the o and den finals share one step
    got = run_region(g.kernel, f.inputs).to_numpy(("t", "o"))
    want = run_region(f.region, f.inputs).to_numpy(("t", "o"))
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)


def test_the_hand_written_tile_matches_its_twin():
    f = zoo.flash_tile()
    got = run_region(f.tile, f.inputs).to_numpy(("t", "o"))
    np.testing.assert_allclose(got, f.oracle(f.numpy_inputs()), rtol=1e-6, atol=1e-7)


def test_the_artifact_variant_yields_out_m_den():
    a = zoo.attention(T=8, E=3, OD=2, artifacts=True)
    (g,) = fusion.plan_region(a.region).groups
    assert g.template == "flash" and g.artifacts == ("m", "den") and _folds(g.kernel) == 3
    got = run_region(g.kernel, a.inputs)
    want = run_region(a.region, a.inputs)
    for x, y in zip(got, want):
        np.testing.assert_allclose(x.to_numpy(y.names), y.arr, rtol=1e-6, atol=1e-7)


def test_bare_row_normalization_stages_its_rows():
    s = zoo.row_softmax()
    (g,) = fusion.plan_region(s.region).groups
    assert g.template == "row-normalization"
    assert g.certificate.verdict == "proved-exact"
    assert any(n.op == "tl.stage" for n in walk_deep(g.kernel))
    np.testing.assert_array_equal(run_region(g.kernel, s.inputs).arr, run_region(s.region, s.inputs).arr)


def test_layernorm_claims_as_row_statistics():
    for affine in (False, True):
        ln = zoo.layernorm(affine=affine)
        (g,) = fusion.plan_region(ln.region).groups
        assert g.template == "row-statistics" and g.certificate.verdict == "proved-exact"


def test_unrecognized_work_refuses_loudly():
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "e"), (4, 3)))
    top = b.emit("tl.argtopk", x, dim="e", k=2, k_name="c")
    plan = fusion.plan_region(Region(params=(x,), body=(b.emit("core.yield", top),)))
    (g,) = plan.groups
    assert (g.template, g.confidence, g.kernel) == ("uncompiled", "red", None)
    assert "tl.argtopk" in g.reason and "no recognized schedule" in g.reason


def test_certification_caps_at_the_program_scale():
    f = zoo.flash_tile(T=4096, E=16, OD=16, SI=2)
    (g,) = fusion.plan_region(f.region).groups
    assert g.template == "flash" and g.confidence == "yellow" and g.certificate is not None


# ------------------------------------------------------------------ launch


def test_the_measured_crash_is_now_a_computed_refusal():
    region = zoo.flash_tile(T=512, E=64, OD=64, SI=32).tile
    ok_full, fp_full = feasible(region, (("t", 512),), SHARED_4090)
    ok_32, fp_32 = feasible(region, (("t", 32),), SHARED_4090)
    assert not ok_full and fp_full > SHARED_4090.tightest()
    assert ok_32 and fp_32 <= SHARED_4090.tightest()
    assert (fp_full, fp_32) == (303104, 49664)


def test_the_ladder_is_smallest_first_and_all_feasible():
    region = zoo.flash_tile(T=512, E=64, OD=64, SI=32).tile
    cands = propose(region, SHARED_4090, floor=1024)
    tiles = [dict(c)["t"] for c in cands if "t" in dict(c)]
    assert tiles == sorted(tiles) and tiles[0] == 16
    assert all(feasible(region, c, SHARED_4090)[0] for c in cands)
    assert 512 not in tiles and 256 not in tiles


def test_plan_region_attaches_the_analytic_default_and_the_prune():
    f = zoo.flash_tile(T=128, E=32, OD=32, SI=2)
    (g0,) = fusion.plan_region(f.region).groups
    assert g0.launch == ()
    (g,) = fusion.plan_region(f.region, machine=SHARED_4090).groups
    assert g.template == "flash" and g.launch and g.launch[0][0] == "t"
    assert g.prune == (("so", (0, 0, 1), (1, 1, 1)),)


def test_the_emptiness_engine_is_three_valued_and_sound():
    mask = fusion.match_flash(zoo.flash_tile().region)["mask"]  # le(iota_s, iota_t)
    assert tri_eval(mask, {"t": (0, 0), "s": (1, 5)}) == ("bool", "F")
    assert tri_eval(mask, {"t": (2, 3), "s": (0, 1)}) == ("bool", "T")
    assert tri_eval(mask, {"t": (2, 3), "s": (2, 4)}) == ("bool", "M")


def test_the_bound_fitter_is_exact_or_absent():
    assert fit_affine([5, 5, 5], 0, 8)[1] == 0
    assert fit_affine([1, 2, 3, 4], 0, 8) == (1, 1, 1)
    assert fit_affine([0, 0, 1, 2], 0, 8) == (-1, 1, 1)
    a, d, c = fit_affine([1, 1, 2, 2, 3, 3], 0, 8)
    assert [min(8, max(0, (a + d * g) // c)) for g in range(6)] == [1, 1, 2, 2, 3, 3]
    assert fit_affine([0, 3, 1, 2], 0, 8) is None


def test_prune_flash_derives_the_causal_bounds():
    naive = zoo.flash_tile(T=128, E=32, OD=32, SI=2).region
    assert fusion.prune_flash(naive, tile=32, si=32) == ((0, 0, 1), (1, 1, 1))
    lo, hi = fusion.prune_flash(naive, tile=16, si=32)
    assert lo == (0, 0, 1)
    assert [min(4, max(0, (hi[0] + hi[1] * g) // hi[2])) for g in range(8)] == [1, 1, 2, 2, 3, 3, 4, 4]


def test_a_fully_masked_row_refuses_pruning():
    region = zoo.attention(T=64, E=32, OD=32, mask="strict").region
    assert fusion.prune_flash(region, tile=16, si=16) is None


# --------------------------------------------------------------- HIP seat


@pytest.mark.parametrize(
    "mask,band",
    [("causal", ("band", None, 0)), ("strict", ("band", None, -1)), ("all", ("none",)),
     (("window", 3), ("band", -2, 0))],
)
def test_the_seat_binds_flash_tiles_and_their_mask_bands(mask, band):
    a = zoo.attention(T=16, E=4, OD=3, mask=mask)
    (g,) = fusion.plan_region(a.region).groups
    fb = H.recognize_flash(g.kernel)
    assert fb is not None and (fb["T"], fb["S"], fb["E"], fb["OD"], fb["si"]) == (16, 16, 4, 3, 8)
    assert H.mask_to_band(fb["mask"], fb["t"], fb["s"], 16, 16) == band


def test_the_seat_binds_the_hand_written_tile_and_the_row_templates():
    assert H.recognize_flash(zoo.flash_tile().tile) is not None
    (g,) = fusion.plan_region(zoo.row_softmax().region).groups
    assert H.recognize_softmax(g.kernel)["s"] == "s"
    (g,) = fusion.plan_region(zoo.layernorm().region).groups
    lb = H.recognize_layernorm(g.kernel)
    assert lb["feat"] == "d" and lb["eps"] == 1e-5 and lb["gamma"] is not None and lb["beta"] is not None


def test_the_seat_refuses_what_it_cannot_bind():
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "s"), (4, 6)))
    y = b.emit("tl.reduce", b.emit("tl.pointwise", x, f="tanh"), dims=("s",), f="prod")
    with pytest.raises(H.Untranslatable, match="no HIP binding"):
        H.compile_tile_hip(Region(params=(x,), body=(b.emit("core.yield", y),)))
    # a rowsum-shaped contraction binds the row-reduce kernel (no launch at bind time)
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "s"), (4, 64)))
    z = b.param(1, tensor_type(("t", "s"), (4, 64)))
    y = b.emit("tl.reduce", b.emit("tl.pointwise", x, z, f="mul"), dims=("s",), f="sum")
    (g,) = fusion.plan_region(Region(params=(x, z), body=(b.emit("core.yield", y),))).groups
    assert g.template == "contraction-epilogue" and dict(g.params)["shape"] == "rowsum"
    run = H.compile_tile_hip(g.kernel)
    assert run.source.startswith("hip:reduce_rows shape=rowsum rows=4 k=64")


def test_launching_a_carried_dim_refuses_with_the_dim_named():
    f = zoo.flash_tile(T=64, E=8, OD=8, SI=8)
    (g,) = fusion.plan_region(f.region).groups
    with pytest.raises(H.Untranslatable, match="'so'"):
        H.compile_tile_hip(g.kernel, (("so", 1),))
    with pytest.raises(H.Untranslatable, match="not an output dim"):
        H.compile_tile_hip(g.kernel, (("q", 4),))
