"""grad's signature and its switch (CPU).

The reference's ``grad(region, target, inputs, seed, wrt, target_unit,
fold_segments, fold_slots, *, names)`` (packages/tensorlib/src/pdum/tl/
autodiff.py:102-113) is called positionally by some callers; the argument
checks follow autodiff.py:181-187. The softmax shift-invariance rewrite is on
by default; with it off the joint routes the softmax max's cotangent through
the first-occurrence adjoint (autodiff.py:635-665) and carries its tl.scan,
and both joints evaluate to the closed-form gradients."""

import numpy as np
import pytest

from oracle import closed_forms as cf
from pdum_dsl_amd.tl import interp, zoo
from pdum_dsl_amd.tl.autodiff import grad, region_names


def _subj():
    return zoo.attention(T=7, S=7, E=4, OD=3, mask="causal", seed=5)


def _names(subj):
    return region_names(subj.region, ("q", "k", "v"), ("out",))


def _ops(region):
    seen, out, stack = set(), [], [n for n in region.body]
    while stack:
        n = stack.pop()
        if id(n) in seen:
            continue
        seen.add(id(n))
        out.append(n.op)
        stack.extend(n.args)
        for r in n.regions:
            stack.extend(r.body)
    return out


def test_a_positional_call_in_the_reference_order_builds_the_keyword_joint():
    subj = _subj()
    kw = grad(subj.region, "out", seed="dO", wrt=("q", "k"), names=_names(subj))
    pos = grad(subj.region, "out", {}, "dO", ("q", "k"), None, None, None, names=_names(subj))
    assert pos.outputs == kw.outputs == ("out", "dq", "dk")
    assert pos.region.key == kw.region.key


def test_a_seed_in_the_third_slot_is_refused_as_inputs():
    subj = _subj()
    with pytest.raises(TypeError, match="inputs must be a dict"):
        grad(subj.region, "out", "dO", names=_names(subj))


def test_fold_schedule_arguments_are_checked_like_the_reference():
    subj = _subj()
    nm = _names(subj)
    with pytest.raises(ValueError, match="not both"):
        grad(subj.region, "out", None, "dO", None, None, 2, 3, names=nm)
    with pytest.raises(ValueError, match="fold_slots must be >= 1"):
        grad(subj.region, "out", None, "dO", fold_slots=0, names=nm)
    # a region without folds: every schedule builds the one-segment joint
    plain = grad(subj.region, "out", seed="dO", names=nm).region.key
    assert grad(subj.region, "out", None, "dO", fold_segments=4, names=nm).region.key == plain
    assert grad(subj.region, "out", None, "dO", fold_slots=2, names=nm).region.key == plain
    with pytest.raises(NotImplementedError, match="target_unit"):
        grad(subj.region, "out", None, "dO", None, "m", names=nm)
    one = grad(subj.region, "out", None, "dO", fold_segments=1, names=nm)
    assert one.region.key == grad(subj.region, "out", seed="dO", names=nm).region.key


def test_the_switch_reproduces_the_reference_joint_with_its_scan():
    subj = _subj()
    nm = _names(subj)
    rewritten = grad(subj.region, "out", seed="dO", names=nm)
    ref = grad(subj.region, "out", seed="dO", names=nm, shift_invariant_softmax=False)
    assert "tl.scan" not in _ops(rewritten.region)
    assert "tl.scan" in _ops(ref.region)
    dO = np.random.default_rng(2).standard_normal((7, 3))
    q, k, v = subj.numpy_inputs()
    want = cf.attention_bwd(q, k, v, dO, scale=1.0, band=(None, 0))
    for rg in (rewritten, ref):
        res = interp.run_region(rg.region, subj.inputs + [interp.field(dO, ("t", "o"))])
        got = [res[1].to_numpy(("t", "e")), res[2].to_numpy(("s", "e")), res[3].to_numpy(("s", "o"))]
        for g, w in zip(got, want):
            np.testing.assert_allclose(g, w, rtol=1e-9, atol=1e-12)
