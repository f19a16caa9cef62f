"""The anchor-and-absorb partitioner on gpt2 (CPU), restating the
reference's packages/tensorlib/tests/test_partition.py:15-121: gpt2 carves
into recognized groups with the same counts, the carved plan executes to the
model's own output bit for bit (group boundaries are only materialized
tensors), repeated layers share kernels and analysis facts, and the
embedding gather is the named red residue."""

from collections import Counter

import numpy as np

from oracle import region_eval as rev
from pdum_dsl_amd.tl import analysis as A
from pdum_dsl_amd.tl import interp, zoo
from pdum_dsl_amd.tl.dialect import OPS
from pdum_dsl_amd.tl.ir import Builder, Region
from pdum_dsl_amd.tl.partition import carve_model, plan_model


def _execute(plan, model):
    """The reference's plan executor (test_partition.py:15-37): a worklist
    over carves; free views (renames) at the edges are resolved from their
    sources; red carves run through the interpreter too (the reference's
    doctrine for red groups)."""
    vals = {id(p): interp.field(model.inputs[model.names[id(p)]], p.type.names) for p in model.region.params}
    pending = [c for c in plan.carves if c.root is not None]
    while pending:
        for c in pending:
            for b in c.bounds:
                if id(b) not in vals and b.op == "tl.rename" and id(b.args[0]) in vals:
                    bb = Builder(OPS)
                    pp = bb.param(0, b.args[0].type)
                    r = Region(params=(pp,), body=(bb.emit("core.yield", bb.emit(b.op, pp, **dict(b.attrs))),))
                    vals[id(b)] = interp.run_region(r, [vals[id(b.args[0])]])
            if all(id(b) in vals for b in c.bounds):
                vals[id(c.root)] = interp.run_region(c.kernel, [vals[id(b)] for b in c.bounds])
                pending.remove(c)
                break
        else:
            raise AssertionError("plan stalled: unresolvable boundary")
    return vals


def test_gpt2_carves_into_recognized_groups():
    plan = plan_model(zoo.gpt2().region)
    by = Counter(c.group.template for c in plan.carves)
    assert by["contraction-epilogue"] == 15  # q, k, v, pv, wo, w1, w2 per block + the head
    assert by["row-normalization"] == 2  # the score contractions dissolve into the softmax claims
    assert by["row-statistics"] == 5
    assert by["map-chain"] == 0  # the mask forests travel with the scores
    assert plan.coverage() > 0.9
    reasons = " ".join(c.group.reason for c in plan.carves if c.group.confidence == "red")
    assert "tl.take" in reasons


def test_the_carved_plan_executes_to_the_models_output():
    m = zoo.gpt2()
    plan = plan_model(m.region)
    vals = _execute(plan, m)
    root = m.region.body[-1].args[0]
    want = interp.run_region(m.region, [interp.field(v, p.type.names) for v, p in zip(m.values(), m.region.params)])
    np.testing.assert_array_equal(vals[id(root)].to_numpy(m.order), want.to_numpy(m.order))
    np.testing.assert_allclose(want.to_numpy(m.order), m.ref(m.inputs), rtol=1e-12, atol=1e-12)
    # and the oracle's own evaluator agrees with the numpy denotation
    got = rev.evaluate(m.region, [rev.value(v, p.type) for v, p in zip(m.values(), m.region.params)])
    np.testing.assert_allclose(got.numpy(m.order), m.ref(m.inputs), rtol=1e-12, atol=1e-12)


def test_repeated_layers_share_kernels_and_analysis():
    m = zoo.gpt2()
    plan = plan_model(m.region)
    rooted = [c for c in plan.carves if c.root is not None]
    assert plan.distinct_kernels() < len(rooted)
    keys = Counter(c.kernel.key for c in plan.carves if c.group.confidence != "red")
    assert max(keys.values()) >= 2
    with A.no_reanalysis():  # a warm re-plan certifies nothing
        again = plan_model(m.region)
    assert again.coverage() == plan.coverage()


def test_the_rowstat_row_claims_every_layernorm_once():
    plan = plan_model(zoo.gpt2().region)
    rs = [c for c in plan.carves if c.group.template == "row-statistics"]
    assert len(rs) == 5
    assert len({c.kernel.key for c in rs}) == 1
    assert rs[0].group.certificate.verdict == "proved-exact"


def test_the_softmax_carve_rederives_its_scores_and_the_mlp_chain_rides_into_w2():
    """The carves the device executor binds: the softmax claim holds the score
    contraction and its mask (dissolved). w1's root has two consumers (the bias
    add and the bias's broadcast, whose lattice it is), so its epilogue walk
    stops at once and the bias + gelu chain is absorbed UP into w2's claim as
    a prologue, with both residual adds as w2's epilogue. wo contracts over
    two dims with the residual add."""
    plan = plan_model(zoo.gpt2().region)
    sm = [c for c in plan.carves if c.group.template == "row-normalization"][0]
    ops = Counter(n.op for n in _nodes(sm.kernel))
    assert ops["tl.reduce"] == 3 and ops["tl.iota"] == 2
    ce = [c for c in plan.carves if c.group.template == "contraction-epilogue"]
    fs = Counter(tuple(sorted(n.attr("f") for n in _nodes(c.kernel) if n.op == "tl.pointwise")) for c in ce)
    assert fs[("add", "add", "add", "mul", "zoo.gelu")] == 2  # w2: gelu(u + b1) prologue, + h + b2
    assert fs[("mul", "mul")] == 2  # q: the score scale as epilogue
    two_dim = [c for c in ce if any(n.op == "tl.reduce" and len(n.attr("dims")) == 2 for n in _nodes(c.kernel))]
    assert len(two_dim) == 2  # wo, per block


def test_carving_is_deterministic_and_claims_are_disjoint():
    m = zoo.gpt2(zoo.GPT2Config(layers=3))
    claims, interior, travel = carve_model(m.region)
    owned = Counter(i for _r, mem, _a in claims for i, n in mem.items()
                    if n.op not in ("core.const", "tl.const", "tl.rename", "tl.repeat_like", "tl.repeat")
                    and i not in travel)
    assert all(v == 1 for v in owned.values())  # no interior value is computed by two claims
    a, b = plan_model(m.region), plan_model(m.region)
    assert [c.kernel.key for c in a.carves] == [c.kernel.key for c in b.carves]
    by = Counter(c.group.template for c in a.carves)
    assert by["contraction-epilogue"] == 22 and by["row-statistics"] == 7 and by["row-normalization"] == 3


def _nodes(region):
    from pdum_dsl_amd.tl.ir import walk

    return walk(region)


def test_the_executor_finds_the_attention_chains_of_each_carve_form():
    """Host-side: the softmax + PV carve pairs the executor launches as one
    flash forward, per traffic-gate form, and the 16-bit width rule."""
    from pdum_dsl_amd.executor import _attention_chains
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.partition import plan_model

    def chains(t, hk, dtype):
        m = zoo.gpt2(zoo.GPT2Config(t=t, d=128, nh=128 // hk, hk=hk, m=512, layers=1, v=64), seed=3)
        return _attention_chains(list(plan_model(m.region).carves), m.region, dtype)

    for t, drop, made in ((64, 2, [None] * 3), (128, 1, [None] * 3), (256, 1, ["m"] * 3)):
        (ch,) = chains(t, 64, "bf16")
        assert len(ch.drop) == drop and (ch.t, ch.s, ch.e, ch.o, ch.heads) == ("t", "s", "hk", "hk", ("nh",))
        assert ch.band == ("band", None, 0) and ch.fill <= -1e6
        assert [None if x is None else "m" for x in ch.sources] == made
        if made[0] is None:
            assert len(ch.bounds) == 3 and ch.merged is None
        else:  # one activation projected by three weight params, q scaled by 1/sqrt(64)
            act, ws, dn, scale = ch.merged
            assert act.type.names == ("t", "d") and dn == "d" and scale == 0.125
            assert all(w.op == "core.param" for w in ws) and ch.bounds == (act,) + ws
    assert chains(128, 32, "bf16") == [] and len(chains(128, 32, "f32")) == 1  # 16-bit flash wants e in {64, 128}
