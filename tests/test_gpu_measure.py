"""Measurements on the device as ledger facts (the reference's
conformance/test_fusion_triton.py:87-117, "the first measurement greens the
group"), and the autotune-lite pick over the decode's split ladder."""

import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(autouse=True)
def _cold():
    from pdum_dsl_amd.tl import analysis as A

    A.clear(ledger_too=True)
    yield
    A.clear(ledger_too=True)


def test_the_first_measurement_greens_the_group(tmp_path):
    from pdum_dsl_amd import measure as M
    from pdum_dsl_amd.tl import analysis as A
    from pdum_dsl_amd.tl import fusion, zoo
    from pdum_dsl_amd.tl.launch import MI355X_SHARED

    machine = M.machine_name()
    assert machine == "gfx950"
    (g,) = fusion.plan_region(zoo.attention(T=256, E=64, OD=64).region, machine=MI355X_SHARED).groups
    green, fact = M.measured_green(g)
    assert (green.template, green.confidence) == ("flash", "green")
    assert fact.value["ms"] > 0 and fact.value["source"].startswith("hip:flash")
    with A.no_reanalysis():  # keyed identically: never measured twice
        assert M.measured_green(g)[1].key == fact.key
    path = tmp_path / "ledger.json"
    assert A.save_ledger(path) == 1
    A.clear(ledger_too=True)
    A.load_ledger(path)
    with A.no_reanalysis():  # across sessions too
        assert M.measured_green(g)[1].value == fact.value


def test_red_groups_have_nothing_to_measure():
    from pdum_dsl_amd import measure as M
    from pdum_dsl_amd.tl.fusion import Group

    with pytest.raises(ValueError, match="no kernel"):
        M.measured_green(Group("uncompiled", None, None, "red", reason="tl.argtopk"))


def test_decode_split_pick_is_measured_and_agrees_with_the_default():
    from pdum_dsl_amd import kernels as K
    from pdum_dsl_amd import measure as M
    from pdum_dsl_amd.tl import analysis as A

    B, Hq, Hkv, S, D = 4, 16, 4, 2048, 128
    best, facts = M.tune_decode_splits(B, Hq, Hkv, S, D, dtype="bf16")
    assert best in M.DECODE_SPLITS and set(facts) == set(M.DECODE_SPLITS)
    assert all(f.value["ms"] > 0 for f in facts.values())
    assert facts[best].value["ms"] == min(f.value["ms"] for f in facts.values())
    with A.no_reanalysis():  # a warm re-tune measures nothing
        assert M.tune_decode_splits(B, Hq, Hkv, S, D, dtype="bf16")[0] == best
    g = torch.Generator(device="cuda").manual_seed(4)
    q = torch.randn((B, Hq, 1, D), generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn((B, Hkv, S, D), generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn((B, Hkv, S, D), generator=g, device="cuda").to(torch.bfloat16)
    o1, l1 = K.attn_decode(q, k, v, nsplit=best)
    o2, l2 = K.attn_decode(q, k, v)
    torch.cuda.synchronize()
    assert (o1.float() - o2.float()).abs().max().item() < 2e-2
    assert (l1 - l2).abs().max().item() < 1e-4
