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


def _scale_program(n, c):
    """out = x * c over n elements: a program of its own (the constant makes
    its specialized source, and so its compile, unique to the caller)."""
    from pdum_dsl_amd import _lib as L

    p = L.EwProgram()
    p.n_insns, p.n_operands, p.ndim, p.out_reg = 3, 1, 1, 2
    p.shape[0], p.start[0], p.out_stride[0] = n, 0, 1
    p.in_stride[0][0] = 1
    p.insns[0].op, p.insns[0].dst, p.insns[0].a = L.EW["LOAD"], 0, 0
    p.insns[1].op, p.insns[1].dst, p.insns[1].imm = L.EW["CONST"], 1, c
    p.insns[2].op, p.insns[2].dst, p.insns[2].a, p.insns[2].b = L.EW["MUL"], 2, 0, 1
    return p


def test_a_compile_inside_a_warm_region_raises_and_a_warm_run_passes():
    """The warmth law of the timed loops (bench_zoo.py:128-152): the first
    launch of a new program compiles it (hipRTC) and must stay out of timing."""
    from pdum_dsl_amd import _lib as L
    from pdum_dsl_amd import kernels as K
    from pdum_dsl_amd import measure as M

    if L.lib().pdh_ew_set_jit(1) == 0:  # restore the setting after the test
        L.lib().pdh_ew_set_jit(0)
        pytest.skip("runtime specialization is disabled in this process")
    x = torch.arange(1024, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    prog = _scale_program(1024, 1.0625 + 2.0 ** -20)
    with pytest.raises(M.WarmthError, match="1 hipRTC compile"):
        with M.no_compiles("cold"):
            K.map_chain(prog, [x], y)
            torch.cuda.synchronize()
    with M.no_compiles("warm"):  # the same program again: cached, no compile
        K.map_chain(prog, [x], y)
        torch.cuda.synchronize()
    assert torch.equal(y, x * (1.0625 + 2.0 ** -20))
