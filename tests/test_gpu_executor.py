"""The carved-plan executor on silicon: gpt2 planned by the anchor-and-absorb
partitioner and run carve by carve on HIP kernels (contractions with
epilogues and prologue packs, row softmax with its re-derived scores,
layernorms, the embedding gather), against the numpy denotation of the model
(zoo.gpt2's ref, the reference's zoo/gpt2.py:141-163 restated). Also the
16-bit row kernels and the gather the executor relies on.

Tolerances: fp32 storage and arithmetic, 1e-4 of the logits' scale; bf16
storage (fp32 accumulation and statistics), the north-star 2e-2 of scale on
GPT-2's own initialization scale (init="gpt2"). The reference toy's draw
(std 0.4 weights and layernorm gains) makes the attention nearly one-hot,
and the softmax amplifies the bf16 rounding of every carve boundary (~23 in
the forward, ~75 in the gradients) beyond it: those stress cases keep their
measured bounds (3e-2 forward, 7e-2 gradients), stated where they are
asserted."""

import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _run(cfg, dtype, seed=7, fuse=True, merge=True, init="toy"):
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.partition import plan_model

    m = zoo.gpt2(cfg, seed=seed, init=init)
    ex = PlanExecutor(plan_model(m.region), m.region, dtype, fuse_attention=fuse, merge_projections=merge)
    ex.bind(m.values())
    out = ex.run()
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    y = m.region.body[-1].args[0]
    got = np.transpose(got, [y.type.names.index(n) for n in m.order])
    return got, m.ref(m.inputs), ex


def test_the_toy_gpt2_runs_carve_by_carve_at_f32():
    from pdum_dsl_amd.tl import zoo

    got, want, ex = _run(zoo.GPT2Config(), "f32", fuse=False)
    assert len(ex.steps) == 23
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-4 * np.abs(want).max())
    # each layer's softmax carve and PV carve launched as one flash forward
    got, want, ex = _run(zoo.GPT2Config(), "f32")
    assert len(ex.steps) == 21 and sum(st.kind == "flash-chain" for st in ex.steps) == 2
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-4 * np.abs(want).max())


@pytest.mark.parametrize("fuse", [True, False])
@pytest.mark.parametrize("dtype,tol", [("f32", 1e-4), ("bf16", 3e-2)])
def test_a_sized_gpt2_matches_the_numpy_model(dtype, tol, fuse):
    from pdum_dsl_amd.tl import zoo

    cfg = zoo.GPT2Config(t=256, d=256, nh=4, hk=64, m=1024, layers=2, v=512)
    got, want, ex = _run(cfg, dtype, seed=3, fuse=fuse)
    src = " | ".join(ex.sources())
    assert "a=direct" in src  # layernorm outputs feed the projections without a pack
    assert ("softmax + PV carves" in src) == fuse
    err = np.abs(got - want).max()
    assert err <= tol * np.abs(want).max(), f"{dtype}: max err {err} vs scale {np.abs(want).max()}"


@pytest.mark.parametrize("fuse", [True, False])
def test_a_sized_gpt2_at_gpt2_init_scale_holds_bf16_to_2e2(fuse):
    """bf16 storage at GPT-2's initialization scale: the whole 2-layer
    forward within the north star's 2e-2 of the logits' scale."""
    from pdum_dsl_amd.tl import zoo

    cfg = zoo.GPT2Config(t=256, d=256, nh=4, hk=64, m=1024, layers=2, v=512)
    got, want, _ = _run(cfg, "bf16", seed=3, fuse=fuse, init="gpt2")
    err = np.abs(got - want).max()
    assert err <= 2e-2 * np.abs(want).max(), f"max err {err} vs scale {np.abs(want).max()}"


@pytest.mark.parametrize("t,form", [(64, "scores carved"), (128, "scores dissolved"), (256, "projections dissolved"),
                                    (256, "projections merged")])
@pytest.mark.parametrize("dtype,tol", [("f32", 1e-4), ("bf16", 3e-2)])
def test_attention_chains_in_each_carve_form(t, form, dtype, tol):
    """The softmax + PV carves launched as one flash forward in each form the
    traffic gate gives them: the scores a carve of their own (t=64), the
    scores dissolved into the softmax carve (t=128), and the q/k/v
    projections dissolved too (t=256), so the launch makes them first: by
    three nested plans, or by one GEMM over the concatenated weights with the
    scale moved into the flash launch. Against the numpy model, and against
    the unfused plan."""
    from pdum_dsl_amd.tl import zoo

    cfg = zoo.GPT2Config(t=t, d=128, nh=2, hk=64, m=512, layers=1, v=64)
    got, want, ex = _run(cfg, dtype, seed=3, merge=form == "projections merged")
    chains = [st for st in ex.steps if st.kind == "flash-chain"]
    assert len(chains) == 1
    made = {"scores carved": "qkv=bbb", "scores dissolved": "qkv=bbb", "projections dissolved": "qkv=mmm",
            "projections merged": "qkv=merged scale=0.125"}[form]
    assert made in chains[0].source
    n_unfused = len(_run(cfg, dtype, seed=3, fuse=False)[2].steps)
    assert len(ex.steps) == n_unfused - (2 if form == "scores carved" else 1)
    err = np.abs(got - want).max()
    assert err <= tol * np.abs(want).max(), f"{dtype} {form}: max err {err} vs scale {np.abs(want).max()}"


def test_an_out_of_range_token_id_is_refused():
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.partition import plan_model

    m = zoo.gpt2()
    ex = PlanExecutor(plan_model(m.region), m.region, "f32")
    vals = m.values()
    vals[0] = np.array([0, 1, 99, 2])  # the vocab is 5
    ex.bind(vals)
    with pytest.raises(IndexError, match="outside the table"):
        ex.run()


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cols", [768, 4096, 5000])
def test_16_bit_row_kernels_match_fp32_math(dt, cols):
    from pdum_dsl_amd import kernels as K

    g = torch.Generator(device="cuda").manual_seed(1)
    x = torch.randn((37, cols), generator=g, device="cuda").to(dt)
    gam = (1 + 0.1 * torch.randn((cols,), generator=g, device="cuda")).to(dt)
    bet = (0.1 * torch.randn((cols,), generator=g, device="cuda")).to(dt)
    y = K.row_softmax(x)
    want = torch.softmax(x.float(), dim=-1)
    assert y.dtype == dt
    assert ((y.float() - want).abs() / want.abs().max()).max().item() < 1e-2
    z = K.layernorm(x, gam, bet, eps=1e-5)
    wz = torch.nn.functional.layer_norm(x.float(), (cols,), gam.float(), bet.float(), eps=1e-5)
    assert (z.float() - wz).abs().max().item() < 2e-2 * wz.abs().max().item()


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_take_rows_is_a_bit_exact_gather(dt):
    from pdum_dsl_amd import kernels as K

    g = torch.Generator(device="cuda").manual_seed(2)
    table = torch.randn((50, 3, 10), generator=g, device="cuda").to(dt)
    idx = torch.randint(0, 50, (4, 7), generator=g, device="cuda")
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    got = K.take_rows(table, idx, bad=bad)
    assert torch.equal(got, table[idx]) and int(bad.item()) == 0
    idx[1, 2] = 50
    got = K.take_rows(table, idx, bad=bad)
    assert int(bad.item()) == 1 and torch.count_nonzero(got[1, 2]).item() == 0


def _add_at_reference(values, idx, n_rows, dt):
    """Row v = the values rows at the positions holding v, summed in
    increasing position order in fp32 and rounded once to dt (numpy's
    unbuffered add.at applies the updates in index order)."""
    row = math.prod(values.shape[idx.dim():])
    v32 = values.float().cpu().numpy().reshape(idx.numel(), row)
    acc = np.zeros((n_rows, row), dtype=np.float32)
    ii = idx.cpu().numpy().reshape(-1)
    keep = (ii >= 0) & (ii < n_rows)
    np.add.at(acc, ii[keep], v32[keep])
    return torch.from_numpy(acc).to(dt)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n_idx,n_rows,row", [(0, 5, 8), (1, 1, 1), (37, 50, 30), (1000, 37, 1500), (700, 5000, 7),
                                              (300, 2, 2049), (65536, 3, 1100)])
def test_scatter_add_rows_sums_duplicates_in_position_order(dt, n_idx, n_rows, row):
    """pdh_scatter_add_rows against numpy's add.at in fp32 rounded once:
    bit-exact, rows nothing lands in zero, across index chunks (n_idx > 256),
    column passes (rows over 1024 elements), odd row widths, and the largest
    batch one launch takes (2^16 positions on 3 rows: every owner's matches
    span the whole mask cache, reused by a second column pass)."""
    from pdum_dsl_amd import kernels as K

    print(f"scatter_add_rows dt={dt} n_idx={n_idx} n_rows={n_rows} row={row}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(n_idx + row)
    values = torch.randn((n_idx, row), generator=g, device="cuda").to(dt)
    idx = torch.randint(0, n_rows, (n_idx,), generator=g, device="cuda")
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.full((n_rows, row), 7.0, device="cuda", dtype=dt)  # every row is rewritten
    got = K.scatter_add_rows(values, idx, n_rows, out=out, bad=bad)
    torch.cuda.synchronize()
    want = _add_at_reference(values, idx, n_rows, dt)
    assert int(bad.item()) == 0
    assert torch.equal(got.cpu(), want)
    again = K.scatter_add_rows(values, idx, n_rows)
    assert torch.equal(again, got)  # deterministic: the same bits on every call


def test_scatter_add_rows_refuses_more_positions_than_one_launch_takes():
    from pdum_dsl_amd import kernels as K
    from pdum_dsl_amd._lib import PdhError

    n = K.SCATTER_MAX_IDX + 1
    values = torch.zeros((n, 4), device="cuda")
    idx = torch.zeros((n,), dtype=torch.int64, device="cuda")
    with pytest.raises(PdhError, match="more than the 65536 one launch takes"):
        K.scatter_add_rows(values, idx, 2)


def test_scatter_add_rows_counts_and_drops_bad_indices_and_takes_strided_rows():
    from pdum_dsl_amd import kernels as K

    g = torch.Generator(device="cuda").manual_seed(5)
    wide = torch.randn((4, 6, 40), generator=g, device="cuda")
    values = wide[..., :33]  # row stride 40, 33 elements a row
    idx = torch.randint(0, 9, (4, 6), generator=g, device="cuda")
    idx[0, 1], idx[3, 5] = -1, 9
    bad = torch.zeros(1, dtype=torch.int32, device="cuda")
    assert not values.is_contiguous()
    got = K.scatter_add_rows(values, idx, 9, bad=bad)
    torch.cuda.synchronize()
    assert int(bad.item()) == 2
    assert torch.equal(got.cpu(), _add_at_reference(values.contiguous(), idx, 9, torch.float32))


@pytest.mark.parametrize("T,D,F,f32c", [(300, 1024, 200, "bf16x6"), (1024, 3072, 64, "bf16x3"), (64, 640, 96, "fma")])
def test_a_small_fp32_contraction_splits_k(T, D, F, f32c):
    """An fp32 contraction whose output tiles cannot fill the chip runs k in
    slices (fp32 partial planes added in order by the epilogue's map chain):
    against the float64 denotation at the mode's tolerance, and against the
    unsplit kernel called directly."""
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.partition import plan_model

    subj = zoo.linear_gelu(T=T, D=D, F=F, seed=T + D)
    ex = PlanExecutor(plan_model(subj.region), subj.region, "f32", f32_contract=f32c)
    assert any("ksplit=" in st.source for st in ex.steps), [st.source for st in ex.steps]
    vals = [f.arr for f in subj.inputs]
    ex.bind(vals)
    got = ex.run().cpu().numpy().astype(np.float64)
    torch.cuda.synchronize()
    want = subj.oracle(vals)
    tol = {"bf16x6": 1e-5, "bf16x3": 2e-4, "fma": 1e-5}[f32c]
    assert np.abs(got - want).max() <= tol * max(1.0, np.abs(want).max())


def test_a_batched_fp32_contraction_splits_k():
    """A contraction batched over a rider dim (12 heads: 12 x 64 x 64 output
    tiles, k = 1024) splits k per batch entry: against the float64 oracle."""
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl.partition import plan_model
    from tests.test_contraction_mapchain import _oracle, gemm_subject

    region, vals = gemm_subject(M=64, K=1024, N=60, epilogue="relu_bias", seed=7, rider=("h", 12))
    ex = PlanExecutor(plan_model(region), region, "f32")
    assert any("ksplit=" in st.source and "batch=12" in st.source for st in ex.steps), [st.source for st in ex.steps]
    ex.bind(vals)
    got = ex.run().cpu().numpy().astype(np.float64)
    torch.cuda.synchronize()
    y = region.body[-1].args[0]
    want = _oracle(region, vals, y.type.names)
    assert np.abs(got - want).max() <= 1e-5 * max(1.0, np.abs(want).max())


def test_a_captured_plan_replays_the_eager_result():
    """The whole carved forward as one HIP graph: replays, with eager work and
    synchronizations between them, each give the eager pass's output."""
    from pdum_dsl_amd import kernels as K
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.partition import plan_model

    cfg = zoo.GPT2Config(t=256, d=256, nh=4, hk=64, m=1024, layers=2, v=512)
    m = zoo.gpt2(cfg, seed=3)
    ex = PlanExecutor(plan_model(m.region), m.region, "bf16")
    ex.bind(m.values())
    eager = ex.run().clone()
    ex.capture()
    for i in range(4):
        junk = K.row_softmax(torch.randn(64, 256, device="cuda"))  # eager work between replays
        torch.cuda.synchronize()
        got = ex.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {i} differs from the eager pass"
        del junk


@pytest.mark.parametrize("dtype,tol", [("f32", 1e-5), ("bf16", 2e-2)])
def test_a_planned_attention_runs_its_flash_carve(dtype, tol):
    """plan_model on the naive attention region gives one flash carve; the
    executor binds it to the flash kernel (mask as a band)."""
    from oracle import closed_forms as cf
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.partition import plan_model

    s = zoo.attention(T=200, S=200, E=64, OD=64, mask="causal", seed=4)
    plan = plan_model(s.region)
    assert [c.group.template for c in plan.carves] == ["flash"]
    ex = PlanExecutor(plan, s.region, dtype)
    vals = s.numpy_inputs()
    if dtype == "bf16":
        vals = [torch.as_tensor(v).to(torch.bfloat16).double().numpy() for v in vals]
    ex.bind(vals)
    got = ex.run().double().cpu().numpy()
    want = cf.attention(*vals, scale=1.0, band=(None, 0))[0]
    assert np.abs(got - want).max() <= tol * max(1.0, np.abs(want).max())


def test_window_decimate_diagonal_views_run_in_a_map_chain():
    """A map chain over window / decimate / diagonal views reads them in
    place (strides and offsets over the stored tensors) on the device."""
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import interp
    from pdum_dsl_amd.tl.partition import plan_model
    from tests.test_views_reducers import _affine_region

    r = _affine_region()
    plan = plan_model(r)
    assert {c.group.template for c in plan.carves} == {"map-chain"}
    rng = np.random.default_rng(14)
    X, Y = rng.standard_normal((3, 30)), rng.standard_normal((12, 3, 14))
    want = interp.run_region(r, [interp.Field(X, r.params[0].type.dims), interp.Field(Y, r.params[1].type.dims)])
    ex = PlanExecutor(plan, r, "f32")
    ex.bind([X, Y])
    got = ex.run().double().cpu().numpy()
    np.testing.assert_allclose(got, want.to_numpy(r.body[-1].args[0].type.names), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("k,dil", [((-2, 1), 1), ((1, 3), 2)])
def test_a_stencil_and_its_joint_run_on_the_device(k, dil):
    """tl.stencil plans red; the executor runs it as a window over a pad of
    its fill, and its joint (the taps' cotangents shifted back, padded) the
    same way."""
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import interp
    from pdum_dsl_amd.tl.autodiff import grad, region_names
    from pdum_dsl_amd.tl.partition import plan_model
    from tests.test_views_reducers import _stencil_region

    r = _stencil_region(k, dil)
    rng = np.random.default_rng(17)
    X = rng.standard_normal((3, 40))
    want = interp.run_region(r, [interp.field(X, ("r", "x"))])
    ex = PlanExecutor(plan_model(r), r, "f32")
    ex.bind([X])
    got = ex.run().double().cpu().numpy()
    np.testing.assert_allclose(got, want.to_numpy(r.body[-1].args[0].type.names), rtol=1e-6, atol=1e-7)
    rg = grad(r, "out", seed="dy", names=region_names(r, ("x",)))
    out_t = r.body[-1].args[0].type
    dy = rng.standard_normal(out_t.shape)
    wj = interp.run_region(rg.region, [interp.field(X, ("r", "x")), interp.Field(dy, out_t.dims)])
    ej = PlanExecutor(plan_model(rg.region), rg.region, "f32")
    ej.bind([X, dy])
    gx = ej.run()[1].double().cpu().numpy()
    np.testing.assert_allclose(gx, wj[1].to_numpy(rg.region.body[-1].args[0].args[1].type.names), rtol=1e-5,
                               atol=1e-6)


@pytest.mark.parametrize("enc", ["bf16", "f16", "f32"])
def test_round_to_runs_as_a_map_chain(enc):
    """round_to plans red (compute vocabulary); the executor runs its carve
    as one map chain with the hardware round trip. On float32 values the
    device's rounding is the interpreter's exactly."""
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import interp
    from pdum_dsl_amd.tl.partition import plan_model
    from tests.test_views_reducers import _round_region

    r = _round_region(enc)
    X = np.random.default_rng(18).standard_normal((64, 96)).astype(np.float32).astype(np.float64)
    plan = plan_model(r)
    ex = PlanExecutor(plan, r, "f32")
    ex.bind([X])
    got = ex.run().cpu().numpy()
    # the interpreter on the device's float32 square, rounded, plus x in float32
    sq = (X.astype(np.float32) * X.astype(np.float32)).astype(np.float64)
    want = (interp.round_to(sq, enc).astype(np.float32) + X.astype(np.float32))
    np.testing.assert_array_equal(got, want)


def test_the_flashsm_program_runs_its_flash_carve():
    """Attention spelled with the flashsm composite reducer: plan_model gives
    one flash carve and the executor runs it on the flash kernel."""
    from oracle import closed_forms as cf
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.partition import plan_model

    s = zoo.flash_attention(T=160, E=64, OD=64, seed=8)
    plan = plan_model(s.region)
    assert [c.group.template for c in plan.carves] == ["flash"]
    ex = PlanExecutor(plan, s.region, "f32")
    vals = s.numpy_inputs()
    ex.bind(vals)
    got = ex.run().double().cpu().numpy()
    want = cf.attention(*vals, scale=1.0, band=(None, 0))[0]
    assert np.abs(got - want).max() <= 1e-5 * max(1.0, np.abs(want).max())


def test_a_planned_flash_joint_runs_forward_and_backward():
    """The joint (out, dq, dk, dv) claimed whole by plan_model runs as the
    forward with artifacts plus the fused backward, against the closed form."""
    from oracle import closed_forms as cf
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.autodiff import grad, region_names
    from pdum_dsl_amd.tl.partition import plan_model

    s = zoo.attention(T=256, S=256, E=64, OD=64, mask="causal", seed=6)
    rg = grad(s.region, "out", seed="dO", wrt=("q", "k", "v"), names=region_names(s.region, ("q", "k", "v"), ("out",)))
    plan = plan_model(rg.region)
    assert [c.group.template for c in plan.carves] == ["flash-joint"]
    ex = PlanExecutor(plan, rg.region, "bf16")
    rng = np.random.default_rng(2)
    vals = s.numpy_inputs() + [rng.standard_normal((256, 64))]
    vals = [torch.as_tensor(v).to(torch.bfloat16).double().numpy() for v in vals]
    ex.bind(vals)
    ys = rg.region.body[-1].args[0].args  # outputs come in their IR types' dim order
    orders = (("t", "o"), ("t", "e"), ("s", "e"), ("s", "o"))
    got = [np.transpose(x.double().cpu().numpy(), [y.type.names.index(n) for n in order])
           for x, y, order in zip(ex.run(), ys, orders)]
    q, k, v, do = vals
    wo = cf.attention(q, k, v, scale=1.0, band=(None, 0))[0]
    wq, wk, wv = cf.attention_bwd(q, k, v, do, scale=1.0, band=(None, 0))
    for g, want in zip(got, (wo, wq, wk, wv)):
        assert np.abs(g - want).max() <= 2e-2 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("f", ["max", "min"])
def test_a_bare_row_max_or_min_runs_on_the_device(f):
    """A bare max / min reduction is a red group in the reference's plan; the
    executor runs it with pdh_reduce_rows_ex (exact: a max selects a value)."""
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import Builder, Dim, Region, TensorType
    from pdum_dsl_amd.tl.partition import plan_model

    b = Builder(OPS)
    x = b.param(0, TensorType((Dim("t", 0, 37), Dim("h", 0, 3), Dim("s", 0, 700))))
    y = b.emit("tl.reduce", x, dims=("s",), f=f)
    region = Region(params=(x,), body=(b.emit("core.yield", y),))
    ex = PlanExecutor(plan_model(region), region, "f32")
    xv = np.random.default_rng(4).standard_normal((37, 3, 700))
    # a NaN anywhere in a row makes its max / min NaN, as numpy's reductions
    # (and the reference's float64 evaluator) have it
    xv[5, 1, 0] = xv[11, 0, 333] = xv[36, 2, 699] = np.nan
    ex.bind([xv])
    got = ex.run().cpu().numpy()
    torch.cuda.synchronize()
    want = getattr(np, f)(xv.astype(np.float32), axis=2)
    want = np.transpose(want, [("t", "h").index(n) for n in y.type.names])
    assert np.isnan(want).sum() == 3
    np.testing.assert_array_equal(got, want)  # NaN positions must agree too


_SMALL = dict(t=64, d=128, nh=2, hk=64, m=512, layers=1, v=64)
_TWO_LAYER = dict(t=256, d=256, nh=4, hk=64, m=1024, layers=2, v=512)
_LONG = dict(t=512, d=128, nh=2, hk=64, m=512, layers=1, v=64)  # the softmax statistics as row partials


@pytest.mark.parametrize("cfg,dtype,f32c,tol,tables,init", [
    (_SMALL, "f32", "bf16x6", 1e-5, False, "toy"), (_SMALL, "f32", "bf16x3", 2e-4, False, "toy"),
    (_SMALL, "f32", "bf16", 3e-2, False, "toy"), (_SMALL, "f32", "fma", 1e-5, False, "toy"),
    (_SMALL, "bf16", "bf16x6", 7e-2, False, "toy"), (_TWO_LAYER, "f32", "bf16x6", 3e-5, False, "toy"),
    (_TWO_LAYER, "f32", "bf16x3", 5e-4, False, "toy"), (_SMALL, "f32", "bf16x6", 1e-5, True, "toy"),
    (_SMALL, "bf16", "bf16x6", 7e-2, True, "toy"), (_TWO_LAYER, "f32", "bf16x6", 3e-5, True, "toy"),
    (_LONG, "f32", "bf16x6", 3e-5, False, "toy"), (_LONG, "f32", "fma", 3e-5, False, "toy"),
    (_SMALL, "bf16", "bf16x6", 2e-2, True, "gpt2"), (_TWO_LAYER, "bf16", "bf16x6", 2e-2, False, "gpt2")])
def test_the_gpt2_weight_gradients_run_carve_by_carve(cfg, dtype, f32c, tol, tables, init):
    """grad of gpt2's logits w.r.t. every weight (the embedding tables too
    when ``tables``: their gradient is a scatter-add of the embedding's
    cotangent, plus the tied head's product for wte), planned by plan_model
    and run on the device (contractions with their epilogues, map chains,
    the layernorm, the gather, the scatter-add and the bare row max),
    against the float64 oracle's evaluation of the same joint. Per output,
    tol of its scale. The zoo's weights (std 0.4) make the attention sharp,
    so rounding the score contraction's operands is amplified by the
    softmax: bf16 storage (every boundary of ~75 carves rounded) measures
    5.2e-2 on the attention weights (4.1e-2 while the softmax's max still
    took its cotangent, whose zero-sum terms re-centred each rounded row); fp32 storage with f32_contract "bf16"
    (only the contraction operands rounded, fp32 accumulation and
    boundaries: an autocast's numerics) 2.3e-2; "bf16x3" 5.5e-5; "bf16x6" and
    "fma" 2e-6 (1e-5 at two layers). At GPT-2's own initialization scale
    (init="gpt2") bf16 storage holds the north star's 2e-2."""
    from oracle import region_eval as rev
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.autodiff import grad, region_names
    from pdum_dsl_amd.tl.partition import plan_model

    m = zoo.gpt2(zoo.GPT2Config(**cfg), seed=3, init=init)
    pn = tuple(m.names[id(p)] for p in m.region.params)
    wrt = tuple(n for n in pn if n not in (("ids",) if tables else ("ids", "wte", "wpe")))
    rg = grad(m.region, "logits", seed="dlogits", wrt=wrt, names=region_names(m.region, pn, ("logits",)))
    dl = np.random.default_rng(2).standard_normal(tuple(rg.region.params[-1].type.shape))
    vals = m.values() + [dl]
    ex = PlanExecutor(plan_model(rg.region), rg.region, dtype, f32_contract=f32c)
    assert any(st.source.startswith("scatter_add_rows") for st in ex.steps) == tables
    if tables:  # repeated tokens: the scatter-add must sum rows, not overwrite them
        ids = vals[pn.index("ids")]
        assert len(np.unique(ids)) < np.size(ids)
    if dtype == "f32":
        assert all(f"f32={f32c}" in st.source for st in ex.steps if st.source.startswith("contract"))
    # the softmax's max takes no cotangent (shift invariance): no scan, no bare max in the backward
    assert not any("split at scan" in st.source for st in ex.steps)
    if cfg is _LONG:  # the recomputed max and denominator never store the scores
        assert sum("rowred=" in st.source for st in ex.steps) == 2, [st.source for st in ex.steps]
    ex.bind(vals)
    outs = ex.run()
    torch.cuda.synchronize()
    want = rev.evaluate(rg.region, [rev.value(v, p.type) for v, p in zip(vals, rg.region.params)])
    assert len(outs) == len(want) == 1 + len(wrt)
    for name, g, w in zip(rg.outputs, outs, want):
        w = w.numpy()
        err = np.abs(g.float().cpu().numpy() - w).max()
        assert err <= tol * max(np.abs(w).max(), 1e-6), f"{dtype} {name}: max err {err} vs scale {np.abs(w).max()}"
