"""The map-chain and contraction-epilogue kernels on silicon.

Through the HIP seat (compile_tile_hip on the planner's generated kernels)
against the float64 oracle evaluation of the naive region
(oracle.region_eval) and numpy closed forms, at the reference's own subject
(relu(a @ b + bias), test_fusion.py:21-42) and at ragged and larger shapes;
and the C ABI directly against a plain fp32 torch reference (pdh_contract with
an identity epilogue is a batched GEMM), plus the refusal of malformed
programs before any launch."""

import numpy as np
import pytest

from tests.test_contraction_mapchain import _oracle, chain_subject, gemm_subject
from tests.tolerances import assert_fp32, assert_lowp

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _gelu_chain_subject(M, K, N, seed=7):
    """gelu_tanh(x) @ w + b: a computed prologue operand, then a bias epilogue."""
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import F64, Builder, Region, tensor_type

    rng = np.random.default_rng(seed)
    b = Builder(OPS)
    c = lambda v: b.emit("core.const", type=F64, value=float(v))  # noqa: E731
    x = b.param(0, tensor_type(("t", "d"), (M, K)))
    w = b.param(1, tensor_type(("d", "f"), (K, N)))
    bias = b.param(2, tensor_type(("f",), (N,)))
    x3 = b.emit("tl.pointwise", b.emit("tl.pointwise", x, x, f="mul"), x, f="mul")
    inner = b.emit("tl.pointwise", b.emit("tl.pointwise", x, b.emit("tl.pointwise", x3, c(0.044715), f="mul"),
                                          f="add"), c(0.7978845608028654), f="mul")
    gx = b.emit("tl.pointwise", b.emit("tl.pointwise", x, c(0.5), f="mul"),
                b.emit("tl.pointwise", b.emit("tl.pointwise", inner, f="tanh"), c(1.0), f="add"), f="mul")
    prod = b.emit("tl.pointwise", b.emit("tl.repeat_like", gx, w), b.emit("tl.repeat_like", w, gx), f="mul")
    z = b.emit("tl.reduce", prod, dims=("d",), f="sum")
    y = b.emit("tl.pointwise", z, b.emit("tl.repeat_like", bias, z), f="add")
    region = Region(params=(x, w, bias), body=(b.emit("core.yield", y),))
    return region, [rng.standard_normal((M, K)) * 0.5, rng.standard_normal((K, N)) * K**-0.5,
                    rng.standard_normal(N)]


def _seat(region, dtype):
    from pdum_dsl_amd.hip_tile import compile_tile_hip
    from pdum_dsl_amd.tl import fusion

    (g,) = fusion.plan_region(region).groups
    return g, compile_tile_hip(g.kernel, g.launch, g.prune, dtype=dtype)


def _check(got, want, dtype, what, k=1):
    if dtype == "f32":
        # fp32 accumulation over k terms: 1e-5 of the result's scale per sqrt(k / 64) of summation depth
        assert_fp32(got, want, rtol=0.0, atol=1e-5 * max(1.0, float(np.abs(want).max())) * max(1.0, (k / 64) ** 0.5),
                    what=what)
    else:
        assert_lowp(got, want, what=what)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(5, 7), (300, 1000), (129, 1001)])  # 1001: one element per lane
def test_map_chain_matches_the_oracle(dtype, shape):
    from pdum_dsl_amd.hip_tile import compile_tile_hip

    region, vals = chain_subject(seed=sum(shape), I=shape[0], J=shape[1])
    run = compile_tile_hip(region, dtype=dtype)
    assert run.template == "map-chain" and run.source.startswith("hip:map_chain")
    got = run(vals)
    y = region.body[-1].args[0]
    want = _oracle(region, vals if dtype == "f32" else [_bf16(v) for v in vals], y.type.names)
    _check(got, want, dtype, f"map chain {shape}")


def _bf16(v):
    return torch.as_tensor(np.asarray(v, dtype=np.float32)).to(torch.bfloat16).float().numpy().astype(np.float64)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize(
    "M,K,N,epi,rider",
    [(6, 8, 5, "relu_bias", None), (200, 100, 130, "relu_bias", None), (256, 768, 384, "gelu_tanh", None),
     (64, 96, 80, None, ("h", 3)), (1, 64, 1, None, None)],
)
def test_contraction_epilogue_matches_the_oracle(dtype, M, K, N, epi, rider):
    region, vals = gemm_subject(M=M, K=K, N=N, epilogue=epi, rider=rider, seed=M + N)
    g, run = _seat(region, dtype)
    assert g.template == "contraction-epilogue" and run.template == "contraction-epilogue"
    got = run(vals)
    names = region.body[-1].args[0].type.names
    want = _oracle(region, vals if dtype == "f32" else [_bf16(v) for v in vals], names)
    _check(got, want, dtype, f"{M}x{K}x{N} {epi} {rider}", k=K)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_a_prologue_chain_runs_before_the_contraction(dtype):
    region, vals = _gelu_chain_subject(96, 160, 72)
    g, run = _seat(region, dtype)
    assert "prologue=chain,param" in run.source
    got = run(vals)
    want = _oracle(region, vals if dtype == "f32" else [_bf16(v) for v in vals], ("t", "f"))
    _check(got, want, dtype, "gelu(x) @ w + b", k=160)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,M,N", [(2, 300, 260), (2, 1100, 2100)])  # 64x64 tiles; 128x128 tiles
def test_the_abi_is_a_batched_gemm_with_an_identity_epilogue(dt, B, M, N):
    from pdum_dsl_amd import _lib as L
    from pdum_dsl_amd import kernels as K

    g = torch.Generator(device="cuda").manual_seed(11)
    Kd = 200
    KP = 256
    a = torch.zeros(B, M, KP, device="cuda", dtype=dt)
    bt = torch.zeros(B, N, KP, device="cuda", dtype=dt)
    a[..., :Kd] = torch.randn(B, M, Kd, device="cuda", generator=g).to(dt)
    bt[..., :Kd] = torch.randn(B, N, Kd, device="cuda", generator=g).to(dt)
    out = torch.empty(B, M, N, device="cuda", dtype=dt)
    p = L.EwProgram()
    p.n_insns, p.n_operands, p.ndim, p.out_reg = 1, 0, 3, 0
    for d, (ext, st) in enumerate(zip((B, M, N), out.stride())):
        p.shape[d], p.out_stride[d] = ext, st
    p.insns[0].op = L.EW["ACC"]
    K.contract(a, bt, Kd, p, [], out)
    torch.cuda.synchronize()
    ref = torch.bmm(a.float(), bt.float().transpose(1, 2).contiguous())  # fp32 reference on the same inputs
    if dt == torch.float32:
        torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-4)
    else:
        assert_lowp(out.float().cpu().numpy(), ref.cpu().numpy(), what="bf16 gemm")


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T,H", [(256, 4), (1024, 12)])
def test_strided_operands_feed_a_head_major_product_without_copies(dt, T, H):
    """scores[h, t, s] = sum_e q[t, h, e] k[s, h, e]: q and k stay in their
    (t, heads, head_dim) storage; the batch is the head (stride head_dim), a
    row is a position (stride heads * head_dim)."""
    from pdum_dsl_amd import _lib as L
    from pdum_dsl_amd import kernels as K

    g = torch.Generator(device="cuda").manual_seed(5)
    E = 64
    q = torch.randn(T, H, E, device="cuda", generator=g).to(dt)
    k = torch.randn(T + 7, H, E, device="cuda", generator=g).to(dt)
    out = torch.empty(H, T, T + 7, device="cuda", dtype=dt)
    p = L.EwProgram()
    p.n_insns, p.n_operands, p.ndim, p.out_reg = 1, 0, 3, 0
    for d, (ext, st) in enumerate(zip(out.shape, out.stride())):
        p.shape[d], p.out_stride[d] = ext, st
    p.insns[0].op = L.EW["ACC"]
    K.contract_strided(q, (E, H * E), k, (E, H * E), (H, T, T + 7, E), p, [], out)
    torch.cuda.synchronize()
    ref = torch.einsum("the,she->hts", q.double().cpu(), k.double().cpu())
    if dt == torch.float32:
        torch.testing.assert_close(out.double().cpu(), ref, rtol=1e-5, atol=1e-4)
    else:
        assert_lowp(out.float().cpu().numpy(), ref.numpy(), what="strided bf16 gemm")


def test_malformed_programs_refuse_without_launching():
    from pdum_dsl_amd import _lib as L
    from pdum_dsl_amd import kernels as K

    x = torch.zeros(4, 8, device="cuda")
    out = torch.empty(4, 8, device="cuda")
    p = L.EwProgram()
    p.n_insns, p.n_operands, p.ndim, p.out_reg = 1, 1, 2, 0
    p.shape[0], p.shape[1] = 4, 8
    p.out_stride[0], p.out_stride[1] = 8, 1
    p.in_stride[0][0], p.in_stride[0][1] = 8, 1
    p.insns[0].op, p.insns[0].dst = L.EW["LOAD"], 16  # register 16 of 16
    with pytest.raises(L.PdhError, match="register out of range"):
        K.map_chain(p, [x], out)
    p.insns[0].dst, p.insns[0].op = 0, L.EW["ACC"]
    with pytest.raises(L.PdhError, match="accumulator"):
        K.map_chain(p, [x], out)
    p.insns[0].op, p.insns[0].a = L.EW["LOAD"], 3  # operand 3 of 1
    with pytest.raises(L.PdhError, match="loads operand"):
        K.map_chain(p, [x], out)
    p.insns[0].a, p.in_stride[0][0] = 0, 9  # a view past the operand's storage
    with pytest.raises(ValueError, match="reaches past"):
        K.map_chain(p, [x], out)


@pytest.mark.parametrize("jit", [True, False])
def test_the_interpreter_and_the_specialized_kernels_agree(jit):
    """Both evaluators of one program (pdh_ew_set_jit): the runtime-specialized
    kernels and the interpreter kernels, each against the oracle; the
    specialized path is the one that ran when enabled."""
    import ctypes as C

    from pdum_dsl_amd import _lib as L

    lib = L.lib()
    prev = lib.pdh_ew_set_jit(1 if jit else 0)
    try:
        before = (C.c_int64 * 3)()
        lib.pdh_ew_jit_stats(before)
        region, vals = gemm_subject(M=130, K=96, N=70, epilogue="gelu_tanh", seed=3)
        _, run = _seat(region, "bf16")
        got = run(vals)
        want = _oracle(region, [_bf16(v) for v in vals], ("m", "n"))
        _check(got, want, "bf16", f"gemm jit={jit}", k=96)
        chain, cvals = chain_subject(seed=4, I=33, J=64)
        from pdum_dsl_amd.hip_tile import compile_tile_hip

        got = compile_tile_hip(chain, dtype="f32")(cvals)
        _check(got, _oracle(chain, cvals, ("i", "j")), "f32", f"chain jit={jit}")
        after = (C.c_int64 * 3)()
        lib.pdh_ew_jit_stats(after)
        launched = after[1] - before[1]
        assert after[2] == before[2], "a specialization failed to compile"
        assert (launched >= 2) if jit else (launched == 0)
    finally:
        lib.pdh_ew_set_jit(prev)


def _identity_epilogue(out):
    from pdum_dsl_amd import _lib as L

    p = L.EwProgram()
    p.n_insns, p.n_operands, p.ndim, p.out_reg = 1, 0, 3, 0
    for d, (ext, st) in enumerate(zip(out.shape, out.stride())):
        p.shape[d], p.out_stride[d] = ext, st
    p.insns[0].op = L.EW["ACC"]
    return p


def _fp32_gemm(a, bt, kd, mode):
    from pdum_dsl_amd import _lib as L
    from pdum_dsl_amd import kernels as K

    lib = L.lib()
    out = torch.empty(a.shape[0], a.shape[1], bt.shape[1], device="cuda", dtype=torch.float32)
    prev = lib.pdh_contract_set_f32_mode(mode)
    try:
        K.contract(a, bt, kd, _identity_epilogue(out), [], out)
        torch.cuda.synchronize()
    finally:
        lib.pdh_contract_set_f32_mode(prev)
    return out.double().cpu().numpy()


@pytest.mark.parametrize("mode", [6, 0])
def test_the_k_split_partials_are_the_slices_products(mode):
    """pdh_contract_strided_ksplit: index e * S + s holds batch entry e's
    product over the s-th k slice, bit for bit the unsplit kernel on that
    slice alone, and the slices sum to the whole product."""
    from pdum_dsl_amd import kernels as K

    g = torch.Generator(device="cuda").manual_seed(12)
    B, M, N, Kd, S = 3, 70, 90, 512, 4
    a = torch.randn(B, M, Kd, generator=g, device="cuda")
    bt = torch.randn(B, N, Kd, generator=g, device="cuda")
    parts = torch.empty(B * S, M, N, device="cuda")
    K.contract_strided(a, (M * Kd, Kd), bt, (N * Kd, Kd), (B, M, N, Kd), _identity_epilogue(parts), [], parts,
                       f32_mode={6: "bf16x6", 0: "fma"}[mode], ksplit=S)
    c = Kd // S
    for s in range(S):
        one = torch.empty(B, M, N, device="cuda")
        K.contract_strided(a[:, :, s * c:], (M * Kd, Kd), bt[:, :, s * c:], (N * Kd, Kd), (B, M, N, c),
                           _identity_epilogue(one), [], one, f32_mode={6: "bf16x6", 0: "fma"}[mode])
        assert torch.equal(parts.view(B, S, M, N)[:, s], one)
    whole = torch.bmm(a.double(), bt.double().transpose(1, 2).contiguous())
    got = parts.view(B, S, M, N).double().sum(1)
    assert ((got - whole).abs().max() / whole.abs().max()).item() < 1e-5
    with pytest.raises(Exception, match="ksplit"):
        K.contract_strided(a, (M * Kd, Kd), bt, (N * Kd, Kd), (B, M, N, Kd), _identity_epilogue(parts), [], parts,
                           ksplit=3)


# mode -> tolerance as a fraction of the output's scale: 6 bf16 products per
# term and VALU fma are fp32 grade; 3 products keep about 2^-16 of each
# product; 1 (bf16-rounded operands) is exact against bf16-rounded inputs
@pytest.mark.parametrize("mode,tol", [(6, 1e-5), (3, 5e-5), (1, 1e-5), (0, 1e-5)])
@pytest.mark.parametrize("B,M,N,Kd", [(2, 300, 260, 200), (1, 1100, 2100, 768)])  # 64x64 tiles; 128x128 tiles
def test_fp32_contractions_against_float64(mode, tol, B, M, N, Kd):
    """fp32 a @ bt^T on the bf16 matrix cores (the operands split into bf16
    planes) or by VALU fma, against float64 numpy on the same fp32 inputs."""
    g = torch.Generator(device="cuda").manual_seed(13)
    KP = (Kd + 63) // 64 * 64
    a = torch.zeros(B, M, KP, device="cuda")
    bt = torch.zeros(B, N, KP, device="cuda")
    a[..., :Kd] = torch.randn(B, M, Kd, device="cuda", generator=g)
    bt[..., :Kd] = torch.randn(B, N, Kd, device="cuda", generator=g) * 3.0
    got = _fp32_gemm(a, bt, Kd, mode)
    an, bn = a.double().cpu().numpy(), bt.double().cpu().numpy()
    if mode == 1:  # operands rounded to bf16 (nearest even), products and sums in fp32
        an, bn = (t.to(torch.bfloat16).double().cpu().numpy() for t in (a, bt))
    want = np.einsum("bmk,bnk->bmn", an, bn)
    err = np.abs(got - want).max()
    assert err <= tol * np.abs(want).max() * max(1.0, (Kd / 64) ** 0.5), f"mode {mode}: max err {err:.3e}"


def test_tiny_fp32_operands_keep_fp32_grade():
    """Leading terms below 2^-100 would leave the split's lower bf16 planes in
    the subnormal range (a 1e-35 operand keeps ~8 of its 24 bits there); the
    workgroups that load one recompute by fp32 fma, so every output stays
    within fp32 accumulation error of the float64 product (1e-6 of the sum of
    |a b|: a CPU simulation of the flushed planes errs by 2e-4 of it), tiny
    rows and ordinary rows alike."""
    g = torch.Generator(device="cuda").manual_seed(23)
    B, M, N, Kd = 1, 300, 260, 256
    a = torch.randn(B, M, Kd, device="cuda", generator=g)
    a[0, :100] *= 1e-35  # tiny rows: one whole 64 x 64 tile and part of another
    bt = torch.randn(B, N, Kd, device="cuda", generator=g) * 1e3
    got = _fp32_gemm(a, bt, Kd, 6)
    ad, bd = a.double().cpu().numpy(), bt.double().cpu().numpy()
    want = np.einsum("bmk,bnk->bmn", ad, bd)
    scale = np.einsum("bmk,bnk->bmn", np.abs(ad), np.abs(bd))
    err = np.abs(got - want) / scale
    assert err[:, :100].max() <= 1e-6, f"tiny rows: {err[:, :100].max():.3e} of sum |a b|"
    assert err[:, 100:].max() <= 1e-6, f"ordinary rows: {err[:, 100:].max():.3e} of sum |a b|"
    assert np.abs(want[:, :100]).max() < 1e-29 and np.abs(got[:, :100]).max() > 0  # the tiny products are normal fp32


@pytest.mark.parametrize("mode", [6, 3])
def test_non_finite_fp32_operands_behave_as_in_fp32(mode):
    """An inf times a value exact in bf16 would meet a zero lower plane (inf *
    0 = NaN); workgroups that load a non-finite value recompute by fp32 fma,
    so infs and NaNs land where IEEE arithmetic puts them, and every other
    workgroup keeps the split result."""
    g = torch.Generator(device="cuda").manual_seed(17)
    B, M, N, Kd = 1, 700, 600, 256
    a = torch.randn(B, M, Kd, device="cuda", generator=g)
    bt = torch.randn(B, N, Kd, device="cuda", generator=g).round()  # integers: exact in bf16, zero lower planes
    bt[bt == 0] = 1.0
    a[0, 5, 17] = float("inf")
    a[0, 650, 3] = -float("inf")
    bt[0, 333, 40] = float("nan")
    got = _fp32_gemm(a, bt, Kd, mode)
    want = np.einsum("bmk,bnk->bmn", a.double().cpu().numpy(), bt.double().cpu().numpy())
    assert np.array_equal(np.isnan(got), np.isnan(want)) and np.isnan(want).sum() == M  # column 333
    assert np.isinf(want).sum() == 2 * (N - 1)  # rows 5 and 650 away from column 333
    assert np.array_equal(np.isinf(got), np.isinf(want)) and np.array_equal(got[np.isinf(got)], want[np.isinf(want)])
    fin = np.isfinite(want)
    tol = (1e-5 if mode == 6 else 5e-5) * np.abs(want[fin]).max() * 2.0
    assert np.abs(got[fin] - want[fin]).max() <= tol
