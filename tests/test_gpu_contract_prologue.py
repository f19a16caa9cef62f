"""Operand prologues computed in the contraction's k loop (pdh_contract_views_pro).

The reference re-derives a contraction's computed operands per tile inside
its k loop (conformance/triton_tile.py:228-371, _dot_at / _reduce_at). Here the
fp32 contractions do the same: a prologue program is evaluated as each k tile
is loaded and the operand never reaches HBM. Checked three ways:
- through the HIP seat and the device executor against the float64 oracle
  evaluation of the naive region (oracle.region_eval);
- through the C ABI against the same contraction over the operand the same
  program materialized first (pdh_map_chain, then pdh_contract_views): equal
  bit for bit under the interpreter (both evaluate each instruction alone), and
  to fp32 rounding with the runtime-specialized evaluators (the compiler may
  fuse a multiply and an add differently in the two kernels);
- with values the bf16 planes cannot carry (an inf from the prologue), where
  both forms take the fp32 fallback and agree.
"""

import numpy as np
import pytest

from tests.test_contraction_mapchain import _oracle
from tests.test_gpu_contract import _check, _gelu_chain_subject, _seat
from tests.tolerances import assert_fp32

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _two_chain_subject(M, K, N, seed=3):
    """(tanh(x) + x / 2) @ (w * s) + b: both operands computed, s broadcast
    along the n side."""
    from pdum_dsl_amd.tl.dialect import OPS
    from pdum_dsl_amd.tl.ir import F64, Builder, Region, tensor_type

    rng = np.random.default_rng(seed)
    b = Builder(OPS)
    c = lambda v: b.emit("core.const", type=F64, value=float(v))  # noqa: E731
    x = b.param(0, tensor_type(("t", "d"), (M, K)))
    w = b.param(1, tensor_type(("d", "f"), (K, N)))
    s = b.param(2, tensor_type(("d",), (K,)))
    bias = b.param(3, tensor_type(("f",), (N,)))
    xa = b.emit("tl.pointwise", b.emit("tl.pointwise", x, f="tanh"), b.emit("tl.pointwise", x, c(0.5), f="mul"),
                f="add")
    wb = b.emit("tl.pointwise", w, b.emit("tl.repeat_like", s, w), f="mul")
    prod = b.emit("tl.pointwise", b.emit("tl.repeat_like", xa, wb), b.emit("tl.repeat_like", wb, xa), f="mul")
    z = b.emit("tl.reduce", prod, dims=("d",), f="sum")
    y = b.emit("tl.pointwise", z, b.emit("tl.repeat_like", bias, z), f="add")
    region = Region(params=(x, w, s, bias), body=(b.emit("core.yield", y),))
    return region, [rng.standard_normal((M, K)), rng.standard_normal((K, N)) * K**-0.5,
                    1.0 + 0.25 * rng.standard_normal(K), rng.standard_normal(N)]


@pytest.mark.parametrize("M,K,N", [(96, 160, 72), (130, 1001, 70), (5, 3, 7), (300, 640, 260)])
def test_the_seat_computes_a_prologue_chain_in_the_k_loop(M, K, N):
    region, vals = _gelu_chain_subject(M, K, N, seed=M + K)
    _g, run = _seat(region, "f32")
    assert run.source.startswith("hip:contract_views_pro") and "prologue=chain,param" in run.source
    got = run(vals)
    _check(got, _oracle(region, vals, ("t", "f")), "f32", f"gelu(x) @ w + b {M}x{K}x{N}", k=K)


@pytest.mark.parametrize("M,K,N", [(64, 96, 80), (257, 333, 129)])
def test_both_operands_computed(M, K, N):
    region, vals = _two_chain_subject(M, K, N, seed=M)
    _g, run = _seat(region, "f32")
    assert "prologue=chain,chain" in run.source
    got = run(vals)
    _check(got, _oracle(region, vals, ("t", "f")), "f32", f"both computed {M}x{K}x{N}", k=K)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_the_executor_fuses_a_computed_operand(dtype):
    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl.partition import plan_model
    from tests.test_gpu_contract import _bf16

    region, vals = _gelu_chain_subject(200, 448, 136, seed=5)
    ex = PlanExecutor(plan_model(region), region, dtype)
    assert any("a=prologue" in s for s in ex.sources())
    ex.bind(vals)
    got = ex.run()  # the one output, dims in the yield's order
    torch.cuda.synchronize()
    want = _oracle(region, vals if dtype == "f32" else [_bf16(v) for v in vals], ("t", "f"))
    _check(got.float().cpu().numpy(), want, dtype, f"executor gelu(x) @ w + b ({dtype})", k=448)


def _programs(B, M, N, Kd, x, s):
    """The a prologue x * s (s broadcast over rows) + tanh(x), as a program
    over (batch, m, k), and an identity epilogue over (batch, m, n)."""
    from pdum_dsl_amd import _lib as L

    pa = L.EwProgram()
    pa.n_operands, pa.ndim, pa.out_reg = 2, 3, 3
    for d, ext in enumerate((B, M, Kd)):
        pa.shape[d] = ext
    for d, st in enumerate((M * Kd, Kd, 1)):
        pa.out_stride[d] = st
        pa.in_stride[0][d] = x.stride()[d]
    for d, st in enumerate((Kd, 0, 1)):  # s[b, k]: broadcast over rows
        pa.in_stride[1][d] = st
    ins = [("LOAD", 0, 0, 0), ("LOAD", 1, 1, 0), ("MUL", 2, 0, 1), ("TANH", 3, 0, 0), ("ADD", 3, 2, 3)]
    pa.n_insns = len(ins)
    for j, (op, dst, a_, b_) in enumerate(ins):
        pa.insns[j].op, pa.insns[j].dst, pa.insns[j].a, pa.insns[j].b = L.EW[op], dst, a_, b_
    return pa


def _identity(shape, out):
    from pdum_dsl_amd import _lib as L

    e = L.EwProgram()
    e.n_insns, e.n_operands, e.ndim, e.out_reg = 1, 0, 3, 0
    for d, (ext, st) in enumerate(zip(shape, out.stride())):
        e.shape[d], e.out_stride[d] = ext, st
    e.insns[0].op = L.EW["ACC"]
    return e


@pytest.mark.parametrize("jit", [True, False])
@pytest.mark.parametrize("mode", ["bf16x6", "bf16x3", "bf16", "fma"])
@pytest.mark.parametrize("B,M,N,Kd,ksplit,bt_rows", [(2, 130, 200, 333, 1, False), (1, 300, 260, 700, 3, True),
                                                     (3, 64, 64, 5, 1, False)])
def test_the_abi_matches_the_materialized_operand(jit, mode, B, M, N, Kd, ksplit, bt_rows):
    from pdum_dsl_amd import _lib as L
    from pdum_dsl_amd import kernels as K

    g = torch.Generator(device="cuda").manual_seed(B * 1000 + Kd)
    x = torch.randn(B, M, Kd, device="cuda", generator=g)
    s = 1.0 + 0.1 * torch.randn(B, Kd, device="cuda", generator=g)
    if bt_rows:  # bt read rows-contiguous (a transposed tensor)
        btt = torch.randn(B, Kd, N, device="cuda", generator=g)
        bt, bst = btt, (Kd * N, 1, N)
    else:
        bt = torch.randn(B, N, Kd, device="cuda", generator=g)
        bst = bt.stride()
    pa = _programs(B, M, N, Kd, x, s)
    out_f = torch.empty(B * ksplit, M, N, device="cuda")
    out_m = torch.empty_like(out_f)
    prev = L.lib().pdh_ew_set_jit(1 if jit else 0)
    try:
        K.contract_views_pro(None, None, bt, bst, (B, M, N, Kd), _identity((B * ksplit, M, N), out_f), [], out_f,
                             pro_a=(pa, [x, s]), f32_mode=mode, ksplit=ksplit)
        a = torch.empty(B, M, Kd, device="cuda")
        K.map_chain(pa, [x, s], a)
        K.contract_views(a, a.stride(), bt, bst, (B, M, N, Kd), _identity((B * ksplit, M, N), out_m), [], out_m,
                         f32_mode=mode, ksplit=ksplit)
        torch.cuda.synchronize()
    finally:
        L.lib().pdh_ew_set_jit(prev)
    what = f"{mode} jit={jit} B{B} M{M} N{N} K{Kd} ksplit={ksplit}"
    if not jit:
        assert torch.equal(out_f, out_m), f"{what}: fused and materialized differ"
    else:
        scale = float(out_m.abs().max())
        assert float((out_f - out_m).abs().max()) <= 1e-6 * max(1.0, scale) * max(1.0, (Kd / 64) ** 0.5), what
    # and the product itself, against fp32 torch on the materialized operand
    ref = torch.bmm(a.double(), (bt.transpose(1, 2) if bt_rows else bt).double().transpose(1, 2).contiguous())
    tot = out_f.reshape(B, ksplit, M, N).double().sum(1)
    tol = {"bf16": 2e-2, "bf16x3": 1e-4}.get(mode, 1e-5)
    assert_fp32(tot.cpu().numpy(), ref.cpu().numpy(), rtol=0.0,
                atol=tol * max(1.0, float(ref.abs().max())) * max(1.0, (Kd / 64) ** 0.5), what=what)


def test_a_prologue_inf_takes_the_fp32_fallback_like_the_materialized_operand():
    from pdum_dsl_amd import kernels as K

    B, M, N, Kd = 1, 128, 96, 200
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(B, M, Kd, device="cuda", generator=g)
    x[0, 7, 11] = 1e30  # x * s overflows fp32 in the prologue: an inf in a's row 7
    s = torch.full((B, Kd), 1e10, device="cuda")
    bt = torch.randn(B, N, Kd, device="cuda", generator=g)
    pa = _programs(B, M, N, Kd, x, s)
    out_f = torch.empty(B, M, N, device="cuda")
    out_m = torch.empty_like(out_f)
    K.contract_views_pro(None, None, bt, bt.stride(), (B, M, N, Kd), _identity((B, M, N), out_f), [], out_f,
                         pro_a=(pa, [x, s]))
    a = torch.empty(B, M, Kd, device="cuda")
    K.map_chain(pa, [x, s], a)
    K.contract_views(a, a.stride(), bt, bt.stride(), (B, M, N, Kd), _identity((B, M, N), out_m), [], out_m)
    torch.cuda.synchronize()
    assert bool(torch.isinf(a).any())
    assert torch.equal(torch.isnan(out_f), torch.isnan(out_m)) and torch.equal(torch.isinf(out_f), torch.isinf(out_m))
    fin = torch.isfinite(out_m)
    assert float((out_f[fin] - out_m[fin]).abs().max()) <= 1e-5 * max(1.0, float(out_m[fin].abs().max()))


def test_a_prologue_over_the_wrong_lattice_is_refused_before_launch():
    from pdum_dsl_amd import _lib as L
    from pdum_dsl_amd import kernels as K

    B, M, N, Kd = 1, 64, 64, 96
    x = torch.randn(B, M, Kd, device="cuda")
    s = torch.ones(B, Kd, device="cuda")
    bt = torch.randn(B, N, Kd, device="cuda")
    pa = _programs(B, M + 1, N, Kd, x, s)  # rows one too many
    out = torch.empty(B, M, N, device="cuda")
    with pytest.raises(ValueError):
        K.contract_views_pro(None, None, bt, bt.stride(), (B, M, N, Kd), _identity((B, M, N), out), [], out,
                             pro_a=(pa, [x, s]))
    # the C entry point refuses it too (status, no launch)
    import ctypes as C

    table = (C.c_void_p * 2)(x.data_ptr(), s.data_ptr())
    rc = L.lib().pdh_contract_views_pro(None, 0, 0, 1, C.byref(pa), table, C.c_void_p(bt.data_ptr()), *bt.stride(),
                                        None, None, B, M, N, Kd, 1, C.byref(_identity((B, M, N), out)), None,
                                        C.c_void_p(out.data_ptr()), 0, None)
    assert rc != 0


@pytest.mark.parametrize("M,K,N", [(96, 160, 72), (130, 1001, 70), (300, 640, 260)])
def test_bf16_prologue_chains_are_computed_in_the_k_loop(M, K, N):
    """At bf16 storage the seat computes the chain operand in the k loop too
    (the param through a one-LOAD program), against the oracle on the same
    bf16-rounded inputs."""
    from tests.test_gpu_contract import _bf16

    region, vals = _gelu_chain_subject(M, K, N, seed=M + 1)
    _g, run = _seat(region, "bf16")
    assert run.source.startswith("hip:contract_views_pro") and "prologue=chain,param" in run.source
    got = run(vals)
    _check(got, _oracle(region, [_bf16(v) for v in vals], ("t", "f")), "bf16", f"bf16 gelu(x) @ w + b {M}x{K}x{N}",
           k=K)


@pytest.mark.parametrize("jit", [True, False])
@pytest.mark.parametrize("B,M,N,Kd", [(2, 130, 200, 333), (1, 300, 260, 700), (3, 64, 64, 5)])
def test_bf16_computed_operands_match_the_materialized_ones(jit, B, M, N, Kd):
    """bf16: the a prologue computed in the k loop and bt through a one-LOAD
    program, against the operand materialized by the same program (a bf16
    buffer) and the product of the bf16 operands by the 16-bit kernel."""
    from pdum_dsl_amd import _lib as L
    from pdum_dsl_amd import kernels as K

    g = torch.Generator(device="cuda").manual_seed(B * 7 + Kd)
    x = torch.randn(B, M, Kd, device="cuda", generator=g).to(torch.bfloat16)
    s = (1.0 + 0.1 * torch.randn(B, Kd, device="cuda", generator=g)).to(torch.bfloat16)
    bt = torch.randn(B, N, Kd, device="cuda", generator=g).to(torch.bfloat16)
    pa = _programs(B, M, N, Kd, x, s)
    out_f = torch.empty(B, M, N, device="cuda", dtype=torch.bfloat16)
    prev = L.lib().pdh_ew_set_jit(1 if jit else 0)
    try:
        K.contract_views_pro(None, None, None, None, (B, M, N, Kd), _identity((B, M, N), out_f), [], out_f,
                             pro_a=(pa, [x, s]), pro_b=(K.view_program((B, N, Kd), bt.stride()), [bt]))
        a = torch.empty(B, M, Kd, device="cuda", dtype=torch.bfloat16)
        K.map_chain(pa, [x, s], a)
        torch.cuda.synchronize()
    finally:
        L.lib().pdh_ew_set_jit(prev)
    ref = torch.bmm(a.double(), bt.double().transpose(1, 2).contiguous())
    got = out_f.double()
    what = f"bf16 jit={jit} B{B} M{M} N{N} K{Kd}"
    # fp32 accumulation of the bf16 operands' exact products, one bf16 rounding of the result
    scale = float(ref.abs().max())
    assert float((got - ref).abs().max()) <= 2 ** -8 * scale + 1e-6 * scale * max(1.0, (Kd / 64) ** 0.5), what


def test_f16_prologues_are_refused():
    from pdum_dsl_amd import _lib as L
    from pdum_dsl_amd import kernels as K

    B, M, N, Kd = 1, 64, 64, 64
    x = torch.randn(B, M, Kd, device="cuda").half()
    bt = torch.randn(B, N, Kd, device="cuda").half()
    out = torch.empty(B, M, N, device="cuda").half()
    with pytest.raises((ValueError, L.PdhError)):
        K.contract_views_pro(None, None, None, None, (B, M, N, Kd), _identity((B, M, N), out), [], out,
                             pro_a=(K.view_program((B, M, Kd), x.stride()), [x]),
                             pro_b=(K.view_program((B, N, Kd), bt.stride()), [bt]))
