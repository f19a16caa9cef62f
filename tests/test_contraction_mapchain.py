"""The contraction-epilogue and map-chain templates on the CPU.

Restates the reference's battery for these rows
(packages/tensorlib/tests/test_fusion.py:21-73, 97-110): recognition, the
generated k-tiled fold, and certification — proved-licensed under
gemm.k-reassoc for a sum (normalization inlines the fold back to one
reduce), licensed-differential for a mean (its finalize is not syntax the
normalizer walks back), proved-exact for map chains. Values are checked
against numpy closed forms and the float64 oracle evaluator.

The HIP seat's lowering of chains to elementwise register programs
(pdum_dsl_amd.ewprog) is pinned here by a numpy emulation of the program
format (include/pdhip.h's opcode table) run against the oracle's evaluation
of the same region — the lowering, not the kernel, is what this checks; the
kernel is pinned on the GPU (test_gpu_contract.py)."""

import ctypes as C
import re
import subprocess
import tempfile
from pathlib import Path

import numpy as np
import pytest

from oracle import region_eval as rev
from pdum_dsl_amd import _lib as L
from pdum_dsl_amd import ewprog
from pdum_dsl_amd import hip_tile as H
from pdum_dsl_amd.tl import fusion, interp
from pdum_dsl_amd.tl.dialect import OPS
from pdum_dsl_amd.tl.ir import F64, Builder, Dim, Region, tensor_type, walk_deep

REPO = Path(__file__).resolve().parents[1]


def _c(b, v):
    return b.emit("core.const", type=F64, value=float(v))


def gemm_subject(M=6, K=8, N=5, *, epilogue="relu_bias", seed=3, f="sum", rider=None):
    """y = relu(a @ b + bias) (test_fusion.py:21-42), optionally batched over a rider dim."""
    rng = np.random.default_rng(seed)
    b = Builder(OPS)
    an, bn = ("m", "k"), ("k", "n")
    ash, bsh = (M, K), (K, N)
    if rider is not None:
        an, bn = (rider[0],) + an, (rider[0],) + bn
        ash, bsh = (rider[1],) + ash, (rider[1],) + bsh
    pa = b.param(0, tensor_type(an, ash))
    pb = b.param(1, tensor_type(bn, bsh))
    prod = b.emit("tl.pointwise", b.emit("tl.repeat_like", pa, pb), b.emit("tl.repeat_like", pb, pa), f="mul")
    z = b.emit("tl.reduce", prod, dims=("k",), f=f)
    vals = [rng.standard_normal(ash), rng.standard_normal(bsh)]
    params = [pa, pb]
    if epilogue == "relu_bias":
        pc = b.param(2, tensor_type(("n",), (N,)))
        zb = b.emit("tl.pointwise", z, b.emit("tl.repeat_like", pc, z), f="add")
        y = b.emit("tl.pointwise", zb, _c(b, 0.0), f="maximum")
        params.append(pc)
        vals.append(rng.standard_normal(N))
    elif epilogue == "gelu_tanh":  # 0.5 z (1 + tanh(0.79788456 (z + 0.044715 z^3)))
        z3 = b.emit("tl.pointwise", b.emit("tl.pointwise", z, z, f="mul"), z, f="mul")
        inner = b.emit("tl.pointwise", z, b.emit("tl.pointwise", z3, _c(b, 0.044715), f="mul"), f="add")
        t = b.emit("tl.pointwise", b.emit("tl.pointwise", inner, _c(b, 0.7978845608028654), f="mul"), f="tanh")
        y = b.emit("tl.pointwise", b.emit("tl.pointwise", z, _c(b, 0.5), f="mul"),
                   b.emit("tl.pointwise", t, _c(b, 1.0), f="add"), f="mul")
    else:
        y = z
    region = Region(params=tuple(params), body=(b.emit("core.yield", y),))
    return region, vals


def _fields(region, vals):
    return [interp.field(v, p.type.names) for p, v in zip(region.params, vals)]


def _oracle(region, vals, names):
    vs = [rev.value(v, p.type) for v, p in zip(vals, region.params)]
    res = rev.evaluate(region, vs)
    return (res[0] if isinstance(res, (tuple, list)) else res).numpy(names)


# ------------------------------------------------------------ recognition


def test_contraction_with_epilogue_is_recognized_and_proved():
    region, vals = gemm_subject()
    (g,) = fusion.plan_region(region).groups
    assert g.template == "contraction-epilogue"
    assert g.certificate.verdict == "proved-licensed"
    assert g.certificate.licenses == ("gemm.k-reassoc",)
    assert g.confidence == "yellow"
    assert dict(g.params)["ki"] == 4 and dict(g.params)["shape"] == "gemm"  # K = 8: largest divisor with >= 2 tiles
    got = interp.run_region(g.kernel, _fields(region, vals)).to_numpy(("m", "n"))
    want = interp.run_region(region, _fields(region, vals)).to_numpy(("m", "n"))
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)
    ref = np.maximum(vals[0] @ vals[1] + vals[2], 0.0)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-7)
    # the oracle's own interpreter agrees on the generated fold
    np.testing.assert_allclose(_oracle(g.kernel, vals, ("m", "n")), ref, rtol=1e-12, atol=1e-12)


def test_bare_contraction_is_recognized_too():
    region, _ = gemm_subject(epilogue=None)
    (g,) = fusion.plan_region(region).groups
    assert g.template == "contraction-epilogue" and g.certificate.verdict == "proved-licensed"


def test_a_mean_contraction_certifies_by_differential():
    region, vals = gemm_subject(epilogue=None, f="mean")
    (g,) = fusion.plan_region(region).groups
    assert g.template == "contraction-epilogue"
    assert g.certificate.verdict == "licensed-differential" and g.certificate.families == ("unit", "wide")
    got = interp.run_region(g.kernel, _fields(region, vals)).to_numpy(("m", "n"))
    np.testing.assert_allclose(got, vals[0] @ vals[1] / 8.0, rtol=1e-12, atol=1e-12)


def test_rowsum_and_plain_shapes_are_recognized():
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "s"), (4, 12)))
    z = b.param(1, tensor_type(("t", "s"), (4, 12)))
    rs = b.emit("tl.reduce", b.emit("tl.pointwise", x, z, f="mul"), dims=("s",), f="sum")
    (g,) = fusion.plan_region(Region(params=(x, z), body=(b.emit("core.yield", rs),))).groups
    assert (g.template, dict(g.params)["shape"], g.certificate.verdict) == ("contraction-epilogue", "rowsum",
                                                                           "proved-licensed")
    b = Builder(OPS)
    x = b.param(0, tensor_type(("t", "s"), (4, 12)))
    pl = b.emit("tl.reduce", x, dims=("t",), f="sum")
    (g,) = fusion.plan_region(Region(params=(x,), body=(b.emit("core.yield", pl),))).groups
    assert (g.template, dict(g.params)["shape"]) == ("contraction-epilogue", "plain")


def test_softmax_and_layernorm_are_not_contractions():
    from pdum_dsl_amd.tl import zoo

    assert fusion.match_contraction_epilogue(zoo.row_softmax().region) is None
    assert fusion.match_contraction_epilogue(zoo.layernorm().region) is None


def test_map_chains_are_recognized_and_exact():
    b = Builder(OPS)
    x = b.param(0, tensor_type(("x", "y"), (4, 6)))
    y = b.emit("tl.pointwise", x, f="exp")
    (g,) = fusion.plan_region(Region(params=(x,), body=(b.emit("core.yield", y),))).groups
    assert (g.template, g.certificate.verdict) == ("map-chain", "proved-exact")


# ------------------------------------------------------- program lowering

_NP = {
    "NEG": np.negative, "EXP": np.exp, "LOG": np.log, "SQRT": np.sqrt, "TANH": np.tanh, "SIN": np.sin,
    "COS": np.cos, "ABS": np.abs, "FLOOR": np.floor, "ADD": np.add, "SUB": np.subtract, "MUL": np.multiply,
    "DIV": np.divide, "MAX": np.maximum, "MIN": np.minimum,
    "EQ": np.equal, "NE": np.not_equal, "LT": np.less, "LE": np.less_equal, "GT": np.greater, "GE": np.greater_equal,
}


def emulate(low: ewprog.Lowered, operands: list, acc=None) -> np.ndarray:
    """The elementwise program format, evaluated with numpy over the whole
    lattice (float64): every register is a lattice-shaped array."""
    shape = tuple(d.size for d in low.dims)
    names = tuple(d.name for d in low.dims)
    regs = [None] * L.EW_MAX_REGS
    for op, dst, a, b, c, imm in low.insns:
        if op == "LOAD":
            node, arr = low.operands[a], operands[a]
            order = [node.type.names.index(n) for n in names if n in node.type.names]
            v = np.transpose(arr, order)
            v = v.reshape([v.shape[order.index(node.type.names.index(n))] if n in node.type.names else 1
                           for n in names])
            regs[dst] = np.broadcast_to(v, shape).astype(np.float64)
        elif op == "ACC":
            regs[dst] = np.broadcast_to(acc, shape)
        elif op == "CONST":
            regs[dst] = np.full(shape, imm, dtype=np.float64)
        elif op == "IOTA":
            d = low.dims[a]
            sh = [1] * len(shape)
            sh[a] = d.size
            regs[dst] = np.broadcast_to(np.arange(d.start, d.stop, dtype=np.float64).reshape(sh), shape)
        elif op == "WHERE":
            regs[dst] = np.where(regs[a] != 0, regs[b], regs[c])
        elif op in ("NEG", "EXP", "LOG", "SQRT", "TANH", "SIN", "COS", "ABS", "FLOOR"):
            regs[dst] = _NP[op](regs[a])
        else:
            regs[dst] = _NP[op](regs[a], regs[b]).astype(np.float64)
    return regs[low.out_reg]


def chain_subject(seed=1, I=5, J=7):
    """A chain over broadcast operands, iotas and a mask: where(iota_j > iota_i,
    tanh(x * s_j) + exp(-|x|), 0) with s:(j,) broadcast over (i, j)."""
    rng = np.random.default_rng(seed)
    b = Builder(OPS)
    x = b.param(0, tensor_type(("i", "j"), (I, J)))
    s = b.param(1, tensor_type(("j",), (J,)))
    sx = b.emit("tl.pointwise", x, b.emit("tl.repeat_like", s, x), f="mul")
    t = b.emit("tl.pointwise", sx, f="tanh")
    e = b.emit("tl.pointwise", b.emit("tl.pointwise", b.emit("tl.pointwise", x, f="abs"), f="neg"), f="exp")
    lat = b.emit("tl.const", value=0.0, dims=(("i", I), ("j", J)))
    ii = b.emit("tl.iota", lat, name="i")
    jj = b.emit("tl.iota", lat, name="j")
    m = b.emit("tl.pointwise", jj, ii, f="gt")
    y = b.emit("tl.pointwise", m, b.emit("tl.pointwise", t, e, f="add"), _c(b, 0.0), f="where")
    region = Region(params=(x, s), body=(b.emit("core.yield", y),))
    return region, [rng.standard_normal((I, J)), rng.standard_normal(J)]


def test_the_lowered_chain_computes_the_oracle_values():
    region, vals = chain_subject()
    y = region.body[-1].args[0]
    low = ewprog.lower(y, y.type.dims, {id(p): p for p in region.params})
    assert low.operands == region.params  # LOAD slots in first-use order
    got = emulate(low, vals)
    want = _oracle(region, vals, y.type.names)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # and the closed form: where(j > i, tanh(x s) + exp(-|x|), 0)
    x, s = vals
    i, j = np.meshgrid(np.arange(5), np.arange(7), indexing="ij")
    np.testing.assert_allclose(got, np.where(j > i, np.tanh(x * s) + np.exp(-np.abs(x)), 0.0), rtol=1e-12)


def test_the_lowered_epilogue_reads_the_accumulator():
    for epi in ("relu_bias", "gelu_tanh"):
        region, vals = gemm_subject(M=4, K=16, N=3, epilogue=epi)
        (g,) = fusion.plan_region(region).groups
        cb = H.recognize_contraction(g.kernel)
        assert cb is not None and (cb["m"], cb["n"], cb["rider"], cb["K"]) == ("m", "n", None, 16)
        y = g.kernel.body[-1].args[0]
        lat = (Dim("_unit0", 0, 1),) + tuple(cb["fold"].type.dim(nm) for nm in ("m", "n"))
        low = ewprog.lower(y, lat, {id(p): p for p in g.kernel.params}, acc=cb["fold"])
        acc = (vals[0] @ vals[1]).reshape(1, 4, 3)
        ops = [vals[g.kernel.params.index(p)] for p in low.operands]
        got = emulate(low, ops, acc=acc)[0]
        np.testing.assert_allclose(got, _oracle(region, vals, ("m", "n")), rtol=1e-12, atol=1e-12)


def test_register_pressure_and_operand_limits_refuse():
    b = Builder(OPS)
    ps = [b.param(i, tensor_type(("x",), (4,))) for i in range(9)]
    acc = ps[0]
    for p in ps[1:]:
        acc = b.emit("tl.pointwise", acc, p, f="add")
    with pytest.raises(ewprog.Unlowerable, match="operands"):
        ewprog.lower(acc, acc.type.dims, {id(p): p for p in ps})
    # 17 terms folded left: each is freed once used, so the chain fits the register file
    b = Builder(OPS)
    x = b.param(0, tensor_type(("x",), (4,)))
    leaves = [b.emit("tl.pointwise", x, _c(b, float(i)), f="add") for i in range(17)]
    tot = leaves[0]
    for lf in leaves[1:]:
        tot = b.emit("tl.pointwise", tot, lf, f="mul")
    low = ewprog.lower(tot, tot.type.dims, {id(x): x})
    assert len(low.insns) <= L.EW_MAX_INSNS and max(i[1] for i in low.insns) < 4


def test_the_program_struct_matches_the_c_header():
    src = f"""
#include "{REPO / 'include' / 'pdhip.h'}"
#include <stdio.h>
#include <stddef.h>
int main(void) {{
  printf("%zu %zu %zu %zu %zu %d\\n", sizeof(pdh_ew_insn), sizeof(pdh_ew_program),
         offsetof(pdh_ew_program, in_stride), offsetof(pdh_ew_program, insns), offsetof(pdh_ew_insn, imm),
         (int)PDH_EW_NOPS);
  return 0;
}}
"""
    with tempfile.TemporaryDirectory() as tmp:
        c = Path(tmp) / "s.c"
        c.write_text(src)
        exe = Path(tmp) / "s"
        subprocess.run(["gcc", str(c), "-o", str(exe)], check=True, capture_output=True)
        got = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    want = [C.sizeof(L.EwInsn), C.sizeof(L.EwProgram), L.EwProgram.in_stride.offset, L.EwProgram.insns.offset,
            L.EwInsn.imm.offset, len(L.EW_OPS)]
    assert [int(v) for v in got] == want


def test_contraction_binding_reads_riders_and_refuses_more():
    region, _ = gemm_subject(M=4, K=16, N=3, epilogue=None, rider=("h", 2))
    (g,) = fusion.plan_region(region).groups
    cb = H.recognize_contraction(g.kernel)
    assert (cb["rider"], cb["m"], cb["n"]) == ("h", "m", "n")
    assert sum(1 for n in walk_deep(g.kernel) if n.op == "tl.fold") == 1


# --------------------------------------------- runtime specialization (hipRTC)


def _zoo_programs():
    from pdum_dsl_amd.tl import zoo

    subj = zoo.linear_gelu(T=64, D=128, F=96)
    (g,) = fusion.plan_region(subj.region).groups
    cb = H.recognize_contraction(g.kernel)
    lat = (Dim("_u", 0, 1), cb["fold"].type.dim("t"), cb["fold"].type.dim("f"))
    low = ewprog.lower(g.kernel.body[-1].args[0], lat, {id(p): p for p in g.kernel.params}, acc=cb["fold"])
    epi = low.program([0, 96, 1], [[0, 0, 1]])
    m = zoo.masked_activation(I=8, J=16)
    (g2,) = fusion.plan_region(m.region).groups
    y = g2.kernel.body[-1].args[0]
    low2 = ewprog.lower(y, y.type.dims, {id(p): p for p in g2.kernel.params})
    chain = low2.program([16, 1], [[16, 1], [0, 1]])
    return epi, chain


def test_specialized_kernels_compile_offline_for_every_element_type():
    """The generated straight-line evaluators compile with hipRTC (no GPU
    needed) for both templates and all three element types, and the source
    carries the program: constants as exact hex floats, one statement per
    instruction."""
    lib = L.lib()
    epi, chain = _zoo_programs()
    for kind, prog in ((1, epi), (0, chain)):
        for dt in (L.PDH_F32, L.PDH_BF16, L.PDH_F16):
            rc = lib.pdh_ew_jit_compile(C.byref(prog), kind, dt)
            assert rc == 0, L.last_error()
    buf = C.create_string_buffer(1 << 16)
    n = lib.pdh_ew_jit_source(C.byref(epi), 1, L.PDH_BF16, buf, len(buf))
    src = buf.value.decode()
    assert n == len(src) and "0x1.988454p-1f" in src and "pdh_tanh(" in src and "acc[e]" in src
    assert len(re.findall(r"^      r\d+ = ", src, re.M)) == epi.n_insns  # one statement per instruction
    assert "contract_mfma_body<PDH_BF16, 64, pdh::GenEval>" in src and "contract_mfma_body<PDH_BF16, 32, pdh::GenEval>" in src


def test_fp32_contractions_compile_in_every_mode():
    """fp32 contractions run on the bf16 matrix cores (operands split into
    bf16 planes, 6 or 3 cross products per term) or by VALU fma; the mode is
    process-wide, refused outside {0, 3, 6}, and each mode's specialized
    kernels compile offline."""
    lib = L.lib()
    epi, _chain = _zoo_programs()
    prev = lib.pdh_contract_set_f32_mode(3)
    try:
        assert prev == 6  # the default: fp32 grade
        assert lib.pdh_contract_set_f32_mode(7) == L.PDH_EINVAL and "mode 7" in L.last_error()
        buf = C.create_string_buffer(1 << 16)
        for mode, body in ((6, "contract_split_body<PDH_F32, 64, 6, 0, pdh::GenEval, -1>"),
                           (3, "contract_split_body<PDH_F32, 32, 3, 0, pdh::GenEval, -1>"),
                           (0, "contract_f32_body<pdh::GenEval, -1>")):
            lib.pdh_contract_set_f32_mode(mode)
            assert lib.pdh_ew_jit_compile(C.byref(epi), 1, L.PDH_F32) == 0, L.last_error()
            lib.pdh_ew_jit_source(C.byref(epi), 1, L.PDH_F32, buf, len(buf))
            assert body in buf.value.decode()
        # the rows-contiguous operand layouts of pdh_contract_views (kinds 2..4: a, bt, both)
        lib.pdh_contract_set_f32_mode(6)
        for kind in (2, 3, 4):
            assert lib.pdh_ew_jit_compile(C.byref(epi), kind, L.PDH_F32) == 0, L.last_error()
            lib.pdh_ew_jit_source(C.byref(epi), kind, L.PDH_F32, buf, len(buf))
            assert f"contract_split_body<PDH_F32, 64, 6, {kind - 1}, pdh::GenEval, -1>" in buf.value.decode()
        # row partials (kinds 5..7: sum, max, min) for pdh_contract_views_rowred
        for kind in (5, 6, 7):
            assert lib.pdh_ew_jit_compile(C.byref(epi), kind, L.PDH_F32) == 0, L.last_error()
            lib.pdh_ew_jit_source(C.byref(epi), kind, L.PDH_F32, buf, len(buf))
            assert f"contract_split_body<PDH_F32, 64, 6, 0, pdh::GenEval, {kind - 5}>" in buf.value.decode()
    finally:
        lib.pdh_contract_set_f32_mode(prev)


def test_the_tanh_identity_the_kernels_use_is_accurate_in_fp32():
    """dev.h's pdh_tanh: tanh|x| = 1 - 2 / (2^(2|x| log2 e) + 1), sign copied.
    The same float32 steps in numpy (exp2 and a correctly rounded reciprocal
    stand in for v_exp_f32 / v_rcp_f32, each within about an ulp) stay within
    3e-7 of tanh over the whole line, are odd, and saturate to exactly 1."""
    x = np.concatenate([np.linspace(-20, 20, 200001), np.geomspace(1e-30, 1e-3, 1000)]).astype(np.float32)
    ax = np.abs(x)
    e = np.exp2(ax * np.float32(2.8853900817779268))
    t = np.float32(1) - np.float32(2) * (np.float32(1) / (e + np.float32(1)))
    got = np.copysign(t, x)
    assert np.abs(got.astype(np.float64) - np.tanh(x.astype(np.float64))).max() < 3e-7
    assert np.all(got[x >= 10] == 1.0) and np.array_equal(np.copysign(t, -x), -got)
    assert abs(2.8853900817779268 - 2 / np.log(2)) < 1e-15
