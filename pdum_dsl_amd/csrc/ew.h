// The elementwise-program interpreter shared by the map-chain kernel and the
// contraction epilogue (program format: pdh_ew_program in include/pdhip.h).
//
// Every lane runs the same instruction stream, read from the kernel
// arguments: the opcode and register numbers are wave-uniform (scalar
// registers), so the dispatch is a scalar branch and the register file is an
// fp32 vector indexed in VGPR-indexing mode (s_set_gpr_idx), not scratch.
// EPT elements per lane share each decoded instruction.
#pragma once

#include "dev.h"

namespace pdh {

struct EwOperands {
  const void* p[PDH_EW_MAX_OPERANDS];
};

__device__ __forceinline__ float ew_load(const void* base, int off, int dtype) {
  if (dtype == PDH_F32) return ld_dt<PDH_F32>(base, off);
  return dtype == PDH_BF16 ? ld_dt<PDH_BF16>(base, off) : ld_dt<PDH_F16>(base, off);
}

__device__ __forceinline__ void ew_store(void* base, long long off, float v, int dtype) {
  if (dtype == PDH_F32)
    st_dt<PDH_F32>(base, off, v);
  else if (dtype == PDH_BF16)
    st_dt<PDH_BF16>(base, off, v);
  else
    st_dt<PDH_F16>(base, off, v);
}

// The interpreter as an evaluator policy (the runtime-specialized kernels
// substitute a generated one with the same interface).
struct InterpEval;

// Runs program p for EPT elements: the element at output coordinates c0
// and EPT - 1 more along the last output dim, es apart (every caller's
// elements lie on one row: es = 1 for consecutive columns, es = 64 when a
// wave's lanes take consecutive columns). acc[e] is what PDH_EW_ACC reads;
// returns r[out_reg] in res. Each instruction is decoded and dispatched once
// for all EPT elements; operand offsets are 32-bit (callers keep every view
// under 2^31 elements).
template <int EPT>
__device__ __forceinline__ void ew_run(const pdh_ew_program& p, const EwOperands& ops, int dtype,
                                       const int (&c0)[PDH_EW_MAX_DIMS], const float (&acc)[EPT],
                                       float (&res)[EPT], int es) {
  f32x16 r[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) r[e] = f32x16{};
  const int n = __builtin_amdgcn_readfirstlane(p.n_insns);
  const int ndim = __builtin_amdgcn_readfirstlane(p.ndim);
  const int last = ndim - 1;
  // the next instruction's scalar load is issued before this one executes
  pdh_ew_insn cur = p.insns[0];
  for (int pc = 0; pc < n; ++pc) {
    const pdh_ew_insn nxt = p.insns[pc + 1 < n ? pc + 1 : pc];
    const int op = __builtin_amdgcn_readfirstlane(cur.op);
    const int d = __builtin_amdgcn_readfirstlane(cur.dst);
    const int ia = __builtin_amdgcn_readfirstlane(cur.a);
    const int ib = __builtin_amdgcn_readfirstlane(cur.b);
    const int ic = __builtin_amdgcn_readfirstlane(cur.c);
    // operands read once, results written once: the register file is only
    // ever touched by single indexed moves, never copied
    float x[EPT], y[EPT], z[EPT], v[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      x[e] = r[e][ia];
      y[e] = r[e][ib];
      z[e] = r[e][ic];
    }
    switch (op) {
      case PDH_EW_LOAD: {
        int off = 0;
#pragma unroll
        for (int dd = 0; dd < PDH_EW_MAX_DIMS; ++dd)
          if (dd < ndim) off += c0[dd] * static_cast<int>(p.in_stride[ia][dd]);
        const int step = es * static_cast<int>(p.in_stride[ia][last]);
        const void* base = ops.p[ia];
#pragma unroll
        for (int e = 0; e < EPT; ++e) v[e] = ew_load(base, off + e * step, dtype);
        break;
      }
      case PDH_EW_ACC:
#pragma unroll
        for (int e = 0; e < EPT; ++e) v[e] = acc[e];
        break;
      case PDH_EW_CONST:
#pragma unroll
        for (int e = 0; e < EPT; ++e) v[e] = cur.imm;
        break;
      case PDH_EW_IOTA: {
        int c = 0;
#pragma unroll
        for (int dd = 0; dd < PDH_EW_MAX_DIMS; ++dd)
          if (dd == ia) c = c0[dd] + static_cast<int>(p.start[dd]);
        const int inc = ia == last ? es : 0;
#pragma unroll
        for (int e = 0; e < EPT; ++e) v[e] = static_cast<float>(c + e * inc);
        break;
      }
#define PDH_EW_CASE(OPC, EXPR)             \
  case OPC:                                \
    _Pragma("unroll") for (int e = 0; e < EPT; ++e) { \
      const float a_ = x[e], b_ = y[e];    \
      (void)b_;                            \
      v[e] = (EXPR);                       \
    }                                      \
    break;
      PDH_EW_CASE(PDH_EW_NEG, -a_)
      PDH_EW_CASE(PDH_EW_EXP, expf(a_))
      PDH_EW_CASE(PDH_EW_LOG, logf(a_))
      PDH_EW_CASE(PDH_EW_SQRT, sqrtf(a_))
      PDH_EW_CASE(PDH_EW_TANH, pdh_tanh(a_))
      PDH_EW_CASE(PDH_EW_SIN, sinf(a_))
      PDH_EW_CASE(PDH_EW_COS, cosf(a_))
      PDH_EW_CASE(PDH_EW_ABS, fabsf(a_))
      PDH_EW_CASE(PDH_EW_FLOOR, floorf(a_))
      PDH_EW_CASE(PDH_EW_ADD, a_ + b_)
      PDH_EW_CASE(PDH_EW_SUB, a_ - b_)
      PDH_EW_CASE(PDH_EW_MUL, a_ * b_)
      PDH_EW_CASE(PDH_EW_DIV, a_ / b_)
      PDH_EW_CASE(PDH_EW_MAX, nan_max(a_, b_))
      PDH_EW_CASE(PDH_EW_MIN, nan_min(a_, b_))
      PDH_EW_CASE(PDH_EW_EQ, a_ == b_ ? 1.f : 0.f)
      PDH_EW_CASE(PDH_EW_NE, a_ != b_ ? 1.f : 0.f)
      PDH_EW_CASE(PDH_EW_LT, a_ < b_ ? 1.f : 0.f)
      PDH_EW_CASE(PDH_EW_LE, a_ <= b_ ? 1.f : 0.f)
      PDH_EW_CASE(PDH_EW_GT, a_ > b_ ? 1.f : 0.f)
      PDH_EW_CASE(PDH_EW_GE, a_ >= b_ ? 1.f : 0.f)
      PDH_EW_CASE(PDH_EW_RBF16, bf16_to_f32(f32_to_bf16(a_)))
      PDH_EW_CASE(PDH_EW_RF16, f16_to_f32(f32_to_f16(a_)))
#undef PDH_EW_CASE
      default:  // PDH_EW_WHERE
#pragma unroll
        for (int e = 0; e < EPT; ++e) v[e] = x[e] != 0.f ? y[e] : z[e];
        break;
    }
#pragma unroll
    for (int e = 0; e < EPT; ++e) r[e][d] = v[e];
    cur = nxt;
  }
  const int o = __builtin_amdgcn_readfirstlane(p.out_reg);
#pragma unroll
  for (int e = 0; e < EPT; ++e) res[e] = r[e][o];
}

struct InterpEval {
  static constexpr bool kVec = false;  // operands read element by element
  // outputs per lane and call in the contraction's store: the interpreter's
  // register file is 16 floats per element, so it runs four at a time
  static constexpr int kStoreRun = 4;
  template <int EPT>
  static __device__ __forceinline__ void run(const pdh_ew_program& p, const EwOperands& ops, int dtype,
                                             const int (&c0)[PDH_EW_MAX_DIMS], const float (&acc)[EPT],
                                             float (&res)[EPT], int es) {
    ew_run<EPT>(p, ops, dtype, c0, acc, res, es);
  }
};

}  // namespace pdh
