// The elementwise-program interpreter shared by the map-chain kernel and the
// contraction epilogue (program format: pdh_ew_program in include/pdhip.h).
//
// Every lane runs the same instruction stream, read from the kernel
// arguments: the opcode and register numbers are wave-uniform (scalar
// registers), so the dispatch is a scalar branch and the register file is an
// fp32 vector indexed in VGPR-indexing mode (s_set_gpr_idx), not scratch.
// EPT elements per lane share each decoded instruction.
#pragma once

#include "common.h"

namespace pdh {

struct EwOperands {
  const void* p[PDH_EW_MAX_OPERANDS];
};

__device__ __forceinline__ float ew_load(const void* base, int off, int dtype) {
  if (dtype == PDH_F32) return static_cast<const float*>(base)[off];
  const uint16_t b = static_cast<const uint16_t*>(base)[off];
  return dtype == PDH_BF16 ? Elem<__hip_bfloat16>::to_f32(b) : Elem<_Float16>::to_f32(b);
}

__device__ __forceinline__ void ew_store(void* base, int64_t off, float v, int dtype) {
  if (dtype == PDH_F32)
    static_cast<float*>(base)[off] = v;
  else if (dtype == PDH_BF16)
    static_cast<uint16_t*>(base)[off] = Elem<__hip_bfloat16>::from_f32(v);
  else
    static_cast<uint16_t*>(base)[off] = Elem<_Float16>::from_f32(v);
}

// Runs program p for EPT elements: the element at output coordinates c0
// and the next EPT - 1 along the last output dim (every caller's elements
// are consecutive there). acc[e] is what PDH_EW_ACC reads; returns
// r[out_reg] in res. Each instruction is decoded and dispatched once for
// all EPT elements; operand offsets are 32-bit (callers keep every view
// under 2^31 elements).
template <int EPT>
__device__ __forceinline__ void ew_run(const pdh_ew_program& p, const EwOperands& ops, int dtype,
                                       const int (&c0)[PDH_EW_MAX_DIMS], const float (&acc)[EPT],
                                       float (&res)[EPT]) {
  f32x16 r[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) r[e] = f32x16{};
  const int n = __builtin_amdgcn_readfirstlane(p.n_insns);
  const int ndim = __builtin_amdgcn_readfirstlane(p.ndim);
  const int last = ndim - 1;
  for (int pc = 0; pc < n; ++pc) {
    const pdh_ew_insn in = p.insns[pc];
    const int op = __builtin_amdgcn_readfirstlane(in.op);
    const int d = __builtin_amdgcn_readfirstlane(in.dst);
    const int ia = __builtin_amdgcn_readfirstlane(in.a);
    const int ib = __builtin_amdgcn_readfirstlane(in.b);
    const int ic = __builtin_amdgcn_readfirstlane(in.c);
    auto un = [&](auto f) {
#pragma unroll
      for (int e = 0; e < EPT; ++e) r[e][d] = f(r[e][ia]);
    };
    auto bin = [&](auto f) {
#pragma unroll
      for (int e = 0; e < EPT; ++e) r[e][d] = f(r[e][ia], r[e][ib]);
    };
    switch (op) {
      case PDH_EW_LOAD: {
        int off = 0;
#pragma unroll
        for (int dd = 0; dd < PDH_EW_MAX_DIMS; ++dd)
          if (dd < ndim) off += c0[dd] * static_cast<int>(p.in_stride[ia][dd]);
        const int step = static_cast<int>(p.in_stride[ia][last]);
        const void* base = ops.p[ia];
#pragma unroll
        for (int e = 0; e < EPT; ++e) r[e][d] = ew_load(base, off + e * step, dtype);
        break;
      }
      case PDH_EW_ACC:
#pragma unroll
        for (int e = 0; e < EPT; ++e) r[e][d] = acc[e];
        break;
      case PDH_EW_CONST:
#pragma unroll
        for (int e = 0; e < EPT; ++e) r[e][d] = in.imm;
        break;
      case PDH_EW_IOTA: {
        int c = 0;
#pragma unroll
        for (int dd = 0; dd < PDH_EW_MAX_DIMS; ++dd)
          if (dd == ia) c = c0[dd] + static_cast<int>(p.start[dd]);
        const int inc = ia == last ? 1 : 0;
#pragma unroll
        for (int e = 0; e < EPT; ++e) r[e][d] = static_cast<float>(c + e * inc);
        break;
      }
      case PDH_EW_NEG: un([](float x) { return -x; }); break;
      case PDH_EW_EXP: un([](float x) { return expf(x); }); break;
      case PDH_EW_LOG: un([](float x) { return logf(x); }); break;
      case PDH_EW_SQRT: un([](float x) { return sqrtf(x); }); break;
      case PDH_EW_TANH: un([](float x) { return tanhf(x); }); break;
      case PDH_EW_SIN: un([](float x) { return sinf(x); }); break;
      case PDH_EW_COS: un([](float x) { return cosf(x); }); break;
      case PDH_EW_ABS: un([](float x) { return fabsf(x); }); break;
      case PDH_EW_FLOOR: un([](float x) { return floorf(x); }); break;
      case PDH_EW_ADD: bin([](float x, float y) { return x + y; }); break;
      case PDH_EW_SUB: bin([](float x, float y) { return x - y; }); break;
      case PDH_EW_MUL: bin([](float x, float y) { return x * y; }); break;
      case PDH_EW_DIV: bin([](float x, float y) { return x / y; }); break;
      case PDH_EW_MAX: bin([](float x, float y) { return fmaxf(x, y); }); break;
      case PDH_EW_MIN: bin([](float x, float y) { return fminf(x, y); }); break;
      case PDH_EW_EQ: bin([](float x, float y) { return x == y ? 1.f : 0.f; }); break;
      case PDH_EW_NE: bin([](float x, float y) { return x != y ? 1.f : 0.f; }); break;
      case PDH_EW_LT: bin([](float x, float y) { return x < y ? 1.f : 0.f; }); break;
      case PDH_EW_LE: bin([](float x, float y) { return x <= y ? 1.f : 0.f; }); break;
      case PDH_EW_GT: bin([](float x, float y) { return x > y ? 1.f : 0.f; }); break;
      case PDH_EW_GE: bin([](float x, float y) { return x >= y ? 1.f : 0.f; }); break;
      default:  // PDH_EW_WHERE
#pragma unroll
        for (int e = 0; e < EPT; ++e) r[e][d] = r[e][ia] != 0.f ? r[e][ib] : r[e][ic];
        break;
    }
  }
  const int o = __builtin_amdgcn_readfirstlane(p.out_reg);
#pragma unroll
  for (int e = 0; e < EPT; ++e) res[e] = r[e][o];
}

}  // namespace pdh
