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

__device__ __forceinline__ float ew_load(const void* base, int64_t off, int dtype) {
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

// Runs program p for EPT elements whose output coordinates are coord[e][d]
// (d < p.ndim); acc[e] is what PDH_EW_ACC reads. Returns r[out_reg] in res.
template <int EPT>
__device__ __forceinline__ void ew_run(const pdh_ew_program& p, const EwOperands& ops, int dtype,
                                       const int (&coord)[EPT][PDH_EW_MAX_DIMS], const float (&acc)[EPT],
                                       float (&res)[EPT]) {
  f32x16 r[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) r[e] = f32x16{};
  const int n = __builtin_amdgcn_readfirstlane(p.n_insns);
  const int ndim = __builtin_amdgcn_readfirstlane(p.ndim);
  for (int pc = 0; pc < n; ++pc) {
    const pdh_ew_insn in = p.insns[pc];
    const int op = __builtin_amdgcn_readfirstlane(in.op);
    const int d = __builtin_amdgcn_readfirstlane(in.dst);
    const int ia = __builtin_amdgcn_readfirstlane(in.a);
    const int ib = __builtin_amdgcn_readfirstlane(in.b);
    const int ic = __builtin_amdgcn_readfirstlane(in.c);
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const float x = r[e][ia], y = r[e][ib];
      float v;
      switch (op) {
        case PDH_EW_LOAD: {
          int64_t off = 0;
#pragma unroll
          for (int dd = 0; dd < PDH_EW_MAX_DIMS; ++dd)
            if (dd < ndim) off += static_cast<int64_t>(coord[e][dd]) * p.in_stride[ia][dd];
          v = ew_load(ops.p[ia], off, dtype);
          break;
        }
        case PDH_EW_ACC: v = acc[e]; break;
        case PDH_EW_CONST: v = in.imm; break;
        case PDH_EW_IOTA: {
          int64_t c = 0;
#pragma unroll
          for (int dd = 0; dd < PDH_EW_MAX_DIMS; ++dd)
            if (dd == ia) c = coord[e][dd] + p.start[dd];
          v = static_cast<float>(c);
          break;
        }
        case PDH_EW_NEG: v = -x; break;
        case PDH_EW_EXP: v = expf(x); break;
        case PDH_EW_LOG: v = logf(x); break;
        case PDH_EW_SQRT: v = sqrtf(x); break;
        case PDH_EW_TANH: v = tanhf(x); break;
        case PDH_EW_SIN: v = sinf(x); break;
        case PDH_EW_COS: v = cosf(x); break;
        case PDH_EW_ABS: v = fabsf(x); break;
        case PDH_EW_FLOOR: v = floorf(x); break;
        case PDH_EW_ADD: v = x + y; break;
        case PDH_EW_SUB: v = x - y; break;
        case PDH_EW_MUL: v = x * y; break;
        case PDH_EW_DIV: v = x / y; break;
        case PDH_EW_MAX: v = fmaxf(x, y); break;
        case PDH_EW_MIN: v = fminf(x, y); break;
        case PDH_EW_EQ: v = x == y ? 1.f : 0.f; break;
        case PDH_EW_NE: v = x != y ? 1.f : 0.f; break;
        case PDH_EW_LT: v = x < y ? 1.f : 0.f; break;
        case PDH_EW_LE: v = x <= y ? 1.f : 0.f; break;
        case PDH_EW_GT: v = x > y ? 1.f : 0.f; break;
        case PDH_EW_GE: v = x >= y ? 1.f : 0.f; break;
        default: v = x != 0.f ? y : r[e][ic]; break;  // PDH_EW_WHERE
      }
      r[e][d] = v;
    }
  }
  const int o = __builtin_amdgcn_readfirstlane(p.out_reg);
#pragma unroll
  for (int e = 0; e < EPT; ++e) res[e] = r[e][o];
}

}  // namespace pdh
