// Device helpers shared by the attention kernels (forward, backward).
#pragma once

#include "common.h"

namespace pdh {

// Row permutation of a 32-row block in LDS. A 32x32x16 MFMA whose A operand
// lane l reads LDS row (l % 32) returns accumulator i of lane-half g = l / 32
// for A-row 8(i/4) + 4g + i%4. Storing logical row r at LDS row kperm_inv(r)
// makes accumulator i hold logical row 16(i/8) + 8g + (i%8): two runs of 8
// consecutive rows per lane-half, which is exactly the k-operand layout of the
// next MFMA (8 consecutive k per lane-half) — so a score tile's accumulators
// feed the second contraction without any register shuffle.
__device__ __forceinline__ int kperm_inv(int r) {
  const int c = r >> 4, g = (r >> 3) & 1, b = (r >> 2) & 1, j = r & 3;
  return 8 * (2 * c + b) + 4 * g + j;
}

// Logical row held by accumulator i of lane-half g (after the permutation).
__device__ __forceinline__ int acc_row(int i, int g) { return (i >> 3) * 16 + g * 8 + (i & 7); }

template <typename T>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);

template <>
__device__ __forceinline__ f32x16 mfma32<__hip_bfloat16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

template <>
__device__ __forceinline__ f32x16 mfma32<_Float16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}

// Pack accumulators [8h, 8h+8) of a 32x32 tile into one 16-bit k-operand.
template <typename T>
__device__ __forceinline__ u32x4 pack8(const f32x16& a, int h) {
  return u32x4{pack2<T>(a[8 * h + 0], a[8 * h + 1]), pack2<T>(a[8 * h + 2], a[8 * h + 3]),
               pack2<T>(a[8 * h + 4], a[8 * h + 5]), pack2<T>(a[8 * h + 6], a[8 * h + 7])};
}

// Combine the lo (sel 0x05040100) or hi (0x07060302) 16-bit halves of two dwords.
__device__ __forceinline__ uint32_t perm_halves(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

}  // namespace pdh
