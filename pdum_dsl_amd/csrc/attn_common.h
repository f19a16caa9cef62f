// Device helpers shared by the attention kernels (forward, backward).
#pragma once

#include "common.h"

namespace pdh {

// v_mfma_f32_16x16x32: lane l holds A[l % 16][8 (l / 16) + j] and
// B[8 (l / 16) + j][l % 16], j = 0..7, and receives D[4 (l / 16) + i][l % 16].
template <typename T>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c);

template <>
__device__ __forceinline__ f32x4 mfma16<__hip_bfloat16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

template <>
__device__ __forceinline__ f32x4 mfma16<_Float16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}

// ------------------------------------------------ LDS staging for key tiles
//
// Key/value tiles are copied HBM -> LDS by direct buffer loads (no VGPR round
// trip): one buffer_load_dwordx4 ... lds writes 16 bytes per lane to
// M0 + 16 * lane, i.e. 1 KB contiguous per wave. Rows are D * 2 bytes with no
// padding; instead, the 16-byte slot that holds chunk c of row r is
// c ^ swz(r), each kernel choosing swz so that its operand reads hit
// distinct banks.

// (dma16 and wait_vmcnt0: dev.h)

// 4 bytes per lane, buffer -> LDS (lane i's dword lands at lds + 4 i).
__device__ __forceinline__ void dma4(rsrc_t r, unsigned char* lds, uint32_t voff, uint32_t soff) {
  // the low 32 bits of a generic LDS address are its LDS offset (no address-space cast needed)
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds" ::"s"(m0), "v"(voff), "s"(r), "s"(soff)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// ds_read_b64_tr_b16: in each 16-lane group, lane 4k + c supplies the address
// of 8 bytes (4 elements); lane i of the group receives element (i % 4) of the
// chunk addressed by lane 4k + i / 4, for k = 0..3. Pointing lane 4k + c at
// row k, features 4c..4c+3 of a row-major tile gives lane i the 4 rows' values
// of feature i: a transposed (k-contiguous) MFMA operand.
typedef short s16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 ds_read_tr16(const unsigned char* p) {
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

}  // namespace pdh
