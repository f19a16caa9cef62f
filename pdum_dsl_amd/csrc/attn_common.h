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


// ------------------------------------------------ LDS staging for key tiles
//
// Key/value tiles are copied HBM -> LDS by direct buffer loads (no VGPR round
// trip): one buffer_load_dwordx4 ... lds writes 16 bytes per lane to
// M0 + 16 * lane, i.e. 1 KB contiguous per wave. Rows are D * 2 bytes with no
// padding; instead, the 16-byte slot that holds chunk c of row r is
// c ^ swz(r), chosen so that the operand reads below hit distinct banks.

__device__ __forceinline__ int swap_bits23(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

// Tiles read BOTH as rows (b128 A operands, lane row swap_bits23(l % 32)) and
// transposed (ds_read_b64_tr_b16) — the backward's Q / dO / K tiles — use one
// table per row % 16, found by exhaustive check to keep both read patterns
// conflict-free for 32- and 64-bank LDS (the conditions are pinned by
// tests/test_lds_layout.py): entry i is the XOR mask of row i's 16-byte slots.
template <int D>
__device__ __forceinline__ int swz_rt(int row) {
  constexpr uint64_t kTable = D == 128 ? 0x0c7a42f8e9356d1bull : 0x1265314603742057ull;
  return static_cast<int>((kTable >> (4 * (row & 15))) & 15u);
}

typedef __attribute__((address_space(3))) void lds_void_t;

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
