// Device-only helpers with no host or library dependencies: the subset the
// map-chain and contraction kernels are built from. The same text compiles
// in the library build (hipcc) and in the runtime-specialized kernels
// (hipRTC, which has no HIP host headers: element types are plain 16-bit
// words here, converted by the functions below).
#pragma once

#if defined(__HIPCC_RTC__)
#include "pdhip.h"
#else
#include "../../include/pdhip.h"
#endif

namespace pdh {

typedef float f32x4 __attribute__((ext_vector_type(4)));
// four floats at any 4-byte boundary: one global_load_dwordx4 / store (the
// hardware takes dword-aligned multi-dword accesses)
typedef float f32x4u __attribute__((ext_vector_type(4), aligned(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Wave index as a scalar (uniform) value.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Sum over the 64 lanes of a wave (butterfly of cross-lane moves); every lane
// gets the total.
__device__ __forceinline__ float wave_total(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---- 16-bit element conversions (round to nearest even; NaN stays NaN) ----

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// round to nearest even by the hardware conversion (v_cvt_pk_bf16_f32, one
// instruction); NaN stays NaN
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ float f16_to_f32(uint16_t b) { return static_cast<float>(__builtin_bit_cast(_Float16, b)); }

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// tanh from the identity tanh|x| = 1 - 2 / (exp(2|x|) + 1), with the
// hardware exp2 (v_exp_f32) and reciprocal (v_rcp_f32): about six
// instructions, absolute error ~2e-7 over the whole line (exp overflow to
// inf gives exactly 1; near 0 the result is |x| to within an ulp of 1), odd
// by construction. NaN stays NaN.
__device__ __forceinline__ float pdh_tanh(float x) {
  const float ax = __builtin_fabsf(x);
  const float e = __builtin_amdgcn_exp2f(ax * 2.8853900817779268f);  // exp(2|x|) = 2^(2|x| log2 e)
  const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
  return __builtin_copysignf(t, x);
}

// max / min that propagate NaN, as numpy's maximum / minimum and its max / min
// reductions do (fmaxf / fminf return the non-NaN operand instead).
__device__ __forceinline__ float nan_max(float x, float y) {
  return (x != x || y != y) ? x + y : __builtin_fmaxf(x, y);
}
__device__ __forceinline__ float nan_min(float x, float y) {
  return (x != x || y != y) ? x + y : __builtin_fminf(x, y);
}

// One element of a PDH_F32 / PDH_BF16 / PDH_F16 buffer as fp32, and back.
template <int DT>
__device__ __forceinline__ float ld_dt(const void* base, int off) {
  if constexpr (DT == PDH_F32)
    return static_cast<const float*>(base)[off];
  else if constexpr (DT == PDH_BF16)
    return bf16_to_f32(static_cast<const uint16_t*>(base)[off]);
  else
    return f16_to_f32(static_cast<const uint16_t*>(base)[off]);
}

template <int DT>
__device__ __forceinline__ void st_dt(void* base, long long off, float v) {
  if constexpr (DT == PDH_F32)
    static_cast<float*>(base)[off] = v;
  else if constexpr (DT == PDH_BF16)
    static_cast<uint16_t*>(base)[off] = f32_to_bf16(v);
  else
    static_cast<uint16_t*>(base)[off] = f32_to_f16(v);
}

// ---- MFMA: v_mfma_f32_32x32x16 on bf16 / f16 operands (8 per lane) ----
template <int DT>
__device__ __forceinline__ f32x16 mfma32_dt(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == PDH_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                   0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
}

// ---- buffer resources and direct HBM -> LDS loads ----

// A scalar V# resource over [base, base + bytes): reads past `bytes` return 0.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kBufferWord3 = 0x00020000;  // gfx9-family dword3: 32-bit data format, untyped access

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(bytes),
                                           kBufferWord3);
}

// 16 bytes per lane, buffer -> LDS (lane i's bytes land at lds + 16 i; lds is
// wave-uniform). Inline asm keeps the compiler's wait-count pass from making
// every later LDS read wait for it: callers wait with s_waitcnt vmcnt(0) and a
// barrier before reading the tile.
__device__ __forceinline__ void dma16(rsrc_t r, unsigned char* lds, uint32_t voff, uint32_t soff) {
  // the low 32 bits of a generic LDS address are its LDS offset (no address-space cast needed)
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds)));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved: listed so the compiler knows it changes
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(m0), "v"(voff), "s"(r), "s"(soff)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// s_waitcnt vmcnt(0) (expcnt / lgkmcnt left at their maxima), issued through
// the builtin so the compiler's own wait-count tracking sees it and adds no
// later vector-memory waits of its own.
__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0f70); }

}  // namespace pdh
