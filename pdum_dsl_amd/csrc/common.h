// Shared device/host helpers for libpdhip (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/pdhip.h"
#include "dev.h"

namespace pdh {

// ---------------------------------------------------------------- host errors

void set_error(const char* fmt, ...);
const std::string& last_error();

#define PDH_REQUIRE(cond, code, ...)      \
  do {                                    \
    if (!(cond)) {                        \
      ::pdh::set_error(__VA_ARGS__);      \
      return (code);                      \
    }                                     \
  } while (0)

// Launch check: a launch error is reported, never swallowed.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return PDH_ELAUNCH;
  }
  return PDH_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------------- device helpers

constexpr int kWave = 64;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Global load / store at a wave-uniform base plus a 32-bit per-lane byte
// offset: the backend emits the saddr form (global_load vOFF, s[BASE]), so the
// 64-bit address arithmetic stays on the scalar unit and each lane carries one
// 32-bit offset instead of a 64-bit pointer.
template <typename V>
__device__ __forceinline__ V gload(const void* base, uint32_t off) {
  return *reinterpret_cast<const V*>(reinterpret_cast<const char*>(base) + off);
}
template <typename V>
__device__ __forceinline__ void gstore(void* base, uint32_t off, V v) {
  *reinterpret_cast<V*>(reinterpret_cast<char*>(base) + off) = v;
}

// Raw buffer loads (make_rsrc: dev.h): a 32-bit per-lane VGPR offset and a
// 32-bit scalar offset. Reads past the resource's end return 0 (the hardware
// range check), which zero-pads tail tiles for free, and the address stays
// one long-lived VGPR instead of a 64-bit pair per load.
__device__ __forceinline__ u32x4 bload128(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ u32x2 bload64(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
}
__device__ __forceinline__ uint32_t bload32(rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

// exp2 of an fp32 argument on the hardware transcendental unit (v_exp_f32).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---- 16-bit element conversions (round to nearest even) ----

template <typename T>
struct Elem;

template <>
struct Elem<__hip_bfloat16> {
  __device__ __forceinline__ static float to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
  }
  __device__ __forceinline__ static uint16_t from_f32(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);  // NaN stays NaN
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
  }
};

template <>
struct Elem<_Float16> {
  __device__ __forceinline__ static float to_f32(uint16_t b) {
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return static_cast<float>(h);
  }
  __device__ __forceinline__ static uint16_t from_f32(float f) {
    _Float16 h = static_cast<_Float16>(f);
    uint16_t b;
    __builtin_memcpy(&b, &h, 2);
    return b;
  }
};

// Pack two fp32 into one dword of two 16-bit elements (lo = a, hi = b), round
// to nearest even (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 on gfx950).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ uint32_t pack2(float a, float b);

template <>
__device__ __forceinline__ uint32_t pack2<__hip_bfloat16>(float a, float b) {
  f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

template <>
__device__ __forceinline__ uint32_t pack2<_Float16>(float a, float b) {
  f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

// Unpack the lo / hi 16-bit element of a dword to fp32.
template <typename T>
__device__ __forceinline__ float lo_f32(uint32_t w) {
  return Elem<T>::to_f32(static_cast<uint16_t>(w & 0xffffu));
}
template <typename T>
__device__ __forceinline__ float hi_f32(uint32_t w) {
  return Elem<T>::to_f32(static_cast<uint16_t>(w >> 16));
}

}  // namespace pdh
