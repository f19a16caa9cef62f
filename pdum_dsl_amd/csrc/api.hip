// Library-wide C ABI: version, thread-local error text, device facts, and the
// MFMA lane-layout probe the attention kernels' operand layouts are tested by.
#include "common.h"

#include <cstring>

namespace pdh {

namespace {
thread_local std::string g_err;
}

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
}

const std::string& last_error() { return g_err; }

namespace {

// v_mfma_f32_32x32x16_bf16: A is 32(m) x 16(k), B is 16(k) x 32(n).
// Lane l holds A[l % 32][8 (l / 32) + j] and B[8 (l / 32) + j][l % 32], j = 0..7,
// and receives D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32], i = 0..15.
__global__ void probe32(const uint16_t* a, const uint16_t* b, float* c) {
  const int l = threadIdx.x;
  const int r = l & 31, g = l >> 5;
  bf16x8 av, bv;
  for (int j = 0; j < 8; ++j) {
    av[j] = __builtin_bit_cast(__bf16, a[r * 16 + g * 8 + j]);
    bv[j] = __builtin_bit_cast(__bf16, b[(g * 8 + j) * 32 + r]);
  }
  f32x16 acc = {};
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
  for (int i = 0; i < 16; ++i) c[((i >> 2) * 8 + g * 4 + (i & 3)) * 32 + r] = acc[i];
}

// v_mfma_f32_16x16x32_bf16: A is 16(m) x 32(k), B is 32(k) x 16(n).
// Lane l holds A[l % 16][8 (l / 16) + j] and B[8 (l / 16) + j][l % 16],
// and receives D[4 (l / 16) + i][l % 16], i = 0..3.
__global__ void probe16(const uint16_t* a, const uint16_t* b, float* c) {
  const int l = threadIdx.x;
  const int r = l & 15, g = l >> 4;
  bf16x8 av, bv;
  for (int j = 0; j < 8; ++j) {
    av[j] = __builtin_bit_cast(__bf16, a[r * 32 + g * 8 + j]);
    bv[j] = __builtin_bit_cast(__bf16, b[(g * 8 + j) * 16 + r]);
  }
  f32x4 acc = {};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc, 0, 0, 0);
  for (int i = 0; i < 4; ++i) c[(g * 4 + i) * 16 + r] = acc[i];
}

}  // namespace
}  // namespace pdh

using namespace pdh;

extern "C" int pdh_version(void) { return 100; }

extern "C" size_t pdh_last_error(char* buf, size_t n) {
  const std::string& e = last_error();
  if (buf && n) {
    const size_t k = e.size() < n - 1 ? e.size() : n - 1;
    std::memcpy(buf, e.data(), k);
    buf[k] = '\0';
  }
  return e.size();
}

extern "C" int pdh_device_cus(void) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  return cus;
}

extern "C" int pdh_probe_mfma(const uint16_t* a32, const uint16_t* b32, float* c32, const uint16_t* a16,
                              const uint16_t* b16, float* c16, void* stream) {
  PDH_REQUIRE(a32 && b32 && c32 && a16 && b16 && c16, PDH_EINVAL, "pdh_probe_mfma: null pointer");
  hipStream_t s = as_stream(stream);
  probe32<<<1, 64, 0, s>>>(a32, b32, c32);
  probe16<<<1, 64, 0, s>>>(a16, b16, c16);
  return check_launch("pdh_probe_mfma");
}
