// Inclusive prefix reduce along one dim: the reference's tl.scan
// (packages/tensorlib/src/pdum/tl/compute.py:318-350: ufunc accumulate; a mean
// divides by the running count). The reference leaves a scan in a red group
// its evaluator serves (the first-occurrence max / min adjoint,
// autodiff.py:635-665, puts one in every joint through a max); the carved-plan
// executor runs it here.
//
// Layout: dense [outer][n][inner], fp32 / bf16 / f16 storage, fp32 arithmetic.
//   inner == 1: one wave per row, 64 elements a step: a wave-wide inclusive
//               scan by shuffles (Hillis-Steele), plus the carry of the
//               previous steps; loads and stores cover 64 consecutive
//               elements (reversed order walks the row from its end);
//   inner > 1:  one thread per (outer, inner) column walking n in order;
//               consecutive threads touch consecutive inner (coalesced).
// Max / min propagate NaN as numpy's accumulate does. y may equal x: every
// element is read before it is written, by the thread that writes it.
#include "common.h"

namespace pdh {
namespace {

template <int F>
__device__ __forceinline__ float scan_op(float a, float b) {
  if constexpr (F == PDH_SCAN_MAX)
    return nan_max(a, b);
  else if constexpr (F == PDH_SCAN_MIN)
    return nan_min(a, b);
  else if constexpr (F == PDH_SCAN_PROD)
    return a * b;
  else
    return a + b;  // sum and mean
}

template <int F>
__device__ __forceinline__ float scan_identity() {
  if constexpr (F == PDH_SCAN_MAX)
    return -__builtin_inff();
  else if constexpr (F == PDH_SCAN_MIN)
    return __builtin_inff();
  else if constexpr (F == PDH_SCAN_PROD)
    return 1.0f;
  else
    return 0.0f;
}

template <int DT>
__device__ __forceinline__ float scan_ld(const void* base, int64_t i) {
  if constexpr (DT == PDH_F32)
    return static_cast<const float*>(base)[i];
  else if constexpr (DT == PDH_BF16)
    return bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
  else
    return f16_to_f32(static_cast<const uint16_t*>(base)[i]);
}

template <int DT, int F>
__global__ __launch_bounds__(256) void scan_rows(const void* x, void* y, int64_t rows, int64_t n, int rev) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t base = row * n;
  float carry = scan_identity<F>();
  for (int64_t c0 = 0; c0 < n; c0 += 64) {
    const int64_t p = c0 + lane;  // position in scan order
    const int64_t idx = rev ? n - 1 - p : p;
    float v = p < n ? scan_ld<DT>(x, base + idx) : scan_identity<F>();
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float u = __shfl_up(v, off, 64);
      if (lane >= off) v = scan_op<F>(u, v);
    }
    v = scan_op<F>(carry, v);
    if (p < n) st_dt<DT>(y, base + idx, F == PDH_SCAN_MEAN ? v / static_cast<float>(p + 1) : v);
    carry = __shfl(v, 63, 64);
  }
}

template <int DT, int F>
__global__ __launch_bounds__(256) void scan_cols(const void* x, void* y, int64_t outer, int64_t n, int64_t inner,
                                                 int rev) {
  const int64_t col = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (col >= outer * inner) return;
  const int64_t o = col / inner, i = col % inner;
  const int64_t base = o * n * inner + i;
  float acc = scan_identity<F>();
  for (int64_t p = 0; p < n; ++p) {
    const int64_t at = base + (rev ? n - 1 - p : p) * inner;
    acc = scan_op<F>(acc, scan_ld<DT>(x, at));
    st_dt<DT>(y, at, F == PDH_SCAN_MEAN ? acc / static_cast<float>(p + 1) : acc);
  }
}

template <int DT, int F>
int launch_scan(const void* x, void* y, int64_t outer, int64_t n, int64_t inner, int rev, hipStream_t st) {
  if (inner == 1) {
    const int64_t blocks = (outer + 3) / 4;
    PDH_REQUIRE(blocks <= INT32_MAX, PDH_EINVAL, "pdh_scan: too many rows (%lld)", (long long)outer);
    scan_rows<DT, F><<<dim3(static_cast<unsigned>(blocks)), 256, 0, st>>>(x, y, outer, n, rev);
  } else {
    const int64_t blocks = (outer * inner + 255) / 256;
    PDH_REQUIRE(blocks <= INT32_MAX, PDH_EINVAL, "pdh_scan: too many columns (%lld)", (long long)(outer * inner));
    scan_cols<DT, F><<<dim3(static_cast<unsigned>(blocks)), 256, 0, st>>>(x, y, outer, n, inner, rev);
  }
  return check_launch("pdh_scan");
}

template <int DT>
int scan_dispatch(const void* x, void* y, int64_t outer, int64_t n, int64_t inner, int reducer, int rev,
                  hipStream_t st) {
  switch (reducer) {
    case PDH_SCAN_SUM: return launch_scan<DT, PDH_SCAN_SUM>(x, y, outer, n, inner, rev, st);
    case PDH_SCAN_MAX: return launch_scan<DT, PDH_SCAN_MAX>(x, y, outer, n, inner, rev, st);
    case PDH_SCAN_MIN: return launch_scan<DT, PDH_SCAN_MIN>(x, y, outer, n, inner, rev, st);
    case PDH_SCAN_PROD: return launch_scan<DT, PDH_SCAN_PROD>(x, y, outer, n, inner, rev, st);
    default: return launch_scan<DT, PDH_SCAN_MEAN>(x, y, outer, n, inner, rev, st);
  }
}

}  // namespace
}  // namespace pdh

using namespace pdh;

extern "C" int pdh_scan(const void* x, void* y, int64_t outer, int64_t n, int64_t inner, int dtype, int reducer,
                        int reverse, void* stream) {
  PDH_REQUIRE(outer >= 0 && n >= 0 && inner >= 1, PDH_EINVAL,
              "pdh_scan: bad shape (outer %lld, n %lld, inner %lld)", (long long)outer, (long long)n,
              (long long)inner);
  PDH_REQUIRE(reducer >= PDH_SCAN_SUM && reducer <= PDH_SCAN_MEAN, PDH_EINVAL,
              "pdh_scan: reducer %d (0 sum, 1 max, 2 min, 3 prod, 4 mean)", reducer);
  PDH_REQUIRE(dtype == PDH_F32 || dtype == PDH_BF16 || dtype == PDH_F16, PDH_EINVAL, "pdh_scan: unknown dtype %d",
              dtype);
  if (outer == 0 || n == 0) return PDH_OK;
  PDH_REQUIRE(x != nullptr && y != nullptr, PDH_EINVAL, "pdh_scan: null pointer");
  PDH_REQUIRE(outer <= INT64_MAX / n / inner, PDH_EINVAL, "pdh_scan: element count overflows");
  hipStream_t st = as_stream(stream);
  const int rev = reverse ? 1 : 0;
  if (dtype == PDH_F32) return scan_dispatch<PDH_F32>(x, y, outer, n, inner, reducer, rev, st);
  if (dtype == PDH_BF16) return scan_dispatch<PDH_BF16>(x, y, outer, n, inner, reducer, rev, st);
  return scan_dispatch<PDH_F16>(x, y, outer, n, inner, reducer, rev, st);
}
