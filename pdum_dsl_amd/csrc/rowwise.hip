// Row-reduction tile columns: fused row softmax ("row-normalization",
// fusion.py:371-400) and two-pass layernorm ("row-statistics",
// fusion.py:403-443; zoo/zoo_common.py:56-60). Both are HBM-bound: one read of
// x and one write of y per element.
//
// Fast path: one wave64 per row, the whole row resident in registers as
// float4 (NV float4 per lane, row length <= 256*NV), 128-bit coalesced loads
// (lane l of a wave reads bytes [16 l, 16 l + 16) of each 1 KiB segment), the
// reductions in registers + cross-lane shuffles — no LDS, no barriers.
// Four rows per 256-thread workgroup.
//
// Fallback: rows longer than 4096 or not 16-byte aligned stream through one
// workgroup per row in several passes (online max/sum for softmax).
#include "common.h"

namespace pdh {
namespace {

constexpr int kRowsPerBlock = 4;
constexpr float kNegInf = -__builtin_inff();

// Four consecutive elements of a PDH_F32 / PDH_BF16 / PDH_F16 row as fp32
// (one 16-byte or 8-byte load), and back; `i` counts groups of four.
template <int DT>
__device__ __forceinline__ f32x4 ld4(const void* row, int i) {
  if constexpr (DT == PDH_F32) {
    return __builtin_nontemporal_load(static_cast<const f32x4*>(row) + i);
  } else {
    const u32x2 w = __builtin_nontemporal_load(static_cast<const u32x2*>(row) + i);
    if constexpr (DT == PDH_BF16)
      return f32x4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
                   __uint_as_float(w.y & 0xffff0000u)};
    else
      return f32x4{f16_to_f32(static_cast<uint16_t>(w.x)), f16_to_f32(static_cast<uint16_t>(w.x >> 16)),
                   f16_to_f32(static_cast<uint16_t>(w.y)), f16_to_f32(static_cast<uint16_t>(w.y >> 16))};
  }
}

// The same four elements through the caches: gamma and beta are read by
// every row, so they must stay resident (a nontemporal load would stream them
// from HBM again for each row).
template <int DT>
__device__ __forceinline__ f32x4 ld4_cached(const void* row, int i) {
  if constexpr (DT == PDH_F32) {
    return static_cast<const f32x4*>(row)[i];
  } else {
    const u32x2 w = static_cast<const u32x2*>(row)[i];
    if constexpr (DT == PDH_BF16)
      return f32x4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
                   __uint_as_float(w.y & 0xffff0000u)};
    else
      return f32x4{f16_to_f32(static_cast<uint16_t>(w.x)), f16_to_f32(static_cast<uint16_t>(w.x >> 16)),
                   f16_to_f32(static_cast<uint16_t>(w.y)), f16_to_f32(static_cast<uint16_t>(w.y >> 16))};
  }
}

template <int DT>
__device__ __forceinline__ void st4(void* row, int i, f32x4 v) {
  if constexpr (DT == PDH_F32) {
    __builtin_nontemporal_store(v, static_cast<f32x4*>(row) + i);
  } else {
    uint16_t e[4];
    e[0] = DT == PDH_BF16 ? f32_to_bf16(v.x) : f32_to_f16(v.x);
    e[1] = DT == PDH_BF16 ? f32_to_bf16(v.y) : f32_to_f16(v.y);
    e[2] = DT == PDH_BF16 ? f32_to_bf16(v.z) : f32_to_f16(v.z);
    e[3] = DT == PDH_BF16 ? f32_to_bf16(v.w) : f32_to_f16(v.w);
    const u32x2 w{static_cast<uint32_t>(e[0]) | (static_cast<uint32_t>(e[1]) << 16),
                  static_cast<uint32_t>(e[2]) | (static_cast<uint32_t>(e[3]) << 16)};
    __builtin_nontemporal_store(w, static_cast<u32x2*>(row) + i);
  }
}

template <int DT>
constexpr int64_t esize() {
  return DT == PDH_F32 ? 4 : 2;
}

template <int DT>
__device__ __forceinline__ const void* row_at(const void* base, int64_t row, int64_t ld) {
  return static_cast<const unsigned char*>(base) + row * ld * esize<DT>();
}

template <int DT>
__device__ __forceinline__ void* row_at(void* base, int64_t row, int64_t ld) {
  return static_cast<unsigned char*>(base) + row * ld * esize<DT>();
}

template <int DT, int NV>
__global__ __launch_bounds__(256) void softmax_rows_v4(const void* __restrict__ x, void* __restrict__ y,
                                                       int64_t rows, int cols, int64_t ldx, int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const void* xr = row_at<DT>(x, row, ldx);
  void* yr = row_at<DT>(y, row, ldy);
  const int nvec = cols >> 2;
  f32x4 v[NV];
  float mx = kNegInf;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int idx = j * 64 + lane;
    if (idx < nvec) {
      v[j] = ld4<DT>(xr, idx);
    } else {
      v[j] = f32x4{kNegInf, kNegInf, kNegInf, kNegInf};
    }
    mx = fmaxf(mx, fmaxf(fmaxf(v[j].x, v[j].y), fmaxf(v[j].z, v[j].w)));
  }
  mx = wave_max(mx);
  const float mxl = mx * kLog2e;
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    // exp(x - m) = exp2(x*log2e - m*log2e); lanes past the row end hold -inf -> 0.
    v[j].x = fast_exp2(__builtin_fmaf(v[j].x, kLog2e, -mxl));
    v[j].y = fast_exp2(__builtin_fmaf(v[j].y, kLog2e, -mxl));
    v[j].z = fast_exp2(__builtin_fmaf(v[j].z, kLog2e, -mxl));
    v[j].w = fast_exp2(__builtin_fmaf(v[j].w, kLog2e, -mxl));
    sum += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  }
  sum = wave_sum(sum);
  const float inv = 1.0f / sum;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int idx = j * 64 + lane;
    if (idx < nvec) st4<DT>(yr, idx, v[j] * inv);
  }
}

// RPW rows per wave: the affine epilogue reads each gamma / beta chunk once for
// all of them (those reads come from L2 and, one row per wave, add as many L2
// bytes again as the row itself). Two rows per wave for rows of 2048+ columns:
// +5.6% on [8192, 4096] fp32 (5.43 -> 5.73 TB/s, same process), at 172 VGPRs.
template <int DT, int NV, bool AFFINE, int RPW = 1>
__global__ __launch_bounds__(256) void layernorm_rows_v4(const void* __restrict__ x, const void* __restrict__ gamma,
                                                         const void* __restrict__ beta, void* __restrict__ y,
                                                         int64_t rows, int cols, int64_t ldx, int64_t ldy,
                                                         float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6)) * RPW;
  if (row0 >= rows) return;
  const int nvec = cols >> 2;
  const float inv_n = 1.0f / static_cast<float>(cols);
  f32x4 v[RPW][NV];
  float mu[RPW], rstd[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const bool live = row0 + r < rows;
    const void* xr = row_at<DT>(x, live ? row0 + r : row0, ldx);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int idx = j * 64 + lane;
      v[r][j] = idx < nvec ? ld4<DT>(xr, idx) : f32x4{0.f, 0.f, 0.f, 0.f};
      s += (v[r][j].x + v[r][j].y) + (v[r][j].z + v[r][j].w);
    }
    mu[r] = wave_sum(s) * inv_n;
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int idx = j * 64 + lane;
      if (idx < nvec) {
        v[r][j] -= mu[r];
        ss += (v[r][j].x * v[r][j].x + v[r][j].y * v[r][j].y) + (v[r][j].z * v[r][j].z + v[r][j].w * v[r][j].w);
      }
    }
    const float var = wave_sum(ss) * inv_n;
    rstd[r] = 1.0f / sqrtf(var + eps);
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int idx = j * 64 + lane;
    if (idx < nvec) {
      f32x4 gm = f32x4{1.f, 1.f, 1.f, 1.f}, bt = f32x4{0.f, 0.f, 0.f, 0.f};
      if (AFFINE) {
        if (gamma) gm = ld4_cached<DT>(gamma, idx);
        if (beta) bt = ld4_cached<DT>(beta, idx);
      }
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        if (row0 + r < rows) {
          f32x4 o = v[r][j] * rstd[r];
          if (AFFINE) o = o * gm + bt;
          st4<DT>(row_at<DT>(y, row0 + r, ldy), idx, o);
        }
      }
    }
  }
}

// ---- streaming fallbacks (any length, any alignment): one workgroup per row ----

__device__ float block_reduce_max(float v, float* sh) {
  v = wave_max(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) sh[w] = v;
  __syncthreads();
  float r = sh[0];
  for (int i = 1; i < static_cast<int>(blockDim.x >> 6); ++i) r = fmaxf(r, sh[i]);
  return r;
}

__device__ float block_reduce_sum(float v, float* sh) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) sh[w] = v;
  __syncthreads();
  float r = 0.f;
  for (int i = 0; i < static_cast<int>(blockDim.x >> 6); ++i) r += sh[i];
  return r;
}

template <int DT>
__global__ __launch_bounds__(256) void softmax_rows_stream(const void* __restrict__ x, void* __restrict__ y,
                                                           int64_t cols, int64_t ldx, int64_t ldy) {
  __shared__ float sh[8];
  const int64_t row = blockIdx.x;
  const void* xr = row_at<DT>(x, row, ldx);
  void* yr = row_at<DT>(y, row, ldy);
  // pass 1: online (max, sum) per thread, then the associative combine across the block
  float m = kNegInf, l = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    const float xv = ld_dt<DT>(xr, static_cast<int>(c));
    if (xv == kNegInf) continue;  // contributes exp(-inf) = 0
    if (xv > m) {
      l = l * fast_exp2((m - xv) * kLog2e) + 1.f;
      m = xv;
    } else {
      l += fast_exp2((xv - m) * kLog2e);
    }
  }
  const float gm = block_reduce_max(m, sh);
  const float scaled = (m == kNegInf) ? 0.f : l * fast_exp2((m - gm) * kLog2e);
  const float gl = block_reduce_sum(scaled, sh);
  const float inv = 1.0f / gl;
  const float gml = gm * kLog2e;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x)
    st_dt<DT>(yr, c, fast_exp2(__builtin_fmaf(ld_dt<DT>(xr, static_cast<int>(c)), kLog2e, -gml)) * inv);
}

template <int DT>
__global__ __launch_bounds__(256) void layernorm_rows_stream(const void* __restrict__ x,
                                                             const void* __restrict__ gamma,
                                                             const void* __restrict__ beta, void* __restrict__ y,
                                                             int64_t cols, int64_t ldx, int64_t ldy, float eps) {
  __shared__ float sh[8];
  const int64_t row = blockIdx.x;
  const void* xr = row_at<DT>(x, row, ldx);
  void* yr = row_at<DT>(y, row, ldy);
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) s += ld_dt<DT>(xr, static_cast<int>(c));
  const float mu = block_reduce_sum(s, sh) / static_cast<float>(cols);
  float ss = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    const float d = ld_dt<DT>(xr, static_cast<int>(c)) - mu;
    ss += d * d;
  }
  const float var = block_reduce_sum(ss, sh) / static_cast<float>(cols);
  const float rstd = 1.0f / sqrtf(var + eps);
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    const int ci = static_cast<int>(c);
    float o = (ld_dt<DT>(xr, ci) - mu) * rstd;
    if (gamma) o *= ld_dt<DT>(gamma, ci);
    if (beta) o += ld_dt<DT>(beta, ci);
    st_dt<DT>(yr, c, o);
  }
}

int pick_nv(int64_t cols) {
  const int64_t per = (cols + 255) / 256;  // float4 per lane
  if (per <= 1) return 1;
  if (per <= 2) return 2;
  if (per <= 4) return 4;
  if (per <= 8) return 8;
  if (per <= 16) return 16;
  return 0;
}

bool aligned_to(const void* p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// The register-resident path: rows of at most 4096 elements, a multiple of
// 4, with every row's start aligned to 4 elements.
bool fast_ok(const void* x, const void* y, int64_t cols, int64_t ldx, int64_t ldy, const void* g, const void* b,
             int dtype) {
  const int64_t al = dtype == PDH_F32 ? 16 : 8;
  return (cols % 4 == 0) && (ldx % 4 == 0) && (ldy % 4 == 0) && aligned_to(x, al) && aligned_to(y, al) &&
         (g == nullptr || aligned_to(g, al)) && (b == nullptr || aligned_to(b, al)) && pick_nv(cols) != 0 &&
         cols <= INT32_MAX;
}

template <int DT>
void launch_softmax(const void* x, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, hipStream_t s) {
  if (fast_ok(x, y, cols, ldx, ldy, nullptr, nullptr, DT)) {
    const dim3 grid(static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const int c = static_cast<int>(cols);
    switch (pick_nv(cols)) {
      case 1: softmax_rows_v4<DT, 1><<<grid, 256, 0, s>>>(x, y, rows, c, ldx, ldy); break;
      case 2: softmax_rows_v4<DT, 2><<<grid, 256, 0, s>>>(x, y, rows, c, ldx, ldy); break;
      case 4: softmax_rows_v4<DT, 4><<<grid, 256, 0, s>>>(x, y, rows, c, ldx, ldy); break;
      case 8: softmax_rows_v4<DT, 8><<<grid, 256, 0, s>>>(x, y, rows, c, ldx, ldy); break;
      default: softmax_rows_v4<DT, 16><<<grid, 256, 0, s>>>(x, y, rows, c, ldx, ldy); break;
    }
  } else {
    softmax_rows_stream<DT><<<dim3(static_cast<unsigned>(rows)), 256, 0, s>>>(x, y, cols, ldx, ldy);
  }
}

template <int DT>
void launch_layernorm(const void* x, const void* gamma, const void* beta, void* y, int64_t rows, int64_t cols,
                      int64_t ldx, int64_t ldy, float eps, hipStream_t s) {
  if (fast_ok(x, y, cols, ldx, ldy, gamma, beta, DT)) {
    const dim3 grid(static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const int c = static_cast<int>(cols);
    const bool aff = gamma || beta;
    // affine rows of 2048+ columns: two rows per wave share the gamma / beta reads
    const dim3 grid2(static_cast<unsigned>((rows + 2 * kRowsPerBlock - 1) / (2 * kRowsPerBlock)));
#define PDH_LN(NV)                                                                                          \
  do {                                                                                                      \
    if (aff && NV >= 8)                                                                        \
      layernorm_rows_v4<DT, NV, true, 2><<<grid2, 256, 0, s>>>(x, gamma, beta, y, rows, c, ldx, ldy, eps); \
    else if (aff)                                                                                           \
      layernorm_rows_v4<DT, NV, true><<<grid, 256, 0, s>>>(x, gamma, beta, y, rows, c, ldx, ldy, eps);     \
    else                                                                                                    \
      layernorm_rows_v4<DT, NV, false><<<grid, 256, 0, s>>>(x, gamma, beta, y, rows, c, ldx, ldy, eps);    \
  } while (0)
    switch (pick_nv(cols)) {
      case 1: PDH_LN(1); break;
      case 2: PDH_LN(2); break;
      case 4: PDH_LN(4); break;
      case 8: PDH_LN(8); break;
      default: PDH_LN(16); break;
    }
#undef PDH_LN
  } else {
    layernorm_rows_stream<DT>
        <<<dim3(static_cast<unsigned>(rows)), 256, 0, s>>>(x, gamma, beta, y, cols, ldx, ldy, eps);
  }
}

}  // namespace
}  // namespace pdh

using namespace pdh;

extern "C" int pdh_row_softmax_dt(const void* x, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy,
                                  int dtype, void* stream) {
  PDH_REQUIRE(dtype == PDH_F32 || dtype == PDH_BF16 || dtype == PDH_F16, PDH_EUNSUPPORTED,
              "pdh_row_softmax: dtype %d", dtype);
  PDH_REQUIRE(rows >= 0 && cols >= 1, PDH_EINVAL, "pdh_row_softmax: need rows >= 0 and cols >= 1 (got %lld, %lld)",
              (long long)rows, (long long)cols);
  PDH_REQUIRE(ldx >= cols && ldy >= cols, PDH_EINVAL,
              "pdh_row_softmax: row strides (%lld, %lld) must be >= cols (%lld)", (long long)ldx, (long long)ldy,
              (long long)cols);
  PDH_REQUIRE(rows == 0 || (x && y), PDH_EINVAL, "pdh_row_softmax: null pointer");
  PDH_REQUIRE(rows <= INT32_MAX, PDH_EINVAL, "pdh_row_softmax: too many rows");
  PDH_REQUIRE(cols <= INT32_MAX, PDH_EINVAL, "pdh_row_softmax: rows longer than 2^31 elements");
  if (rows == 0) return PDH_OK;
  hipStream_t s = as_stream(stream);
  if (dtype == PDH_F32)
    launch_softmax<PDH_F32>(x, y, rows, cols, ldx, ldy, s);
  else if (dtype == PDH_BF16)
    launch_softmax<PDH_BF16>(x, y, rows, cols, ldx, ldy, s);
  else
    launch_softmax<PDH_F16>(x, y, rows, cols, ldx, ldy, s);
  return check_launch("pdh_row_softmax");
}

extern "C" int pdh_row_softmax(const float* x, float* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy,
                               void* stream) {
  return pdh_row_softmax_dt(x, y, rows, cols, ldx, ldy, PDH_F32, stream);
}

extern "C" int pdh_layernorm_dt(const void* x, const void* gamma, const void* beta, void* y, int64_t rows,
                                int64_t cols, int64_t ldx, int64_t ldy, float eps, int dtype, void* stream) {
  PDH_REQUIRE(dtype == PDH_F32 || dtype == PDH_BF16 || dtype == PDH_F16, PDH_EUNSUPPORTED,
              "pdh_layernorm: dtype %d", dtype);
  PDH_REQUIRE(rows >= 0 && cols >= 1, PDH_EINVAL, "pdh_layernorm: need rows >= 0 and cols >= 1 (got %lld, %lld)",
              (long long)rows, (long long)cols);
  PDH_REQUIRE(ldx >= cols && ldy >= cols, PDH_EINVAL,
              "pdh_layernorm: row strides (%lld, %lld) must be >= cols (%lld)", (long long)ldx, (long long)ldy,
              (long long)cols);
  PDH_REQUIRE(rows == 0 || (x && y), PDH_EINVAL, "pdh_layernorm: null pointer");
  PDH_REQUIRE(eps >= 0.f, PDH_EINVAL, "pdh_layernorm: eps must be >= 0");
  PDH_REQUIRE(rows <= INT32_MAX, PDH_EINVAL, "pdh_layernorm: too many rows");
  PDH_REQUIRE(cols <= INT32_MAX, PDH_EINVAL, "pdh_layernorm: rows longer than 2^31 elements");
  if (rows == 0) return PDH_OK;
  hipStream_t s = as_stream(stream);
  if (dtype == PDH_F32)
    launch_layernorm<PDH_F32>(x, gamma, beta, y, rows, cols, ldx, ldy, eps, s);
  else if (dtype == PDH_BF16)
    launch_layernorm<PDH_BF16>(x, gamma, beta, y, rows, cols, ldx, ldy, eps, s);
  else
    launch_layernorm<PDH_F16>(x, gamma, beta, y, rows, cols, ldx, ldy, eps, s);
  return check_launch("pdh_layernorm");
}

extern "C" int pdh_layernorm(const float* x, const float* gamma, const float* beta, float* y, int64_t rows,
                             int64_t cols, int64_t ldx, int64_t ldy, float eps, void* stream) {
  return pdh_layernorm_dt(x, gamma, beta, y, rows, cols, ldx, ldy, eps, PDH_F32, stream);
}
