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

template <int NV>
__global__ __launch_bounds__(256) void softmax_rows_v4(const float* __restrict__ x, float* __restrict__ y,
                                                       int64_t rows, int cols, int64_t ldx, int64_t ldy) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const f32x4* xr = reinterpret_cast<const f32x4*>(x + row * ldx);
  f32x4* yr = reinterpret_cast<f32x4*>(y + row * ldy);
  const int nvec = cols >> 2;
  f32x4 v[NV];
  float mx = kNegInf;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int idx = j * 64 + lane;
    if (idx < nvec) {
      v[j] = __builtin_nontemporal_load(xr + idx);
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
    if (idx < nvec) __builtin_nontemporal_store(v[j] * inv, yr + idx);
  }
}

template <int NV, bool AFFINE>
__global__ __launch_bounds__(256) void layernorm_rows_v4(const float* __restrict__ x,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta, float* __restrict__ y,
                                                         int64_t rows, int cols, int64_t ldx, int64_t ldy,
                                                         float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const f32x4* xr = reinterpret_cast<const f32x4*>(x + row * ldx);
  f32x4* yr = reinterpret_cast<f32x4*>(y + row * ldy);
  const int nvec = cols >> 2;
  f32x4 v[NV];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int idx = j * 64 + lane;
    v[j] = idx < nvec ? __builtin_nontemporal_load(xr + idx) : f32x4{0.f, 0.f, 0.f, 0.f};
    s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  }
  const float inv_n = 1.0f / static_cast<float>(cols);
  const float mu = wave_sum(s) * inv_n;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int idx = j * 64 + lane;
    if (idx < nvec) {
      v[j] -= mu;
      ss += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
    }
  }
  const float var = wave_sum(ss) * inv_n;
  const float rstd = 1.0f / sqrtf(var + eps);
  const f32x4* g4 = reinterpret_cast<const f32x4*>(gamma);
  const f32x4* b4 = reinterpret_cast<const f32x4*>(beta);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int idx = j * 64 + lane;
    if (idx < nvec) {
      f32x4 o = v[j] * rstd;
      if (AFFINE) {
        if (gamma) o *= g4[idx];
        if (beta) o += b4[idx];
      }
      __builtin_nontemporal_store(o, yr + idx);
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

__global__ __launch_bounds__(256) void softmax_rows_stream(const float* __restrict__ x, float* __restrict__ y,
                                                           int64_t cols, int64_t ldx, int64_t ldy) {
  __shared__ float sh[8];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * ldx;
  float* yr = y + row * ldy;
  // pass 1: online (max, sum) per thread, then the associative combine across the block
  float m = kNegInf, l = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    const float xv = xr[c];
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
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) yr[c] = fast_exp2(__builtin_fmaf(xr[c], kLog2e, -gml)) * inv;
}

__global__ __launch_bounds__(256) void layernorm_rows_stream(const float* __restrict__ x,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta, float* __restrict__ y,
                                                             int64_t cols, int64_t ldx, int64_t ldy, float eps) {
  __shared__ float sh[8];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * ldx;
  float* yr = y + row * ldy;
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) s += xr[c];
  const float mu = block_reduce_sum(s, sh) / static_cast<float>(cols);
  float ss = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    const float d = xr[c] - mu;
    ss += d * d;
  }
  const float var = block_reduce_sum(ss, sh) / static_cast<float>(cols);
  const float rstd = 1.0f / sqrtf(var + eps);
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    float o = (xr[c] - mu) * rstd;
    if (gamma) o *= gamma[c];
    if (beta) o += beta[c];
    yr[c] = o;
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

bool fast_ok(const float* x, const float* y, int64_t cols, int64_t ldx, int64_t ldy, const float* g,
             const float* b) {
  return (cols % 4 == 0) && (ldx % 4 == 0) && (ldy % 4 == 0) && aligned16(x) && aligned16(y) &&
         (g == nullptr || aligned16(g)) && (b == nullptr || aligned16(b)) && pick_nv(cols) != 0 &&
         cols <= INT32_MAX;
}

}  // namespace
}  // namespace pdh

using namespace pdh;

extern "C" int pdh_row_softmax(const float* x, float* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy,
                               void* stream) {
  PDH_REQUIRE(rows >= 0 && cols >= 1, PDH_EINVAL, "pdh_row_softmax: need rows >= 0 and cols >= 1 (got %lld, %lld)",
              (long long)rows, (long long)cols);
  PDH_REQUIRE(ldx >= cols && ldy >= cols, PDH_EINVAL,
              "pdh_row_softmax: row strides (%lld, %lld) must be >= cols (%lld)", (long long)ldx, (long long)ldy,
              (long long)cols);
  PDH_REQUIRE(rows == 0 || (x && y), PDH_EINVAL, "pdh_row_softmax: null pointer");
  PDH_REQUIRE(rows <= (int64_t)INT32_MAX * kRowsPerBlock, PDH_EINVAL, "pdh_row_softmax: too many rows");
  if (rows == 0) return PDH_OK;
  hipStream_t s = as_stream(stream);
  if (fast_ok(x, y, cols, ldx, ldy, nullptr, nullptr)) {
    const dim3 grid(static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const int c = static_cast<int>(cols);
    switch (pick_nv(cols)) {
      case 1: softmax_rows_v4<1><<<grid, 256, 0, s>>>(x, y, rows, c, ldx, ldy); break;
      case 2: softmax_rows_v4<2><<<grid, 256, 0, s>>>(x, y, rows, c, ldx, ldy); break;
      case 4: softmax_rows_v4<4><<<grid, 256, 0, s>>>(x, y, rows, c, ldx, ldy); break;
      case 8: softmax_rows_v4<8><<<grid, 256, 0, s>>>(x, y, rows, c, ldx, ldy); break;
      default: softmax_rows_v4<16><<<grid, 256, 0, s>>>(x, y, rows, c, ldx, ldy); break;
    }
  } else {
    PDH_REQUIRE(rows <= INT32_MAX, PDH_EINVAL, "pdh_row_softmax: too many rows");
    softmax_rows_stream<<<dim3(static_cast<unsigned>(rows)), 256, 0, s>>>(x, y, cols, ldx, ldy);
  }
  return check_launch("pdh_row_softmax");
}

extern "C" int pdh_layernorm(const float* x, const float* gamma, const float* beta, float* y, int64_t rows,
                             int64_t cols, int64_t ldx, int64_t ldy, float eps, void* stream) {
  PDH_REQUIRE(rows >= 0 && cols >= 1, PDH_EINVAL, "pdh_layernorm: need rows >= 0 and cols >= 1 (got %lld, %lld)",
              (long long)rows, (long long)cols);
  PDH_REQUIRE(ldx >= cols && ldy >= cols, PDH_EINVAL,
              "pdh_layernorm: row strides (%lld, %lld) must be >= cols (%lld)", (long long)ldx, (long long)ldy,
              (long long)cols);
  PDH_REQUIRE(rows == 0 || (x && y), PDH_EINVAL, "pdh_layernorm: null pointer");
  PDH_REQUIRE(eps >= 0.f, PDH_EINVAL, "pdh_layernorm: eps must be >= 0");
  PDH_REQUIRE(rows <= (int64_t)INT32_MAX * kRowsPerBlock, PDH_EINVAL, "pdh_layernorm: too many rows");
  if (rows == 0) return PDH_OK;
  hipStream_t s = as_stream(stream);
  if (fast_ok(x, y, cols, ldx, ldy, gamma, beta)) {
    const dim3 grid(static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const int c = static_cast<int>(cols);
    const bool aff = gamma || beta;
#define PDH_LN(NV)                                                                                   \
  do {                                                                                               \
    if (aff)                                                                                         \
      layernorm_rows_v4<NV, true><<<grid, 256, 0, s>>>(x, gamma, beta, y, rows, c, ldx, ldy, eps);  \
    else                                                                                             \
      layernorm_rows_v4<NV, false><<<grid, 256, 0, s>>>(x, gamma, beta, y, rows, c, ldx, ldy, eps); \
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
    PDH_REQUIRE(rows <= INT32_MAX, PDH_EINVAL, "pdh_layernorm: too many rows");
    layernorm_rows_stream<<<dim3(static_cast<unsigned>(rows)), 256, 0, s>>>(x, gamma, beta, y, cols, ldx, ldy, eps);
  }
  return check_launch("pdh_layernorm");
}
