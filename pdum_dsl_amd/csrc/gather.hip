// Row gather: out[i, :] = table[idx[i], :] — the device form of tl.take along
// a table's leading dim (indexing.py:192-230 in the reference), which the
// carved-plan executor runs for a model's embedding lookup. The reference has
// no template row for a gather (the planner marks it red); its executor runs
// red groups through the CPU oracle, this build runs this one on the device.
//
// One workgroup copies one output row in 16-byte, 4-byte or 2-byte words
// (the widest the row's bytes and alignments allow). An index outside
// [0, n_rows) writes a zero row and is counted in *bad (a device int the
// caller clears and reads back), since a kernel cannot raise.
//
// Row scatter-add: out[v, :] = sum of values[i, :] over the i with
// idx[i] == v — tl.scatter_add, the gather's adjoint (indexing.py:153-190,
// 223-259), which a model's gradient needs for its embedding tables. It is
// deterministic without sorting or scratch memory: rows start at zero, and
// the workgroup of the FIRST position holding v owns row v (a later
// position finds an earlier equal index and leaves), sums the matching
// value rows in increasing position order in fp32 and rounds once. Finding
// the owner and its matches reads the index array once per position
// (n_idx^2 / 2 int64 compares from L2 in all), so the entry point accepts
// at most kScatterMaxIdx = 2^16 indices (an embedding batch of 64K tokens:
// ~2^31 compares, some milliseconds) and refuses more. The owner records
// the matches as 64-bit lane masks in LDS (8 KB at the limit) once, so rows
// wider than one 1024-column pass do not repeat the scan.
#include "common.h"

namespace pdh {
namespace {

template <typename W>
__global__ __launch_bounds__(256) void take_rows(const unsigned char* __restrict__ table,
                                                 const int64_t* __restrict__ idx, unsigned char* __restrict__ out,
                                                 int64_t n_rows, int64_t words, int64_t ld_table_b,
                                                 int64_t ld_out_b, int* __restrict__ bad) {
  const int64_t i = blockIdx.x;
  const int64_t r = idx[i];
  W* dst = reinterpret_cast<W*>(out + i * ld_out_b);
  if (r < 0 || r >= n_rows) {
    for (int64_t w = threadIdx.x; w < words; w += blockDim.x) dst[w] = W{};
    if (threadIdx.x == 0 && bad) atomicAdd(bad, 1);
    return;
  }
  const W* src = reinterpret_cast<const W*>(table + r * ld_table_b);
  for (int64_t w = threadIdx.x; w < words; w += blockDim.x) dst[w] = src[w];
}

template <typename W>
__global__ __launch_bounds__(256) void zero_rows(unsigned char* __restrict__ out, int64_t n_rows, int64_t words,
                                                 int64_t ld_out_b) {
  for (int64_t r = blockIdx.x; r < n_rows; r += gridDim.x) {
    W* dst = reinterpret_cast<W*>(out + r * ld_out_b);
    for (int64_t w = threadIdx.x; w < words; w += blockDim.x) dst[w] = W{};
  }
}

constexpr int kScatterCols = 4;                 // columns per lane per pass over the matches: 1024 per workgroup
constexpr int64_t kScatterMaxIdx = int64_t{1} << 16;  // positions per launch (the scan is quadratic)

// One workgroup per index position i (256 lanes, 4 waves).
template <int DT>
__global__ __launch_bounds__(256) void scatter_add_rows(const unsigned char* __restrict__ values,
                                                        const int64_t* __restrict__ idx,
                                                        unsigned char* __restrict__ out, int64_t n_idx,
                                                        int64_t row_elems, int64_t n_rows, int64_t ld_values_b,
                                                        int64_t ld_out_b, int* __restrict__ bad) {
  // hit masks of positions [i, n_idx): mask k covers positions i + 64 k .. + 63
  __shared__ uint64_t hits[kScatterMaxIdx / 64];
  const int64_t i = blockIdx.x;
  const int64_t v = idx[i];
  if (v < 0 || v >= n_rows) {  // dropped, and counted once per position
    if (threadIdx.x == 0 && bad) atomicAdd(bad, 1);
    return;
  }
  for (int64_t j0 = 0; j0 < i; j0 += 256) {  // an earlier equal index owns the row
    const int64_t j = j0 + threadIdx.x;
    if (__syncthreads_or(j < i && idx[j] == v)) return;
  }
  const int lane = threadIdx.x & 63;
  const int64_t nm = (n_idx - i + 63) / 64;  // masks over [i, n_idx)
  for (int64_t k0 = 0; k0 < nm; k0 += 4) {
    const int64_t k = k0 + (threadIdx.x >> 6), j = i + 64 * k + lane;
    const uint64_t m = __builtin_amdgcn_ballot_w64(j < n_idx && idx[j] == v);
    if (lane == 0 && k < nm) hits[k] = m;
  }
  __syncthreads();
  for (int64_t c0 = 0; c0 < row_elems; c0 += 256 * kScatterCols) {
    float acc[kScatterCols] = {};
    for (int64_t k = 0; k < nm; ++k) {
      for (uint64_t mm = hits[k]; mm; mm &= mm - 1) {  // matches in increasing position order
        const unsigned char* row = values + (i + 64 * k + __builtin_ctzll(mm)) * ld_values_b;
#pragma unroll
        for (int c = 0; c < kScatterCols; ++c) {
          const int64_t col = c0 + threadIdx.x + c * 256;
          if (col < row_elems) acc[c] += ld_dt<DT>(row, static_cast<int>(col));
        }
      }
    }
    unsigned char* orow = out + v * ld_out_b;
#pragma unroll
    for (int c = 0; c < kScatterCols; ++c) {
      const int64_t col = c0 + threadIdx.x + c * 256;
      if (col < row_elems) st_dt<DT>(orow, col, acc[c]);
    }
  }
}

}  // namespace
}  // namespace pdh

using namespace pdh;

extern "C" int pdh_take_rows(const void* table, const int64_t* idx, void* out, int64_t n_idx, int64_t row_elems,
                             int64_t n_rows, int64_t ld_table, int64_t ld_out, int dtype, int* bad, void* stream) {
  PDH_REQUIRE(dtype == PDH_F32 || dtype == PDH_BF16 || dtype == PDH_F16, PDH_EUNSUPPORTED,
              "pdh_take_rows: dtype %d", dtype);
  PDH_REQUIRE(n_idx >= 0 && row_elems >= 1 && n_rows >= 1, PDH_EINVAL,
              "pdh_take_rows: need n_idx >= 0, row_elems >= 1, n_rows >= 1");
  PDH_REQUIRE(ld_table >= row_elems && ld_out >= row_elems, PDH_EINVAL,
              "pdh_take_rows: row strides must be >= row_elems");
  PDH_REQUIRE(n_idx <= INT32_MAX, PDH_EINVAL, "pdh_take_rows: too many indices");
  if (n_idx == 0) return PDH_OK;
  PDH_REQUIRE(table && idx && out, PDH_EINVAL, "pdh_take_rows: null pointer");
  const int64_t es = dtype == PDH_F32 ? 4 : 2;
  const int64_t row_b = row_elems * es, lt = ld_table * es, lo = ld_out * es;
  const uintptr_t al = reinterpret_cast<uintptr_t>(table) | reinterpret_cast<uintptr_t>(out);
  hipStream_t s = as_stream(stream);
  const dim3 grid(static_cast<unsigned>(n_idx));
  auto fits = [&](int64_t w) { return row_b % w == 0 && lt % w == 0 && lo % w == 0 && al % w == 0; };
  const auto* tb = static_cast<const unsigned char*>(table);
  auto* ob = static_cast<unsigned char*>(out);
  if (fits(16))
    take_rows<u32x4><<<grid, 256, 0, s>>>(tb, idx, ob, n_rows, row_b / 16, lt, lo, bad);
  else if (fits(4))
    take_rows<uint32_t><<<grid, 256, 0, s>>>(tb, idx, ob, n_rows, row_b / 4, lt, lo, bad);
  else
    take_rows<uint16_t><<<grid, 256, 0, s>>>(tb, idx, ob, n_rows, row_b / 2, lt, lo, bad);
  return check_launch("pdh_take_rows");
}

extern "C" int pdh_scatter_add_rows(const void* values, const int64_t* idx, void* out, int64_t n_idx,
                                    int64_t row_elems, int64_t n_rows, int64_t ld_values, int64_t ld_out, int dtype,
                                    int* bad, void* stream) {
  PDH_REQUIRE(dtype == PDH_F32 || dtype == PDH_BF16 || dtype == PDH_F16, PDH_EUNSUPPORTED,
              "pdh_scatter_add_rows: dtype %d", dtype);
  PDH_REQUIRE(n_idx >= 0 && row_elems >= 1 && n_rows >= 1, PDH_EINVAL,
              "pdh_scatter_add_rows: need n_idx >= 0, row_elems >= 1, n_rows >= 1");
  PDH_REQUIRE(row_elems <= INT32_MAX, PDH_EINVAL, "pdh_scatter_add_rows: rows of more than 2^31 - 1 elements");
  PDH_REQUIRE(ld_values >= row_elems && ld_out >= row_elems, PDH_EINVAL,
              "pdh_scatter_add_rows: row strides must be >= row_elems");
  PDH_REQUIRE(n_idx <= kScatterMaxIdx, PDH_EUNSUPPORTED,
              "pdh_scatter_add_rows: %lld indices, more than the %lld one launch takes (the owner scan is quadratic)",
              (long long)n_idx, (long long)kScatterMaxIdx);
  PDH_REQUIRE(out && (n_idx == 0 || (values && idx)), PDH_EINVAL, "pdh_scatter_add_rows: null pointer");
  const int64_t es = dtype == PDH_F32 ? 4 : 2;
  const int64_t row_b = row_elems * es, lo = ld_out * es;
  const uintptr_t al = reinterpret_cast<uintptr_t>(out);
  hipStream_t s = as_stream(stream);
  auto* ob = static_cast<unsigned char*>(out);
  const dim3 zgrid(static_cast<unsigned>(n_rows < 8192 ? n_rows : 8192));
  auto fits = [&](int64_t w) { return row_b % w == 0 && lo % w == 0 && al % w == 0; };
  if (fits(16))
    zero_rows<u32x4><<<zgrid, 256, 0, s>>>(ob, n_rows, row_b / 16, lo);
  else if (fits(4))
    zero_rows<uint32_t><<<zgrid, 256, 0, s>>>(ob, n_rows, row_b / 4, lo);
  else
    zero_rows<uint16_t><<<zgrid, 256, 0, s>>>(ob, n_rows, row_b / 2, lo);
  if (int rc = check_launch("pdh_scatter_add_rows (zero)"); rc != PDH_OK) return rc;
  if (n_idx == 0) return PDH_OK;
  const auto* vb = static_cast<const unsigned char*>(values);
  const dim3 grid(static_cast<unsigned>(n_idx));
  const int64_t lv = ld_values * es;
  if (dtype == PDH_F32)
    scatter_add_rows<PDH_F32><<<grid, 256, 0, s>>>(vb, idx, ob, n_idx, row_elems, n_rows, lv, lo, bad);
  else if (dtype == PDH_BF16)
    scatter_add_rows<PDH_BF16><<<grid, 256, 0, s>>>(vb, idx, ob, n_idx, row_elems, n_rows, lv, lo, bad);
  else
    scatter_add_rows<PDH_F16><<<grid, 256, 0, s>>>(vb, idx, ob, n_idx, row_elems, n_rows, lv, lo, bad);
  return check_launch("pdh_scatter_add_rows");
}
