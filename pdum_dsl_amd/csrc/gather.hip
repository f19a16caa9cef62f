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
