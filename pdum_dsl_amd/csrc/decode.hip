// Decode attention, split over the key axis — the flash row at a handful of
// query rows per head, where the work is reading the key/value cache once.
//
// Pass 1 (decode_split): one workgroup per (batch, kv head, split). The
// heads_q / heads_kv query heads of the group (x t query rows, at most 16)
// are packed into the workgroup, so every cache byte is read from HBM exactly
// once. Each wave sweeps every fourth 32-key block of its split, with the next
// block's K and V rows in flight (registers) while the current one computes:
//   S^T = K Q^T    v_mfma_f32_16x16x32, K rows straight from the loads as the
//                  A operand (16 keys x 32 features per lane group), the query
//                  rows as the B operand (16 columns; unused ones are zero)
//   online softmax per query column (lane = column; max over the 4 lane groups)
//   O^T += V^T P^T the probabilities stay in registers as the B operand; V goes
//                  through a wave-private LDS tile and comes back transposed
//                  (ds_read_b64_tr_b16) as the A operand.
// The waves' states combine through LDS and the workgroup writes one partial
// (m, den, o) per query row. The work per cache byte is a few MFMA cycles, so
// the sweep runs at the rate the loads arrive.
//
// Pass 2 (decode_merge): one wave per query row folds the splits' partials
// with the associative online-softmax combine (flashsm, zoo/attention.py:40-46):
//   m = max(mL, mR); den = denL e^(mL-m) + denR e^(mR-m); o likewise.
#include "attn_common.h"

#include <mutex>

namespace pdh {
namespace {

constexpr float kInf = __builtin_inff();
constexpr int kMaxNq = 16;  // query rows per workgroup (heads_q / heads_kv * t): the MFMA's 16 columns

struct DecArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t heads_q, heads_kv, t, s;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st;
  float c2;  // scale * log2(e)
  int nsplit;
  int64_t chunk;  // keys per split (multiple of 32)
  float* ws;      // [batch*heads_q*t][nsplit][2 + D]
};

// Block geometry: 32 keys per block (two 16-key score tiles).
template <int D>
struct DecCfg {
  static constexpr int KB = 32;
  static constexpr int KS = D / 32;       // k-steps of the score product (16x16x32)
  static constexpr int ET = D / 16;       // 16-feature tiles of the output product
  static constexpr int CPR = D / 8;       // 16-byte chunks per cache row
  static constexpr int RPI = 64 / CPR;    // value rows per 1 KB wave load
  static constexpr int VL = KB / RPI;     // value loads per block
  static constexpr int VROW = D * 2 + 32; // LDS bytes per value row (32-byte pad: conflict-free transposed reads)
  static constexpr int VTILE = KB * VROW; // one wave's value tile
  static constexpr int RS = 2 + D;        // floats per (wave, query row) record
  static constexpr int RED = 4 * kMaxNq * RS * 4;
  static constexpr int LDS = 4 * VTILE > RED ? 4 * VTILE : RED;
};

template <typename T, int D>
__global__ __launch_bounds__(256, 2) void decode_split(DecArgs a) {
  using C = DecCfg<D>;
  constexpr int KS = C::KS, ET = C::ET, VL = C::VL;
  extern __shared__ __attribute__((aligned(1024))) unsigned char dsm[];
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int col = lane & 15, g = lane >> 4;  // MFMA column (query row) and lane group
  const int R = static_cast<int>(a.heads_q / a.heads_kv);
  const int64_t nsplit = a.nsplit;
  const int64_t split = blockIdx.x % nsplit;
  const int64_t grp = blockIdx.x / nsplit;  // (batch, kv head)
  const int64_t b = grp / a.heads_kv, hk = grp % a.heads_kv;
  const uint16_t* kp = a.k + b * a.k_sb + hk * a.k_sh;
  const uint16_t* vp = a.v + b * a.v_sb + hk * a.v_sh;
  const int nq = R * static_cast<int>(a.t);

  // query rows as the score product's B operand: lane (col, g) holds row col
  // (= r * t + tq), features 32 s + 8 g .. +8; columns past nq are zero
  u32x4 qb[KS];
  {
    const bool live = col < nq;
    const int qc = live ? col : 0;
    const int64_t hq = hk * R + qc / a.t, tq = qc % a.t;
    const uint16_t* qrow = a.q + b * a.q_sb + hq * a.q_sh + tq * a.q_st;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(qrow + s * 32 + g * 8);
      qb[s] = live ? v : u32x4{0u, 0u, 0u, 0u};
    }
  }

  const int64_t k_begin = split * a.chunk;
  const int64_t k_end = (k_begin + a.chunk < a.s) ? k_begin + a.chunk : a.s;
  unsigned char* vt = dsm + w * C::VTILE;
  const uint32_t kst2 = static_cast<uint32_t>(a.k_st * 2), vst2 = static_cast<uint32_t>(a.v_st * 2);
  const int vrow = lane / C::CPR, vch = lane % C::CPR;  // value loads: row j * RPI + vrow, chunk vch
  // transposed value reads: lane 4k + c of group g addresses row 4 g + k, features 4 c .. +3 (+ 16 t)
  const int trb = (4 * g + (col >> 2)) * C::VROW + (col & 3) * 8;

  // Cache rows past k_end are clamped to the last live row (their scores are masked).
  auto load = [&](int64_t kb, u32x4(&kr)[2 * KS], u32x4(&vr)[VL]) {
    const int lim = static_cast<int>(k_end - 1 - kb < 31 ? k_end - 1 - kb : 31);
    const uint16_t* kbase = kp + kb * a.k_st;
    const uint16_t* vbase = vp + kb * a.v_st;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const int r = 16 * kt + col < lim ? 16 * kt + col : lim;
      const uint32_t off = static_cast<uint32_t>(r) * kst2 + g * 16;
#pragma unroll
      for (int s = 0; s < KS; ++s) kr[kt * KS + s] = gload<u32x4>(kbase, off + s * 64);
    }
#pragma unroll
    for (int j = 0; j < VL; ++j) {
      const int r = j * C::RPI + vrow < lim ? j * C::RPI + vrow : lim;
      vr[j] = gload<u32x4>(vbase, static_cast<uint32_t>(r) * vst2 + vch * 16);
    }
  };

  float m = -kInf, lsum = 0.f;  // running max (log2 units) and partial sum of query row col
  f32x4 o[ET];                  // O^T: o[t][i] = feature 16 t + 4 g + i of query row col
#pragma unroll
  for (int t = 0; t < ET; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto block = [&](int64_t kb, const u32x4(&kr)[2 * KS], const u32x4(&vr)[VL]) {
    // value rows -> this wave's LDS tile (row-major, padded rows)
#pragma unroll
    for (int j = 0; j < VL; ++j) *reinterpret_cast<u32x4*>(vt + (j * C::RPI + vrow) * C::VROW + vch * 16) = vr[j];
    // S^T = K Q^T for keys kb + 16 kt + 4 g + i (accumulator i), query row col
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      s0 = mfma16<T>(kr[s], qb[s], s0);
      s1 = mfma16<T>(kr[KS + s], qb[s], s1);
    }
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = s0[i] * a.c2;
      x[4 + i] = s1[i] * a.c2;
    }
    if (kb + C::KB > k_end) {  // the split's last block: keys past k_end are masked
      const int live = static_cast<int>(k_end - kb);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (4 * g + i >= live) x[i] = -kInf;
        if (16 + 4 * g + i >= live) x[4 + i] = -kInf;
      }
    }
    float mx = x[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mx = fmaxf(mx, x[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float mnew = fmaxf(m, mx);  // finite: every block holds a live key
    if (__builtin_amdgcn_ballot_w64(mnew > m) != 0) {  // some row's max grew: rescale (rare after warm-up)
      const float alpha = fast_exp2(m - mnew);
      lsum *= alpha;
#pragma unroll
      for (int t = 0; t < ET; ++t) o[t] *= alpha;
      m = mnew;
    }
    float p[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p[i] = fast_exp2(x[i] - m);
      lsum += p[i];
    }
    // P^T as the output product's B operand: slot j < 4 is key 4 g + j, j >= 4 key 16 + 4 g + j - 4
    const u32x4 pb = {pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3]), pack2<T>(p[4], p[5]), pack2<T>(p[6], p[7])};
    // O^T += V^T P^T: A operand lane (e = 16 t + col, group g) holds those 8 keys' values
#pragma unroll
    for (int t = 0; t < ET; ++t) {
      const u32x2 lo = ds_read_tr16(vt + trb + 32 * t);
      const u32x2 hi = ds_read_tr16(vt + trb + 16 * C::VROW + 32 * t);
      o[t] = mfma16<T>(u32x4{lo.x, lo.y, hi.x, hi.y}, pb, o[t]);
    }
  };

  // Each wave takes every fourth block; the next block's K and V rows are in
  // flight (registers) while this one is computed. The loads are issued
  // unconditionally (past the wave's last block they re-read that block, an
  // L2 hit) so the compiler's wait counts stay exact: a block waits only for
  // its own rows, never for the prefetch behind them.
  const int64_t stride = 4 * C::KB;
  const int64_t kb0 = k_begin + C::KB * w;
  if (kb0 < k_end) {
    const int64_t kb_last = kb0 + (k_end - 1 - kb0) / stride * stride;
    auto next = [&](int64_t kb) { return kb + stride < kb_last ? kb + stride : kb_last; };
    u32x4 ka0[2 * KS], va0[VL], ka1[2 * KS], va1[VL];
    int64_t kb = kb0;
    load(kb, ka0, va0);
    for (;;) {
      load(next(kb), ka1, va1);
      block(kb, ka0, va0);
      kb += stride;
      if (kb >= k_end) break;
      load(next(kb), ka0, va0);
      block(kb, ka1, va1);
      kb += stride;
      if (kb >= k_end) break;
    }
  }
  lsum += __shfl_xor(lsum, 16, kWave);
  lsum += __shfl_xor(lsum, 32, kWave);

  // per-wave state -> LDS (over the value tiles), then combine the four waves
  __syncthreads();
  constexpr int RS = C::RS;
  float* red = reinterpret_cast<float*>(dsm);
  if (col < nq) {
    float* rec = red + (w * kMaxNq + col) * RS;
    if (g == 0) {
      rec[0] = m;
      rec[1] = lsum;
    }
#pragma unroll
    for (int t = 0; t < ET; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) rec[2 + 16 * t + 4 * g + i] = o[t][i];
  }
  __syncthreads();
  const int64_t q_row0 = (b * a.heads_q + hk * R) * a.t;  // first stats row of the group
  for (int c = tid; c < nq * RS; c += 256) {
    const int qi = c / RS, f = c % RS;
    float mm = -kInf;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) mm = fmaxf(mm, red[(ww * kMaxNq + qi) * RS]);
    float val = 0.f;
    if (f == 0) {
      val = mm;
    } else {
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        const float mw = red[(ww * kMaxNq + qi) * RS];
        const float sc = mw == -kInf ? 0.f : fast_exp2(mw - mm);
        val += red[(ww * kMaxNq + qi) * RS + f] * sc;
      }
    }
    // qi = r * t + tq matches the stats row order (head-major, then row)
    a.ws[((q_row0 + qi) * nsplit + split) * RS + f] = val;
  }
}

template <typename T, int D>
__global__ __launch_bounds__(256) void decode_merge(const float* __restrict__ ws, uint16_t* o, float* lse,
                                                    int64_t nrows, int nsplit, int64_t heads_q, int64_t t,
                                                    int64_t o_sb, int64_t o_sh, int64_t o_st) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= nrows) return;
  const float* pr = ws + row * nsplit * (2 + D);
  float mm = -kInf;
  for (int sp = 0; sp < nsplit; ++sp) mm = fmaxf(mm, pr[sp * (2 + D)]);
  float den = 0.f;
  float acc[D / 64];
#pragma unroll
  for (int j = 0; j < D / 64; ++j) acc[j] = 0.f;
  for (int sp = 0; sp < nsplit; ++sp) {
    const float* ps = pr + sp * (2 + D);
    const float sc = ps[0] == -kInf ? 0.f : fast_exp2(ps[0] - mm);
    den += ps[1] * sc;
#pragma unroll
    for (int j = 0; j < D / 64; ++j) acc[j] += ps[2 + j * 64 + lane] * sc;
  }
  const int64_t inst = row / t, tq = row % t;
  const int64_t b = inst / heads_q, hq = inst % heads_q;
  uint16_t* orow = o + b * o_sb + hq * o_sh + tq * o_st;
  const float inv = 1.0f / den;
#pragma unroll
  for (int j = 0; j < D / 64; ++j) orow[j * 64 + lane] = Elem<T>::from_f32(acc[j] * inv);
  if (lane == 0 && lse) lse[row] = (mm + __log2f(den)) * kLn2;
}

template <typename T, int D>
int launch_decode(const DecArgs& a, int64_t nrows, uint16_t* o, float* lse, int64_t o_sb, int64_t o_sh,
                  int64_t o_st, int64_t groups, hipStream_t st) {
  const int64_t nblk = groups * a.nsplit;
  PDH_REQUIRE(nblk <= INT32_MAX, PDH_EINVAL, "pdh_attn_decode: grid too large");
  const dim3 grid(static_cast<unsigned>(nblk));
  constexpr int lds = DecCfg<D>::LDS;
  hipFuncSetAttribute(reinterpret_cast<const void*>(decode_split<T, D>), hipFuncAttributeMaxDynamicSharedMemorySize,
                      lds);
  decode_split<T, D><<<grid, 256, lds, st>>>(a);
  int rc = check_launch("pdh_attn_decode (split)");
  if (rc) return rc;
  decode_merge<T, D><<<dim3(static_cast<unsigned>((nrows + 3) / 4)), 256, 0, st>>>(
      a.ws, o, lse, nrows, a.nsplit, a.heads_q, a.t, o_sb, o_sh, o_st);
  return check_launch("pdh_attn_decode (merge)");
}

}  // namespace
}  // namespace pdh

using namespace pdh;

// ---- the allocation-free variant: the split workspace in a library-held array
//
// One array per GPU, of PDH_DECODE_SCRATCH_BYTES, in the code object's device
// memory (allocated when the library's code object loads on that GPU, held
// until the process ends). Host code must never pass `pdh_decode_scratch` itself
// to a kernel: in host code the name is a host-side stand-in, not a device
// address. Its device address is looked up once per device, with that device
// current, by hipGetSymbolAddress, and kept per device; only that address is
// handed to the kernels. Every call on a GPU shares that GPU's array (calls
// that overlap on one GPU race); each call writes every (row, split) partial
// it reads, so nothing has to be cleared between calls.
// External linkage on purpose: with `static` the array is a local (STB_LOCAL)
// symbol of the device code object, which the runtime's symbol lookup behind
// hipGetSymbolAddress cannot resolve; the pdh_ prefix keeps the name unique.
__device__ __align__(256) unsigned char pdh_decode_scratch[PDH_DECODE_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};

int decode_scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  PDH_REQUIRE(e == hipSuccess, PDH_ELAUNCH, "pdh_attn_decode_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
  PDH_REQUIRE(dev >= 0 && dev < kMaxDevices, PDH_EUNSUPPORTED, "pdh_attn_decode_noalloc: device %d >= %d", dev,
              kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(pdh_decode_scratch));
    PDH_REQUIRE(e == hipSuccess && p != nullptr, PDH_ELAUNCH,
                "pdh_attn_decode_noalloc: hipGetSymbolAddress(pdh_decode_scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return PDH_OK;
}

}  // namespace

extern "C" size_t pdh_attn_decode_workspace(const pdh_attn_geom* g, int nsplit) {
  if (!g || nsplit < 1 || g->batch < 0 || g->heads_q < 1 || g->t < 0 || g->od < 1) return 0;
  return static_cast<size_t>(g->batch * g->heads_q * g->t) * static_cast<size_t>(nsplit) *
         static_cast<size_t>(2 + g->od) * sizeof(float);
}

extern "C" int pdh_attn_decode(const void* q, const void* k, const void* v, void* o, float* lse_out,
                               const pdh_attn_geom* gm, int dtype, float scale, int nsplit, void* ws,
                               size_t ws_bytes, void* stream) {
  PDH_REQUIRE(gm != nullptr, PDH_EINVAL, "pdh_attn_decode: null geometry");
  const pdh_attn_geom G = *gm;
  PDH_REQUIRE(G.batch >= 0 && G.heads_q >= 1 && G.heads_kv >= 1 && G.t >= 1 && G.s >= 1, PDH_EINVAL,
              "pdh_attn_decode: bad shape");
  PDH_REQUIRE(G.heads_q % G.heads_kv == 0, PDH_EINVAL, "pdh_attn_decode: heads_q must be a multiple of heads_kv");
  PDH_REQUIRE(dtype == PDH_BF16 || dtype == PDH_F16, PDH_EUNSUPPORTED, "pdh_attn_decode: dtype must be bf16 or f16");
  PDH_REQUIRE(G.e == G.od && (G.e == 64 || G.e == 128), PDH_EUNSUPPORTED,
              "pdh_attn_decode: need e == od in {64, 128} (got %lld, %lld)", (long long)G.e, (long long)G.od);
  const int64_t nq = (G.heads_q / G.heads_kv) * G.t;
  PDH_REQUIRE(nq <= kMaxNq, PDH_EUNSUPPORTED,
              "pdh_attn_decode: heads_q/heads_kv * t = %lld query rows per kv head exceeds %d (use pdh_flash_fwd)",
              (long long)nq, kMaxNq);
  PDH_REQUIRE(nsplit >= 1, PDH_EINVAL, "pdh_attn_decode: nsplit must be >= 1");
  PDH_REQUIRE(q && k && v && o && ws, PDH_EINVAL, "pdh_attn_decode: null pointer");
  PDH_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(ws), PDH_EINVAL,
              "pdh_attn_decode: q/k/v/ws must be 16-byte aligned");
  PDH_REQUIRE(G.q_st % 8 == 0 && G.k_st % 8 == 0 && G.v_st % 8 == 0 && G.q_sh % 8 == 0 && G.k_sh % 8 == 0 &&
                  G.v_sh % 8 == 0 && G.q_sb % 8 == 0 && G.k_sb % 8 == 0 && G.v_sb % 8 == 0,
              PDH_EINVAL, "pdh_attn_decode: strides must be multiples of 8 elements");
  const size_t need = pdh_attn_decode_workspace(gm, nsplit);
  PDH_REQUIRE(G.k_st < (1 << 24) && G.v_st < (1 << 24), PDH_EINVAL,
              "pdh_attn_decode: row strides must be < 2^24 elements");
  PDH_REQUIRE(ws_bytes >= need, PDH_EINVAL, "pdh_attn_decode: workspace %zu bytes < required %zu", ws_bytes, need);
  if (G.batch == 0) return PDH_OK;
  int64_t chunk = (G.s + nsplit - 1) / nsplit;
  chunk = (chunk + 31) / 32 * 32;
  DecArgs a{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
            G.heads_q, G.heads_kv, G.t, G.s, G.q_sb, G.q_sh, G.q_st, G.k_sb, G.k_sh, G.k_st, G.v_sb, G.v_sh,
            G.v_st, scale * kLog2e, nsplit, chunk, static_cast<float*>(ws)};
  const int64_t nrows = G.batch * G.heads_q * G.t;
  const int64_t groups = G.batch * G.heads_kv;
  hipStream_t st = as_stream(stream);
  uint16_t* op = static_cast<uint16_t*>(o);
  if (dtype == PDH_BF16)
    return G.e == 128 ? launch_decode<__hip_bfloat16, 128>(a, nrows, op, lse_out, G.o_sb, G.o_sh, G.o_st,
                                                           groups, st)
                      : launch_decode<__hip_bfloat16, 64>(a, nrows, op, lse_out, G.o_sb, G.o_sh, G.o_st,
                                                          groups, st);
  return G.e == 128
             ? launch_decode<_Float16, 128>(a, nrows, op, lse_out, G.o_sb, G.o_sh, G.o_st, groups, st)
             : launch_decode<_Float16, 64>(a, nrows, op, lse_out, G.o_sb, G.o_sh, G.o_st, groups, st);
}

extern "C" int pdh_attn_decode_noalloc(const void* q, const void* k, const void* v, void* o, float* lse_out,
                                       const pdh_attn_geom* gm, int dtype, float scale, int nsplit, void* stream) {
  PDH_REQUIRE(gm != nullptr, PDH_EINVAL, "pdh_attn_decode_noalloc: null geometry");
  PDH_REQUIRE(nsplit >= 1, PDH_EINVAL, "pdh_attn_decode_noalloc: nsplit must be >= 1");
  const size_t need = pdh_attn_decode_workspace(gm, nsplit);
  PDH_REQUIRE(need <= PDH_DECODE_SCRATCH_BYTES, PDH_EINVAL,
              "pdh_attn_decode_noalloc: this request needs %zu bytes of split workspace; the library's scratch "
              "array holds %zu (fewer splits or rows, or pdh_attn_decode with a caller workspace)",
              need, static_cast<size_t>(PDH_DECODE_SCRATCH_BYTES));
  void* ws = nullptr;
  const int rc = decode_scratch_address(&ws);
  if (rc != PDH_OK) return rc;
  return pdh_attn_decode(q, k, v, o, lse_out, gm, dtype, scale, nsplit, ws, PDH_DECODE_SCRATCH_BYTES, stream);
}
