// Flash-attention backward — the closed form of the flash joint's gradients
// (autodiff.grad over the naive twin, autodiff.py:102-122; the reference
// executes it as a carved plan of contraction kernels, partition.py:586-607).
// Like the reference's carving, every output is owned by exactly one program
// (330 §7.8 ruling 4): no atomics.
//
//   bwd_stats : per query row: -delta (delta = sum_d dO O), -lse / scale and
//               pm, the probability of a MASKED score (0 unless every key of
//               the row is masked; then 1/den, the uniform-softmax row)  (HBM-bound)
//   bwd16_dkdv: grid over 128-key blocks (4 waves x 32 keys); sweeps query
//               tiles; each wave keeps its K and V rows in registers and
//               accumulates dK^T, dV^T:
//                 S = Q K^T - lse, dP = dO V^T - delta  (A = Q / dO rows from LDS)
//                 P = exp(scale S), dS = P dP
//                 dV^T += dO^T P, dK^T += Q^T dS        (A = dO^T / Q^T from LDS)
//   bwd16_dq  : grid over 128-query blocks; sweeps key tiles:
//                 S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T
//
// Grouped-query attention (heads_q = group x heads_kv, query head h reading
// K / V head h / group): a dK / dV workgroup sweeps the query tiles of every
// query head of its group in turn into the same accumulators, and a dQ
// workgroup reads its group's K and V. Every output still has one owner.
//
// All products are v_mfma_f32_16x16x32 (bf16 / f16 in, fp32 accumulate), in
// the forward's layout (see the 16x16x32 section): the score accumulators
// feed the next contraction's k operand with no register shuffle, and the
// transposed operands (Q^T, dO^T, K^T) are read from the same LDS tiles by
// ds_read_b64_tr_b16. Tiles live for the whole workgroup run a mask-free
// body; masked tiles give a masked score its row's pm as probability (0 for
// any row with a live key) and no gradient (dS = 0), as the where() adjoint.
#include "attn_common.h"

#include <type_traits>

namespace pdh {
namespace {

struct BwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const float* lse;
  const float* m_in;    // optional forward artifacts (exact fully-masked rows)
  const float* den_in;
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  float* ws;            // [3][rows]: -delta, lse2, pm
  int64_t rows;         // batch * heads * t (query rows)
  int64_t heads, t, s;  // heads: query heads
  int64_t heads_kv;     // K / V heads; query head h reads K / V head h / group
  int group;            // heads / heads_kv
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
  float scale, c2, fill2;
  int masked;
  int64_t band_lo, band_hi;
  int prune;
  int ninst;          // batch * heads (query instances)
  int ninst_kv;       // batch * heads_kv (K / V instances)
  int nkblk, nqblk;   // 128-key blocks (dK, dV) per K / V instance, 128-query blocks (dQ) per query instance
  int xcd_remap;
  // the band clamped to +-(2^29 + 64): with t, s <= 2^29 every key - query
  // difference compares the same against these as against the 64-bit band
  int band_lo32, band_hi32;
};

// ---------------------------------------------------------------- row stats

// One row per D/8 lanes (16 bytes of O and dO each): 8 rows per wave at D = 64.
template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_stats(BwdArgs a) {
  constexpr int LPR = D / 8, RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR;
  const int sub = lane % LPR;
  float acc = 0.f;
  if (row < a.rows) {
    const int64_t inst = row / a.t, tq = row % a.t;
    const int64_t b = inst / a.heads, h = inst % a.heads;
    const int64_t off = b * a.o_sb + h * a.o_sh + tq * a.o_st + sub * 8;
    const u32x4 o4 = *reinterpret_cast<const u32x4*>(a.o + off);
    const u32x4 d4 = *reinterpret_cast<const u32x4*>(a.dout + off);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc += lo_f32<T>(o4[j]) * lo_f32<T>(d4[j]) + hi_f32<T>(o4[j]) * hi_f32<T>(d4[j]);
  }
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (row < a.rows && sub == 0) {
    float lse2, pm = 0.f;
    if (a.m_in != nullptr) {
      const float m2 = a.m_in[row] * kLog2e, den = a.den_in[row];
      lse2 = m2 + __log2f(den);
      if (a.masked) pm = fast_exp2(a.fill2 - m2) / den;  // exact 1/den for a fully-masked row
    } else {
      lse2 = a.lse[row] * kLog2e;
      // fully masked: lse = fill + log(s) is the fill in fp32 (uniform row, P = 1/s)
      if (a.masked) pm = (lse2 - a.fill2 < 64.f) ? 1.0f / static_cast<float>(a.s) : fast_exp2(a.fill2 - lse2);
    }
    a.ws[row] = -acc;  // -delta: the dP accumulators start from it
    a.ws[a.rows + row] = -lse2 / a.c2;  // -lse / scale: the S accumulators of the dK / dV role start from it
    a.ws[2 * a.rows + row] = pm;
  }
}

// ---------------------------------------------------- 16x16x32 backward
//
// Both roles in the forward's layout: v_mfma_f32_16x16x32 products, a wave
// owning 32 rows of its role's side as two 16-row halves (lane 16 G + c owns
// rows c and 16 + c), the swept tiles' 32 rows seen by a lane as {4G .. 4G+3}
// and {16+4G .. 16+4G+3}. Those eight rows are the k operand (k = 8G + j:
// row 4G + j for j < 4, 16 + 4G + j - 4 for j >= 4) of the second
// contraction, and the transposed LDS read names the same rows per 16-lane
// group, so the score accumulators feed it with no register shuffle. Tiles
// fully live for the whole workgroup run a mask-free body; the sweep runs in
// buffer pairs so every LDS address is a lane offset plus an immediate.

#ifndef PDH_BWD_SUB
#define PDH_BWD_SUB 2
#endif

template <int D>
struct B16 {
  static constexpr int NSUB = D == 64 ? PDH_BWD_SUB : 1;  // tiles staged per barrier (double buffered)
  static constexpr int ROWB = D * 2, CPR = D / 8, TILEB = 32 * ROWB, RPK = 1024 / ROWB, NBLK = TILEB / 1024;
  static constexpr int NDMA = (NBLK + 3) / 4;
  static constexpr int KS = D / 32;  // k-steps of 32 features
  static constexpr int FB = D / 16;  // 16-feature output blocks
};

// One XOR mask per row % 16 that keeps both read patterns of a tile
// bank-conflict free on gfx950's LDS, whose behaviour an in-bounds probe
// measured: a ds_read_b128 serves 16 lanes per cycle over 256 bytes of
// banks, and the 16 are not consecutive: within each 32-lane half, the
// quads (lane / 4 = q, 0..7) of even bit parity {0, 3, 5, 6} share a cycle
// and those of odd parity {1, 2, 4, 7} another, so their 16-byte slots must
// differ mod 16; an 8-byte read (ds_read_b64, ds_read_b64_tr_b16) serves 32
// consecutive lanes over 256 bytes (8-byte units mod 32). The patterns are
// row reads (lanes 16 G + c read row c at chunk 4 ks + G) and transposed
// reads (16-lane group G reads rows 4 G .. 4 G + 3, 32 bytes each);
// tests/test_lds_layout.py re-checks both.
template <int D>
__device__ __forceinline__ int swz16_rt(int row) {
  constexpr uint64_t kTable = D == 128 ? 0x6e4c2a08e6c4a280ull : 0x2266004466224400ull;
  return static_cast<int>((kTable >> (4 * (row & 15))) & 15u);
}

// Per-lane offsets into a 32-row tile (the same for every tensor: they share
// the layout) and the direct-load offsets of one tensor.
template <int D>
struct Lane16 {
  using C = B16<D>;
  int rowr[C::KS];  // row reads: row c, chunk 4 ks + G (+ 16 rows: immediate)
  int tr[C::FB];    // transposed reads: row 4 G + k4, features 16 fb + 4 cc (+ 16 rows: immediate)
  __device__ __forceinline__ void init(int lane) {
    const int G = lane >> 4, c = lane & 15, k4 = (lane >> 2) & 3, cc = lane & 3, row = 4 * G + k4;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) rowr[ks] = c * C::ROWB + (((4 * ks + G) ^ swz16_rt<D>(c)) << 4);
#pragma unroll
    for (int fb = 0; fb < C::FB; ++fb)
      tr[fb] = row * C::ROWB + (((2 * fb + (cc >> 1)) ^ swz16_rt<D>(row)) << 4) + ((cc & 1) << 3);
  }
  // A operand: rows 16 half + (0..15) x features 32 ks .. +32
  __device__ __forceinline__ u32x4 row_frag(const unsigned char* t, int half, int ks) const {
    return *reinterpret_cast<const u32x4*>(t + half * 16 * C::ROWB + rowr[ks]);
  }
  // A operand, transposed: features 16 fb .. +16 x the tile's 32 rows in k order
  __device__ __forceinline__ u32x4 tr_frag(const unsigned char* t, int fb) const {
    const u32x2 lo = ds_read_tr16(t + tr[fb]);
    const u32x2 hi = ds_read_tr16(t + 16 * C::ROWB + tr[fb]);
    return u32x4{lo.x, lo.y, hi.x, hi.y};
  }
};

// The tile rows cc (0..31, a compile-time index of each accumulator element)
// a lane keeps in a masked tile, as the window lo <= cc <= lo + span: each
// element's test is one unsigned compare whose result is used at once, so no
// per-element lane masks stay live across the tile (they would not fit the
// scalar registers). An empty window is lo = 32.
struct CutWindow {
  int lo;
  uint32_t span;
  __device__ __forceinline__ bool live(int cc) const { return static_cast<uint32_t>(cc - lo) <= span; }
};
__device__ __forceinline__ CutWindow cut_window(int lo, int hi) {
  lo = lo > 0 ? lo : 0;
  hi = hi < 31 ? hi : 31;
  if (hi < lo) lo = hi = 32;
  uint32_t span = static_cast<uint32_t>(hi - lo);
  // opaque to the optimizer: the element tests are made here, per tile, not
  // hoisted out of the sweep as lane masks that would not fit the scalar file
  asm volatile("" : "+v"(lo), "+v"(span));
  return CutWindow{lo, span};
}

template <int D>
__device__ __forceinline__ void dma_offsets(uint32_t (&off)[B16<D>::NDMA], int lane, int w, uint32_t gr) {
  using C = B16<D>;
  const int lrow = lane / C::CPR, slot = lane % C::CPR;
#pragma unroll
  for (int i = 0; i < C::NDMA; ++i) {
    const int rho = (i * 4 + w) * C::RPK + lrow;
    off[i] = lrow * gr + ((slot ^ swz16_rt<D>(rho)) << 4);
  }
}

// rows [row0, row0 + 32) of a tensor into a tile (every wave calls this)
template <int D>
__device__ __forceinline__ void dma_tile(rsrc_t r, unsigned char* lds, const uint32_t (&off)[B16<D>::NDMA],
                                         uint32_t row0, uint32_t gr, int w) {
  using C = B16<D>;
#pragma unroll
  for (int i = 0; i < C::NDMA; ++i) {
    const int blk = i * 4 + w;
    if (C::NBLK % 4 != 0 && blk >= C::NBLK) break;
    dma16(r, lds + blk * 1024, off[i], (row0 + blk * C::RPK) * gr);
  }
}

// The swept tiles of a 128-row owned block: the live range [lo, hi) and the
// run [flo, fhi) of tiles live for every (owned row, swept row) pair and
// inside the swept extent. d = key - query; owner_is_query picks the side.
struct Sweep {
  int lo, hi, flo, fhi;
};

__device__ __forceinline__ Sweep sweep_plan(const BwdArgs& a, int o0, int ext, bool owner_is_query) {
  constexpr int BO = 128, BT = 32;
  const int ntiles = (ext + BT - 1) / BT;
  int lo = 0, hi = ntiles;
  const int blo = a.band_lo32, bhi = a.band_hi32;
  if (a.masked && a.prune) {
    // swept rows x live for some owned row o in [o0, o0 + BO): lo_d <= d <= hi_d
    const int xmin = owner_is_query ? o0 + blo : o0 - bhi;
    const int xmax = owner_is_query ? o0 + BO - 1 + bhi : o0 + BO - 1 - blo;
    lo = xmin <= 0 ? 0 : (xmin / BT < ntiles ? xmin / BT : ntiles);
    hi = xmax < 0 ? 0 : (xmax / BT + 1 < ntiles ? xmax / BT + 1 : ntiles);
  }
  // fully live tiles: every d over the (owned block, tile) box inside the band, the tile inside ext
  int flo = lo, fhi = ext / BT < hi ? ext / BT : hi;
  if (a.masked) {
    // d ranges over [x0 - (o0 + BO - 1), x0 + BT - 1 - o0] (owner query) or [o0 - x0 - BT + 1, o0 + BO - 1 - x0]
    if (owner_is_query) {
      // x0 >= o0 + BO - 1 + blo and x0 + BT - 1 <= o0 + bhi
      const int a0 = o0 + BO - 1 + blo, b0 = o0 + bhi - (BT - 1);
      const int f0 = a0 <= 0 ? 0 : (a0 + BT - 1) / BT;
      const int f1 = b0 < 0 ? 0 : b0 / BT + 1;
      flo = flo > f0 ? flo : f0;
      fhi = fhi < f1 ? fhi : f1;
    } else {
      // o0 - (x0 + BT - 1) >= blo and o0 + BO - 1 - x0 <= bhi
      const int a0 = o0 + BO - 1 - bhi, b0 = o0 - blo - (BT - 1);
      const int f0 = a0 <= 0 ? 0 : (a0 + BT - 1) / BT;
      const int f1 = b0 < 0 ? 0 : b0 / BT + 1;
      flo = flo > f0 ? flo : f0;
      fhi = fhi < f1 ? fhi : f1;
    }
  }
  if (flo < lo) flo = lo;
  if (fhi > hi) fhi = hi;
  if (flo >= fhi) flo = fhi = hi;
  return Sweep{lo, hi, flo, fhi};
}

// f(integral_constant<0>), ..., f(integral_constant<N - 1>), in order.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (N > 0) {
    static_for<N - 1>(f);
    f(std::integral_constant<int, N - 1>{});
  }
}

// Stages of NSUB tiles from sw.lo: stages [0, f0) and [f1, n) hold a tile
// outside the fully-live run (or past the range), stages [f0, f1) only
// fully-live tiles.
struct Stages {
  int n, f0, f1;
};

template <int NSUB>
__device__ __forceinline__ Stages stage_plan(const Sweep& sw) {
  const int n = (sw.hi - sw.lo + NSUB - 1) / NSUB;
  int f0 = (sw.flo - sw.lo + NSUB - 1) / NSUB, f1 = (sw.fhi - sw.lo) / NSUB;
  if (f1 < f0) f1 = f0;
  return Stages{n, f0, f1};
}

// -------------------------------------------------------------------- dQ
//
// Workgroup: 4 waves x 32 query rows; key tiles of 32 rows (K, V) double
// buffered. Per wave and tile (lane: queries c, 16 + c; keys 4G + i, 16 + 4G + i):
//   S^T = K Q^T, dP^T = V dO^T (from -delta)   (A = K / V rows, B = Q / dO in registers)
//   dS^T = exp2(S^T c2 - lse2) dP^T
//   dQ^T += K^T dS^T                           (A = K transposed from LDS)

template <typename T, int D>
__device__ __forceinline__ void bwd16_dq(const BwdArgs& a, int bid, unsigned char* smem) {  // smem: K[2], V[2]
  using C = B16<D>;
  const int lane = threadIdx.x & 63, w = wave_id(), c = lane & 15, G = lane >> 4;
  const int64_t inst = bid / a.nqblk;
  const int qb = a.nqblk - 1 - (bid % a.nqblk);  // heavy (late) query blocks first
  const int64_t b = inst / a.heads, h = inst % a.heads, hkv = h / a.group;
  const uint16_t* qp = a.q + b * a.q_sb + h * a.q_sh;
  const uint16_t* kp = a.k + b * a.k_sb + hkv * a.k_sh;
  const uint16_t* vp = a.v + b * a.v_sb + hkv * a.v_sh;
  const uint16_t* dop = a.dout + b * a.o_sb + h * a.o_sh;
  const int T_ = static_cast<int>(a.t), S_ = static_cast<int>(a.s);
  const int q0 = qb * 128, qw0 = q0 + 32 * w;
  const int qr[2] = {qw0 + c, qw0 + 16 + c};
  const int cmg = c - 4 * G;

  u32x4 qreg[2][C::KS], doreg[2][C::KS];
  float ndl[2], lse2[2];
  {
    const uint32_t qoff = static_cast<uint32_t>(c * a.q_st * 2 + G * 16);
    const uint32_t ooff = static_cast<uint32_t>(c * a.o_st * 2 + G * 16);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const bool ok = qr[hh] < T_;
      const uint16_t* qbs = qp + static_cast<int64_t>(qw0 + 16 * hh) * a.q_st;
      const uint16_t* obs = dop + static_cast<int64_t>(qw0 + 16 * hh) * a.o_st;
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) {
        qreg[hh][ks] = ok ? gload<u32x4>(qbs + ks * 32, qoff) : u32x4{0u, 0u, 0u, 0u};
        doreg[hh][ks] = ok ? gload<u32x4>(obs + ks * 32, ooff) : u32x4{0u, 0u, 0u, 0u};
      }
      const int64_t srow = inst * a.t + qr[hh];
      ndl[hh] = ok ? a.ws[srow] : 0.f;  // -delta
      lse2[hh] = ok ? -a.ws[a.rows + srow] * a.c2 : 0.f;  // the stat is -lse / scale
    }
  }
  const Sweep sw = sweep_plan(a, q0, S_, true);

  const uint32_t grk = static_cast<uint32_t>(a.k_st * 2), grv = static_cast<uint32_t>(a.v_st * 2);
  const rsrc_t kr = make_rsrc(kp, static_cast<uint32_t>((a.s - 1) * a.k_st * 2 + D * 2));
  const rsrc_t vr = make_rsrc(vp, static_cast<uint32_t>((a.s - 1) * a.v_st * 2 + D * 2));
  uint32_t dk_off[C::NDMA], dv_off[C::NDMA];
  dma_offsets<D>(dk_off, lane, w, grk);
  dma_offsets<D>(dv_off, lane, w, grv);
  Lane16<D> L;
  L.init(lane);
  const int kt_lo = sw.lo, kt_hi = sw.hi;
  // K tiles [buf][sub] from 0, V tiles after them
  auto stage = [&](int st, int buf) {
#pragma unroll
    for (int j = 0; j < C::NSUB; ++j) {
      const int tile = kt_lo + st * C::NSUB + j;
      if (tile >= kt_hi) break;
      dma_tile<D>(kr, smem + (buf * C::NSUB + j) * C::TILEB, dk_off, static_cast<uint32_t>(tile * 32), grk, w);
      dma_tile<D>(vr, smem + ((2 + buf) * C::NSUB + j) * C::TILEB, dv_off, static_cast<uint32_t>(tile * 32), grv, w);
    }
  };

  f32x4 dqacc[C::FB][2];
#pragma unroll
  for (int fb = 0; fb < C::FB; ++fb) dqacc[fb][0] = dqacc[fb][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto tile = [&](auto slotc, int key0, auto cutc) {
    constexpr bool CUT = decltype(cutc)::value;
    constexpr int slot = decltype(slotc)::value;  // buf * NSUB + sub
    const unsigned char* kt = smem + slot * C::TILEB;
    const unsigned char* vt = smem + (2 * C::NSUB + slot) * C::TILEB;
    f32x4 sacc[2][2], pacc[2][2];  // [key half][query half]
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        sacc[kb][hh] = f32x4{0.f, 0.f, 0.f, 0.f};
        pacc[kb][hh] = f32x4{ndl[hh], ndl[hh], ndl[hh], ndl[hh]};
      }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int n = 0; n < 2 * C::KS; ++n) {
      const int ks = n >> 1, kb = n & 1;
      const u32x4 kk = L.row_frag(kt, kb, ks);
      const u32x4 vv = L.row_frag(vt, kb, ks);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        sacc[kb][hh] = mfma16<T>(kk, qreg[hh][ks], sacc[kb][hh]);
        pacc[kb][hh] = mfma16<T>(vv, doreg[hh][ks], pacc[kb][hh]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    u32x4 ds[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      float e[8];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          e[4 * kb + i] = fast_exp2(__builtin_fmaf(sacc[kb][hh][i], a.c2, -lse2[hh])) * pacc[kb][hh][i];
      if constexpr (CUT) {
        // live: key < s, query < t, lo <= key - query <= hi (32-bit: |key - query| < 2^29 + 64)
        // key - query = (key0 - qw0 - 16 hh) - (c - 4 G) + (16 kb + i): a scalar plus one lane constant
        // the scalar parts fenced in scalar registers before the lane constants
        // join them: no reassociated lane-dependent bounds kept live across the sweep
        int sd = key0 - qw0 - 16 * hh, sk = S_ - key0;
        asm volatile("" : "+s"(sd), "+s"(sk));
        int dl = sd - cmg;
        int kl = sk - 4 * G;  // key 16 kb + i of the tile exists below this
        asm volatile("" : "+v"(dl), "+v"(kl));
        const bool rowok = qw0 + 16 * hh + c < T_;
        // band_lo <= dl + cc <= band_hi, cc < kl, and a live query row
        int lo = a.masked ? a.band_lo32 - dl : 0, hi = kl - 1;
        if (a.masked && a.band_hi32 - dl < hi) hi = a.band_hi32 - dl;
        const CutWindow win = cut_window(rowok ? lo : 32, hi);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) e[4 * kb + i] = win.live(16 * kb + i) ? e[4 * kb + i] : 0.f;
      }
      ds[hh] = u32x4{pack2<T>(e[0], e[1]), pack2<T>(e[2], e[3]), pack2<T>(e[4], e[5]), pack2<T>(e[6], e[7])};
    }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int fb = 0; fb < C::FB; ++fb) {
      const u32x4 kf = L.tr_frag(kt, fb);
      dqacc[fb][0] = mfma16<T>(kf, ds[0], dqacc[fb][0]);
      dqacc[fb][1] = mfma16<T>(kf, ds[1], dqacc[fb][1]);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  const Stages sp = stage_plan<C::NSUB>(sw);
  if (sp.n > 0) stage(0, 0);
  // stage st lives in buffer st & 1; its tiles run with that buffer a
  // compile-time constant, so every LDS address is a lane offset plus an immediate
  auto one = [&](int st, auto bufc, auto cutc) {
    constexpr int buf = decltype(bufc)::value;
    wait_vmcnt0();
    __syncthreads();
    if (st + 1 < sp.n) stage(st + 1, buf ^ 1);
    static_for<C::NSUB>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      const int kt = kt_lo + st * C::NSUB + j;
      bool dead = decltype(cutc)::value && kt >= kt_hi;  // past the range (last stage only)
      const int key0 = kt * 32;
      if (decltype(cutc)::value && a.masked && a.prune) {  // this wave's rows see no live key here
        const int dmin = key0 - (qw0 + 31), dmax = key0 + 31 - qw0;
        dead = dead || dmin > a.band_hi32 || dmax < a.band_lo32;
      }
      if (!dead) tile(std::integral_constant<int, buf * C::NSUB + j>{}, key0, cutc);
    });
  };
  auto sweep = [&](int from, int to, auto cutc) {
    int st = from;
    if (st < to && (st & 1)) one(st++, std::integral_constant<int, 1>{}, cutc);
    for (; st + 1 < to; st += 2) {
      one(st, std::integral_constant<int, 0>{}, cutc);
      one(st + 1, std::integral_constant<int, 1>{}, cutc);
    }
    if (st < to) one(st, std::integral_constant<int, 0>{}, cutc);
  };
  sweep(0, sp.f0, std::true_type{});
  sweep(sp.f0, sp.f1, std::false_type{});
  sweep(sp.f1, sp.n, std::true_type{});
  wait_vmcnt0();

#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    if (qr[hh] >= T_) continue;
    uint16_t* base = a.dq + b * a.q_sb + h * a.q_sh + static_cast<int64_t>(qw0 + 16 * hh) * a.q_st;
    const uint32_t off = static_cast<uint32_t>(c * a.q_st * 2 + G * 8);
#pragma unroll
    for (int fb = 0; fb < C::FB; ++fb) {
      const f32x4 x = dqacc[fb][hh];
      gstore<u32x2>(base + 16 * fb, off,
                    u32x2{pack2<T>(x[0] * a.scale, x[1] * a.scale), pack2<T>(x[2] * a.scale, x[3] * a.scale)});
    }
  }
}

// ---------------------------------------------------------------- dK / dV
//
// Workgroup: 4 waves x 32 key rows (K, V in registers as B operands); query
// tiles of 32 rows (Q, dO and their rows' -delta / lse2 / pm) double
// buffered; grouped-query: the group's query heads one after another into
// the same accumulators. Per wave and tile (lane: keys c, 16 + c; queries
// 4G + i, 16 + 4G + i):
//   S = Q K^T, dP = dO V^T (from -delta)        (A = Q / dO rows from LDS)
//   P = exp2(S c2 - lse2), dS = P dP
//   dV^T += dO^T P, dK^T += Q^T dS               (A = dO / Q transposed from LDS)

template <typename T, int D>
__device__ __forceinline__ void bwd16_dkdv(const BwdArgs& a, int bid, unsigned char* smem) {  // Q[2], dO[2], stats[2]
  using C = B16<D>;
  constexpr int STATB = 4 * C::NSUB * C::TILEB;  // [2 * NSUB][-delta | -lse / scale | pm] x 32 floats
  const int lane = threadIdx.x & 63, w = wave_id(), c = lane & 15, G = lane >> 4;
  const int64_t kinst = bid / a.nkblk;
  const int kblk = bid % a.nkblk;  // early key blocks see the most queries under causal masks: launched first
  const int64_t b = kinst / a.heads_kv, hkv = kinst % a.heads_kv;
  const uint16_t* kp = a.k + b * a.k_sb + hkv * a.k_sh;
  const uint16_t* vp = a.v + b * a.v_sb + hkv * a.v_sh;
  const int T_ = static_cast<int>(a.t), S_ = static_cast<int>(a.s);
  const int k0 = kblk * 128, kw0 = k0 + 32 * w;
  const int cmg = c - 4 * G;

  u32x4 kreg[2][C::KS], vreg[2][C::KS];
  {
    const uint32_t koff = static_cast<uint32_t>(c * a.k_st * 2 + G * 16);
    const uint32_t voff = static_cast<uint32_t>(c * a.v_st * 2 + G * 16);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const bool ok = kw0 + 16 * hh + c < S_;
      const uint16_t* kbs = kp + static_cast<int64_t>(kw0 + 16 * hh) * a.k_st;
      const uint16_t* vbs = vp + static_cast<int64_t>(kw0 + 16 * hh) * a.v_st;
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks) {
        kreg[hh][ks] = ok ? gload<u32x4>(kbs + ks * 32, koff) : u32x4{0u, 0u, 0u, 0u};
        vreg[hh][ks] = ok ? gload<u32x4>(vbs + ks * 32, voff) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
  const Sweep sw = sweep_plan(a, k0, T_, false);
  const int nlive = sw.hi - sw.lo;

  const uint32_t grq = static_cast<uint32_t>(a.q_st * 2), gro = static_cast<uint32_t>(a.o_st * 2);
  uint32_t dq_off[C::NDMA], do_off[C::NDMA];
  dma_offsets<D>(dq_off, lane, w, grq);
  dma_offsets<D>(do_off, lane, w, gro);
  Lane16<D> L;
  L.init(lane);
  const rsrc_t sr = make_rsrc(a.ws, static_cast<uint32_t>(3 * a.rows * 4));
  // stats: wave 0 loads -delta (lanes 0-31) and lse2 (32-63), then pm (0-31)
  const uint32_t st_lane = static_cast<uint32_t>(((lane >> 5) * a.rows + (lane & 31)) * 4);
  const int64_t hq0 = hkv * a.group;  // the group's first query head
  // the staging cursor: (query head of the group, query tile), head-major
  const Stages sp = stage_plan<C::NSUB>(sw);
  // the staging cursor: (query head of the group, stage), head-major; Q tiles
  // [buf][sub] from 0, dO tiles after them, then the rows' statistics
  int s_gq = 0, s_st = 0;
  // the staged head's Q and dO (buffer descriptors) and its first statistics
  // row, advanced only when the cursor moves to the next head of the group:
  // the per-stage work is 32-bit offsets from these
  const uint32_t qbytes = static_cast<uint32_t>((a.t - 1) * a.q_st * 2 + D * 2);
  const uint32_t obytes = static_cast<uint32_t>((a.t - 1) * a.o_st * 2 + D * 2);
  const uint16_t* qh = a.q + b * a.q_sb + hq0 * a.q_sh;
  const uint16_t* oh = a.dout + b * a.o_sb + hq0 * a.o_sh;
  rsrc_t qr = make_rsrc(qh, qbytes), orr = make_rsrc(oh, obytes);
  uint32_t srow_h = static_cast<uint32_t>((b * a.heads + hq0) * a.t * 4);
  const uint32_t stat_plane = static_cast<uint32_t>(2 * a.rows * 4);
  auto stage = [&](int buf) {
#pragma unroll
    for (int j = 0; j < C::NSUB; ++j) {
      const int qt = sw.lo + s_st * C::NSUB + j;
      if (qt >= sw.hi) break;
      const int slot = buf * C::NSUB + j;
      dma_tile<D>(qr, smem + slot * C::TILEB, dq_off, static_cast<uint32_t>(qt * 32), grq, w);
      dma_tile<D>(orr, smem + (2 * C::NSUB + slot) * C::TILEB, do_off, static_cast<uint32_t>(qt * 32), gro, w);
      if (w == 0) {
        unsigned char* sl = smem + STATB + slot * 3 * 32 * 4;
        const uint32_t srow = srow_h + static_cast<uint32_t>(qt * 32 * 4);
        dma4(sr, sl, st_lane, srow);
        if (lane < 32) dma4(sr, sl + 2 * 32 * 4, st_lane, srow + stat_plane);
      }
    }
    if (++s_st == sp.n) {
      s_st = 0;
      if (++s_gq < a.group) {
        qh += a.q_sh;
        oh += a.o_sh;
        qr = make_rsrc(qh, qbytes);
        orr = make_rsrc(oh, obytes);
        srow_h += static_cast<uint32_t>(a.t * 4);
      }
    }
  };

  f32x4 dkacc[C::FB][2], dvacc[C::FB][2];
#pragma unroll
  for (int fb = 0; fb < C::FB; ++fb)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) dkacc[fb][hh] = dvacc[fb][hh] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto tile = [&](auto slotc, int q0, auto cutc) {
    constexpr bool CUT = decltype(cutc)::value;
    constexpr int slot = decltype(slotc)::value;  // buf * NSUB + sub
    const unsigned char* qt = smem + slot * C::TILEB;
    const unsigned char* ot = smem + (2 * C::NSUB + slot) * C::TILEB;
    const float* stl = reinterpret_cast<const float*>(smem + STATB + slot * 3 * 32 * 4);
    // S accumulates from -lse (score units) and dP from -delta, both per query
    // row, so the products leave S - lse and dP - delta
    f32x4 sacc[2][2], pacc[2][2];  // [query half][key half]
#pragma unroll
    for (int qh = 0; qh < 2; ++qh) {
      const f32x4 nd = *reinterpret_cast<const f32x4*>(stl + 16 * qh + 4 * G);  // -delta of queries 16 qh + 4 G + i
      const f32x4 nl = *reinterpret_cast<const f32x4*>(stl + 32 + 16 * qh + 4 * G);  // -lse / scale
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        sacc[qh][hh] = nl;
        pacc[qh][hh] = nd;
      }
    }
    // operands n = 2 ks + qh, read one step ahead of their four products
    u32x4 qq[2], oo[2];
    qq[0] = L.row_frag(qt, 0, 0);
    oo[0] = L.row_frag(ot, 0, 0);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int n = 0; n < 2 * C::KS; ++n) {
      const int ks = n >> 1, qh = n & 1;
      if (n + 1 < 2 * C::KS) {
        qq[(n + 1) & 1] = L.row_frag(qt, (n + 1) & 1, (n + 1) >> 1);
        oo[(n + 1) & 1] = L.row_frag(ot, (n + 1) & 1, (n + 1) >> 1);
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        sacc[qh][hh] = mfma16<T>(qq[n & 1], kreg[hh][ks], sacc[qh][hh]);
        pacc[qh][hh] = mfma16<T>(oo[n & 1], vreg[hh][ks], pacc[qh][hh]);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 p[2], ds[2];
    f32x4 pmv[2];  // a masked score's probability per query row: its row's pm if the row exists, else 0
    int sr = T_ - q0;
    if constexpr (CUT) asm volatile("" : "+s"(sr));  // per tile (as dl below)
    int rl = sr - 4 * G;  // query 16 qh + i of the tile exists below this
    if constexpr (CUT) asm volatile("" : "+v"(rl));
    if constexpr (CUT) {
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        pmv[qh] = *reinterpret_cast<const f32x4*>(stl + 64 + 16 * qh + 4 * G);
#pragma unroll
        for (int i = 0; i < 4; ++i) pmv[qh][i] = 16 * qh + i < rl ? pmv[qh][i] : 0.f;
      }
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      float e[8], g[8];
#pragma unroll
      for (int qh = 0; qh < 2; ++qh)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pr = fast_exp2(sacc[qh][hh][i] * a.c2);
          e[4 * qh + i] = pr;
          g[4 * qh + i] = pr * pacc[qh][hh][i];
        }
      if constexpr (CUT) {
        // live: query < t, lo <= key - query <= hi; a masked score's probability
        // is its row's pm (0 unless the row is fully masked) and carries no gradient
        // key - query = (kw0 + 16 hh - q0) + (c - 4 G) - (16 qh + i): a scalar plus one lane constant
        int sd = kw0 + 16 * hh - q0;
        asm volatile("" : "+s"(sd));
        int dl = sd + cmg;
        asm volatile("" : "+v"(dl));
        // band_lo <= dl - cc <= band_hi and cc < rl
        int lo = a.masked ? dl - a.band_hi32 : 0, hi = rl - 1;
        if (a.masked && dl - a.band_lo32 < hi) hi = dl - a.band_lo32;
        const CutWindow win = cut_window(lo, hi);
#pragma unroll
        for (int qh = 0; qh < 2; ++qh)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool live = win.live(16 * qh + i);
            e[4 * qh + i] = live ? e[4 * qh + i] : pmv[qh][i];
            g[4 * qh + i] = live ? g[4 * qh + i] : 0.f;
          }
      }
      p[hh] = u32x4{pack2<T>(e[0], e[1]), pack2<T>(e[2], e[3]), pack2<T>(e[4], e[5]), pack2<T>(e[6], e[7])};
      ds[hh] = u32x4{pack2<T>(g[0], g[1]), pack2<T>(g[2], g[3]), pack2<T>(g[4], g[5]), pack2<T>(g[6], g[7])};
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
    u32x4 of[2], qf[2];
    of[0] = L.tr_frag(ot, 0);
    qf[0] = L.tr_frag(qt, 0);
#pragma unroll
    for (int fb = 0; fb < C::FB; ++fb) {
      if (fb + 1 < C::FB) {
        of[(fb + 1) & 1] = L.tr_frag(ot, fb + 1);
        qf[(fb + 1) & 1] = L.tr_frag(qt, fb + 1);
      }
      dvacc[fb][0] = mfma16<T>(of[fb & 1], p[0], dvacc[fb][0]);
      dvacc[fb][1] = mfma16<T>(of[fb & 1], p[1], dvacc[fb][1]);
      dkacc[fb][0] = mfma16<T>(qf[fb & 1], ds[0], dkacc[fb][0]);
      dkacc[fb][1] = mfma16<T>(qf[fb & 1], ds[1], dkacc[fb][1]);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  // stage J = gq * sp.n + st lives in buffer J & 1; the staging cursor runs one stage ahead
  const int nst = nlive > 0 ? a.group * sp.n : 0;
  if (nst > 0) stage(0);
  auto one = [&](int J, int st, auto bufc, auto cutc) {
    constexpr int buf = decltype(bufc)::value;
    wait_vmcnt0();
    __syncthreads();
    if (J + 1 < nst) stage(buf ^ 1);
    static_for<C::NSUB>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      const int qt = sw.lo + st * C::NSUB + j;
      bool dead = decltype(cutc)::value && qt >= sw.hi;  // past the range (last stage only)
      const int q0 = qt * 32;
      if (decltype(cutc)::value && a.masked && a.prune) {  // this wave's keys see no live query here
        const int dmin = kw0 - (q0 + 31), dmax = kw0 + 31 - q0;
        dead = dead || dmin > a.band_hi32 || dmax < a.band_lo32;
      }
      if (!dead) tile(std::integral_constant<int, buf * C::NSUB + j>{}, q0, cutc);
    });
  };
  for (int gq = 0; gq < a.group && nlive > 0; ++gq) {
    const int J0 = gq * sp.n;  // stage st of this head: J0 + st
    auto sweep = [&](int from, int to, auto cutc) {
      int st = from;
      if (st < to && ((J0 + st) & 1)) {
        one(J0 + st, st, std::integral_constant<int, 1>{}, cutc);
        ++st;
      }
      for (; st + 1 < to; st += 2) {
        one(J0 + st, st, std::integral_constant<int, 0>{}, cutc);
        one(J0 + st + 1, st + 1, std::integral_constant<int, 1>{}, cutc);
      }
      if (st < to) one(J0 + st, st, std::integral_constant<int, 0>{}, cutc);
    };
    sweep(0, sp.f0, std::true_type{});
    sweep(sp.f0, sp.f1, std::false_type{});
    sweep(sp.f1, sp.n, std::true_type{});
  }
  wait_vmcnt0();

#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    if (kw0 + 16 * hh + c >= S_) continue;
    const uint32_t koff = static_cast<uint32_t>(c * a.k_st * 2 + G * 8);
    const uint32_t voff = static_cast<uint32_t>(c * a.v_st * 2 + G * 8);
    uint16_t* kbase = a.dk + b * a.k_sb + hkv * a.k_sh + static_cast<int64_t>(kw0 + 16 * hh) * a.k_st;
    uint16_t* vbase = a.dv + b * a.v_sb + hkv * a.v_sh + static_cast<int64_t>(kw0 + 16 * hh) * a.v_st;
#pragma unroll
    for (int fb = 0; fb < C::FB; ++fb) {
      const f32x4 x = dkacc[fb][hh], y = dvacc[fb][hh];
      gstore<u32x2>(kbase + 16 * fb, koff,
                    u32x2{pack2<T>(x[0] * a.scale, x[1] * a.scale), pack2<T>(x[2] * a.scale, x[3] * a.scale)});
      gstore<u32x2>(vbase + 16 * fb, voff, u32x2{pack2<T>(y[0], y[1]), pack2<T>(y[2], y[3])});
    }
  }
}

// dK/dV and dQ blocks share one launch (they depend only on the row
// statistics): logical blocks alternate between the two roles so the heavy
// causal blocks of both go first and each fills the other's tail.
template <typename T, int D>
__global__ __launch_bounds__(256, D == 64 ? 3 : 1) void bwd_main(BwdArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  int bid = blockIdx.x;
  int role, idx;
  if (a.xcd_remap == 2) {
    // Within an XCD (bid % 8) workgroups go in order round-robin to its four
    // shader engines (r % 4): four consecutive r take the same role and block
    // position of four instances, so every engine receives the same sequence
    // of workgroup lengths (the roles alternate, heavy blocks first) and
    // in-order dispatch never stalls on an engine that drew the heavier work.
    // Needs nkblk == nqblk and instances in multiples of 32.
    const int x = bid & 7, r = bid >> 3, s4 = r & 3, m4 = r >> 2;
    const int nb = a.nkblk, per_inst = 2 * nb;
    const int ipx = (gridDim.x >> 3) / per_inst;  // instances per XCD
    const int inst = x * ipx + (m4 / per_inst) * 4 + s4, step = m4 % per_inst;
    role = step & 1;
    idx = inst * nb + (step >> 1);
  } else {
    if (a.xcd_remap) {  // consecutive logical blocks (one instance's) share an XCD's L2
      const int per = gridDim.x >> 3;
      bid = (bid & 7) * per + (bid >> 3);
    }
    const int nk = a.ninst_kv * a.nkblk, nq = a.ninst * a.nqblk;
    const int both = 2 * (nk < nq ? nk : nq);
    if (bid < both) {
      role = bid & 1;
      idx = bid >> 1;
    } else {
      role = nk > nq ? 0 : 1;
      idx = both / 2 + (bid - both);
    }
  }
  // one call site per role: each role's code appears once in the kernel
  if (role == 0)
    bwd16_dkdv<T, D>(a, idx, smem);
  else
    bwd16_dq<T, D>(a, idx, smem);
}

// ---------------------------------------------------------------- fp32 column
//
// The fp32 backward (any e, od <= 512): the column the reference's f32 runner
// occupies for the backward carves (conformance/triton_tile.py). VALU only,
// one wave per row: bwd_rows_f32<0> owns a query row (dQ), <1> a key row
// (dK, dV); keys / queries in chunks of 64, one per lane. Row statistics come
// from the same workspace layout as the 16-bit path (-delta, lse2, pm).

struct GenBwdArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* o;
  const float* dout;
  const float* lse;
  const float* m_in;
  const float* den_in;
  float* dq;
  float* dk;
  float* dv;
  float* ws;
  int64_t rows, heads, t, s, e, od;  // heads: query heads
  int64_t heads_kv, group;           // query head h reads K / V head h / group
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
  float scale, c2, fill2;
  int masked;
  int64_t band_lo, band_hi;
  int prune;
};

constexpr int kGenPerLane = 8;  // e, od <= 512 held in registers

__global__ __launch_bounds__(256) void bwd_stats_f32(GenBwdArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int64_t inst = row / a.t, tq = row % a.t;
  const int64_t b = inst / a.heads, h = inst % a.heads;
  const float* orow = a.o + b * a.o_sb + h * a.o_sh + tq * a.o_st;
  const float* drow = a.dout + b * a.o_sb + h * a.o_sh + tq * a.o_st;
  float acc = 0.f;
  for (int64_t d = lane; d < a.od; d += 64) acc = __builtin_fmaf(orow[d], drow[d], acc);
  acc = wave_sum(acc);
  if (lane == 0) {
    float lse2, pm = 0.f;
    if (a.m_in != nullptr) {
      const float m2 = a.m_in[row] * kLog2e, den = a.den_in[row];
      lse2 = m2 + __log2f(den);
      if (a.masked) pm = fast_exp2(a.fill2 - m2) / den;
    } else {
      lse2 = a.lse[row] * kLog2e;
      if (a.masked) pm = (lse2 - a.fill2 < 64.f) ? 1.0f / static_cast<float>(a.s) : fast_exp2(a.fill2 - lse2);
    }
    a.ws[row] = -acc;  // -delta: the dP accumulators start from it
    a.ws[a.rows + row] = lse2;
    a.ws[2 * a.rows + row] = pm;
  }
}

// ROLE 0: wave per query row (dQ); ROLE 1: wave per key row (dK, dV).
template <int ROLE>
__global__ __launch_bounds__(256) void bwd_rows_f32(GenBwdArgs a, int64_t nrows) {
  const int lane = threadIdx.x & 63;
  const int64_t grow = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (grow >= nrows) return;
  const int64_t len = ROLE == 0 ? a.t : a.s;  // rows per instance of the owned side
  const int64_t inst = grow / len, r = grow % len;  // ROLE 0: a query instance; ROLE 1: a K / V instance
  const int64_t b = inst / (ROLE == 0 ? a.heads : a.heads_kv), hh = inst % (ROLE == 0 ? a.heads : a.heads_kv);
  const int64_t hkv = ROLE == 0 ? hh / a.group : hh;
  const float* kp = a.k + b * a.k_sb + hkv * a.k_sh;
  const float* vp = a.v + b * a.v_sb + hkv * a.v_sh;
  const int64_t other = ROLE == 0 ? a.s : a.t;  // the swept side
  // swept range: live pairs satisfy band_lo <= key - query <= band_hi
  int64_t lo = 0, hi = other;
  if (a.masked && a.prune) {
    if (ROLE == 0) {
      if (a.band_lo > INT64_MIN / 4) lo = r + a.band_lo > 0 ? r + a.band_lo : 0;
      if (a.band_hi < INT64_MAX / 4) hi = r + a.band_hi + 1 < other ? r + a.band_hi + 1 : other;
    } else {
      if (a.band_hi < INT64_MAX / 4) lo = r - a.band_hi > 0 ? r - a.band_hi : 0;
      if (a.band_lo > INT64_MIN / 4) hi = r - a.band_lo + 1 < other ? r - a.band_lo + 1 : other;
    }
    if (hi < lo) hi = lo;
  }
  float acc0[kGenPerLane], acc1[kGenPerLane];  // dq | dk, dv
#pragma unroll
  for (int j = 0; j < kGenPerLane; ++j) acc0[j] = acc1[j] = 0.f;
  // ROLE 0 sweeps its own query head; ROLE 1 every query head of its group in turn
  for (int64_t gq = 0; gq < (ROLE == 0 ? 1 : a.group); ++gq) {
    const int64_t hq = ROLE == 0 ? hh : hkv * a.group + gq, qinst = b * a.heads + hq;
    const float* qp = a.q + b * a.q_sb + hq * a.q_sh;
    const float* dop = a.dout + b * a.o_sb + hq * a.o_sh;
    const float* delp = a.ws + qinst * a.t;
    const float* lsep = a.ws + a.rows + qinst * a.t;
    const float* pmp = a.ws + 2 * a.rows + qinst * a.t;
    for (int64_t c0 = lo - (lo % 64); c0 < hi; c0 += 64) {
      const int64_t x = c0 + lane;  // this lane's key (ROLE 0) or query (ROLE 1)
      const int64_t tq = ROLE == 0 ? r : x, sk = ROLE == 0 ? x : r;
      float p = 0.f, ds = 0.f;
      if (x >= lo && x < hi) {
        const float* qr = qp + tq * a.q_st;
        const float* kr = kp + sk * a.k_st;
        const float* vr = vp + sk * a.v_st;
        const float* dr = dop + tq * a.o_st;
        float sc = 0.f, dp = 0.f;
        for (int64_t e = 0; e < a.e; ++e) sc = __builtin_fmaf(qr[e], kr[e], sc);
        for (int64_t o = 0; o < a.od; ++o) dp = __builtin_fmaf(dr[o], vr[o], dp);
        const int64_t d = sk - tq;
        if (a.masked && (d < a.band_lo || d > a.band_hi)) {
          p = pmp[tq];  // masked score: the row's masked-entry probability, no gradient
        } else {
          p = fast_exp2(__builtin_fmaf(sc, a.c2, -lsep[tq]));
          ds = p * (dp + delp[tq]);  // delp holds -delta
        }
      }
      const int64_t n = (hi - c0) < 64 ? (hi - c0) : 64;
      for (int kk = 0; kk < n; ++kk) {
        const float pk = __shfl(p, kk, 64), dk_ = __shfl(ds, kk, 64);
        const int64_t xx = c0 + kk;
        if (xx < lo) continue;
        if (ROLE == 0) {  // dq_r += ds_(r, key xx) k_xx
          const float* kr = kp + xx * a.k_st;
  #pragma unroll
          for (int j = 0; j < kGenPerLane; ++j) {
            const int64_t e = j * 64 + lane;
            if (e < a.e) acc0[j] = __builtin_fmaf(dk_, kr[e], acc0[j]);
          }
        } else {  // dk_r += ds_(query xx, r) q_xx ; dv_r += p_(xx, r) dO_xx
          const float* qr = qp + xx * a.q_st;
          const float* dr = dop + xx * a.o_st;
  #pragma unroll
          for (int j = 0; j < kGenPerLane; ++j) {
            const int64_t e = j * 64 + lane;
            if (e < a.e) acc0[j] = __builtin_fmaf(dk_, qr[e], acc0[j]);
            if (e < a.od) acc1[j] = __builtin_fmaf(pk, dr[e], acc1[j]);
          }
        }
      }
    }
  }  // query heads
  if (ROLE == 0) {
    float* out = a.dq + b * a.q_sb + hh * a.q_sh + r * a.q_st;
#pragma unroll
    for (int j = 0; j < kGenPerLane; ++j) {
      const int64_t e = j * 64 + lane;
      if (e < a.e) out[e] = acc0[j] * a.scale;
    }
  } else {
    float* ok = a.dk + b * a.k_sb + hkv * a.k_sh + r * a.k_st;
    float* ov = a.dv + b * a.v_sb + hkv * a.v_sh + r * a.v_st;
#pragma unroll
    for (int j = 0; j < kGenPerLane; ++j) {
      const int64_t e = j * 64 + lane;
      if (e < a.e) ok[e] = acc0[j] * a.scale;
      if (e < a.od) ov[e] = acc1[j];
    }
  }
}

bool band_has_empty_row(int64_t T, int64_t S, int64_t lo, int64_t hi) {
  if (lo > hi) return true;
  if (hi < 0) return true;
  if (lo > INT64_MIN / 4 && (T - 1) + lo > S - 1) return true;
  return false;
}

template <typename T, int D>
int launch_bwd(BwdArgs a, hipStream_t st) {
  constexpr int RPB = 4 * (64 / (D / 8));  // rows per stats workgroup
  bwd_stats<T, D><<<dim3(static_cast<unsigned>((a.rows + RPB - 1) / RPB)), 256, 0, st>>>(a);
  int rc = check_launch("pdh_flash_bwd (row stats)");
  if (rc) return rc;
  // the larger of the two roles' needs: dK/dV's Q, dO and row statistics, [2 buffers][NSUB] each
  constexpr int lds = 2 * B16<D>::NSUB * (2 * B16<D>::TILEB + 3 * 32 * 4);
  const int64_t nblk = static_cast<int64_t>(a.ninst_kv) * a.nkblk + static_cast<int64_t>(a.ninst) * a.nqblk;
  a.xcd_remap = nblk % 8 == 0 ? ((a.ninst % 32 == 0 && a.nkblk == a.nqblk && a.group == 1) ? 2 : 1) : 0;
  bwd_main<T, D><<<dim3(static_cast<unsigned>(nblk)), 256, lds, st>>>(a);
  return check_launch("pdh_flash_bwd (dk, dv, dq)");
}

}  // namespace
}  // namespace pdh

using namespace pdh;

extern "C" int pdh_flash_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout,
                             const float* lse, const float* m_in, const float* den_in, void* dq, void* dk,
                             void* dv, float* ws, const pdh_attn_geom* gm, int dtype, float scale, float fill, int mask_kind,
                             int64_t band_lo, int64_t band_hi, void* stream) {
  PDH_REQUIRE(gm != nullptr, PDH_EINVAL, "pdh_flash_bwd: null geometry");
  const pdh_attn_geom G = *gm;
  PDH_REQUIRE(G.batch >= 0 && G.heads_q >= 1 && G.heads_kv >= 1 && G.t >= 0 && G.s >= 1, PDH_EINVAL,
              "pdh_flash_bwd: bad shape");
  PDH_REQUIRE(G.heads_q % G.heads_kv == 0, PDH_EINVAL,
              "pdh_flash_bwd: heads_q (%lld) must be a multiple of heads_kv (%lld)", (long long)G.heads_q,
              (long long)G.heads_kv);
  const int64_t group = G.heads_q / G.heads_kv;
  PDH_REQUIRE(mask_kind == PDH_MASK_NONE || mask_kind == PDH_MASK_BAND, PDH_EINVAL,
              "pdh_flash_bwd: unknown mask kind %d", mask_kind);
  PDH_REQUIRE(q && k && v && o && dout && lse && dq && dk && dv && ws, PDH_EINVAL, "pdh_flash_bwd: null pointer");
  PDH_REQUIRE((m_in == nullptr) == (den_in == nullptr), PDH_EINVAL, "pdh_flash_bwd: pass both m and den, or neither");
  if (dtype == PDH_F32) {
    PDH_REQUIRE(G.e >= 1 && G.od >= 1 && G.e <= 64 * kGenPerLane && G.od <= 64 * kGenPerLane, PDH_EUNSUPPORTED,
                "pdh_flash_bwd: fp32 needs 1 <= e, od <= %d (got %lld, %lld)", 64 * kGenPerLane, (long long)G.e,
                (long long)G.od);
    const int64_t ninst = G.batch * G.heads_q, ninst_kv = G.batch * G.heads_kv;
    if (ninst == 0 || G.t == 0) return PDH_OK;
    PDH_REQUIRE((ninst * G.t + 3) / 4 <= INT32_MAX && (ninst_kv * G.s + 3) / 4 <= INT32_MAX, PDH_EINVAL,
                "pdh_flash_bwd: too many rows");
    const int masked = mask_kind == PDH_MASK_BAND;
    GenBwdArgs ga{static_cast<const float*>(q), static_cast<const float*>(k), static_cast<const float*>(v),
                  static_cast<const float*>(o), static_cast<const float*>(dout), lse, m_in, den_in,
                  static_cast<float*>(dq), static_cast<float*>(dk), static_cast<float*>(dv), ws, ninst * G.t,
                  G.heads_q, G.t, G.s, G.e, G.od, G.heads_kv, group, G.q_sb, G.q_sh, G.q_st, G.k_sb, G.k_sh, G.k_st,
                  G.v_sb, G.v_sh, G.v_st, G.o_sb, G.o_sh, G.o_st, scale, scale * kLog2e, fill * kLog2e, masked,
                  band_lo, band_hi, masked && !band_has_empty_row(G.t, G.s, band_lo, band_hi)};
    hipStream_t st = as_stream(stream);
    bwd_stats_f32<<<dim3(static_cast<unsigned>((ga.rows + 3) / 4)), 256, 0, st>>>(ga);
    int rc = check_launch("pdh_flash_bwd (fp32 row stats)");
    if (rc) return rc;
    bwd_rows_f32<0><<<dim3(static_cast<unsigned>((ninst * G.t + 3) / 4)), 256, 0, st>>>(ga, ninst * G.t);
    rc = check_launch("pdh_flash_bwd (fp32 dq)");
    if (rc) return rc;
    bwd_rows_f32<1><<<dim3(static_cast<unsigned>((ninst_kv * G.s + 3) / 4)), 256, 0, st>>>(ga, ninst_kv * G.s);
    return check_launch("pdh_flash_bwd (fp32 dk, dv)");
  }
  PDH_REQUIRE(dtype == PDH_BF16 || dtype == PDH_F16, PDH_EINVAL, "pdh_flash_bwd: unknown dtype %d", dtype);
  PDH_REQUIRE(G.e == G.od && (G.e == 64 || G.e == 128), PDH_EUNSUPPORTED,
              "pdh_flash_bwd: 16-bit kernels need e == od in {64, 128} (got %lld, %lld)", (long long)G.e,
              (long long)G.od);
  PDH_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o) && aligned16(dout) && aligned16(dq) &&
                  aligned16(dk) && aligned16(dv) && aligned16(lse),
              PDH_EINVAL, "pdh_flash_bwd: tensors must be 16-byte aligned");
  PDH_REQUIRE(G.q_st % 8 == 0 && G.k_st % 8 == 0 && G.v_st % 8 == 0 && G.o_st % 8 == 0 && G.q_sh % 8 == 0 &&
                  G.k_sh % 8 == 0 && G.v_sh % 8 == 0 && G.o_sh % 8 == 0 && G.q_sb % 8 == 0 && G.k_sb % 8 == 0 &&
                  G.v_sb % 8 == 0 && G.o_sb % 8 == 0,
              PDH_EINVAL, "pdh_flash_bwd: strides must be multiples of 8 elements");
  PDH_REQUIRE(G.q_st < (1 << 24) && G.k_st < (1 << 24) && G.v_st < (1 << 24) && G.o_st < (1 << 24), PDH_EINVAL,
              "pdh_flash_bwd: row strides must be < 2^24 elements");
  PDH_REQUIRE(G.t <= (1 << 29) && G.s <= (1 << 29), PDH_EINVAL, "pdh_flash_bwd: sequence too long (t, s <= 2^29)");
  PDH_REQUIRE(G.s * G.k_st * 2 < INT32_MAX && G.s * G.v_st * 2 < INT32_MAX && G.t * G.q_st * 2 < INT32_MAX &&
                  G.t * G.o_st * 2 < INT32_MAX,
              PDH_EINVAL, "pdh_flash_bwd: one instance's rows must span < 2 GiB");
  PDH_REQUIRE(G.batch * (G.heads_kv * ((G.s + 127) / 128) + G.heads_q * ((G.t + 127) / 128)) < INT32_MAX / 2,
              PDH_EINVAL, "pdh_flash_bwd: grid too large");
  PDH_REQUIRE(G.batch * G.heads_q * G.t * 12 < INT32_MAX, PDH_EINVAL,
              "pdh_flash_bwd: the row-statistics workspace must span < 2 GiB");
  const int64_t ninst = G.batch * G.heads_q;
  if (ninst == 0 || G.t == 0) return PDH_OK;
  const int masked = mask_kind == PDH_MASK_BAND;
  const int prune_ok = masked && !band_has_empty_row(G.t, G.s, band_lo, band_hi);
  BwdArgs a{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
            static_cast<const uint16_t*>(o), static_cast<const uint16_t*>(dout), lse, m_in, den_in,
            static_cast<uint16_t*>(dq), static_cast<uint16_t*>(dk), static_cast<uint16_t*>(dv), ws,
            ninst * G.t, G.heads_q, G.t, G.s, G.heads_kv, static_cast<int>(group), G.q_sb, G.q_sh, G.q_st, G.k_sb,
            G.k_sh, G.k_st, G.v_sb, G.v_sh, G.v_st, G.o_sb, G.o_sh, G.o_st, scale, scale * kLog2e, fill * kLog2e,
            masked, band_lo, band_hi, prune_ok, static_cast<int>(ninst), static_cast<int>(G.batch * G.heads_kv),
            static_cast<int>((G.s + 127) / 128), static_cast<int>((G.t + 127) / 128), 0};
  {
    constexpr int64_t kBand32 = (int64_t{1} << 29) + 64;
    auto clamp32 = [](int64_t x) { return static_cast<int>(x < -kBand32 ? -kBand32 : (x > kBand32 ? kBand32 : x)); };
    a.band_lo32 = clamp32(band_lo);
    a.band_hi32 = clamp32(band_hi);
  }
  hipStream_t st = as_stream(stream);
  if (dtype == PDH_BF16)
    return G.e == 128 ? launch_bwd<__hip_bfloat16, 128>(a, st) : launch_bwd<__hip_bfloat16, 64>(a, st);
  return G.e == 128 ? launch_bwd<_Float16, 128>(a, st) : launch_bwd<_Float16, 64>(a, st);
}
