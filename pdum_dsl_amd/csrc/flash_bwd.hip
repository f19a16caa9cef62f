// Flash-attention backward — the closed form of the flash joint's gradients
// (autodiff.grad over the naive twin, autodiff.py:102-122; the reference
// executes it as a carved plan of contraction kernels, partition.py:586-607).
// Like the reference's carving, every output is owned by exactly one program
// (330 §7.8 ruling 4): no atomics.
//
//   bwd_stats : per query row: -delta (delta = sum_d dO O), the log2-domain statistic
//               lse2 (P = exp2(x - lse2) for live scores) and pm, the
//               probability of a MASKED score (0 unless every key of the
//               row is masked; then 1/den, the uniform-softmax row)  (HBM-bound)
//   bwd_dkdv  : grid over 128-key blocks (4 waves x 32 keys); sweeps query
//               tiles; each wave keeps its K and V rows in registers and
//               accumulates dK^T, dV^T:
//                 S = Q K^T, dP = dO V^T          (A = Q / dO rows from LDS)
//                 P = exp(scale S - lse), dS = P (dP - delta)
//                 dV^T += dO^T P, dK^T += Q^T dS  (A = dO^T / Q^T from LDS)
//   bwd_dq    : grid over 128-query blocks; sweeps key tiles:
//                 S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T
//
// Grouped-query attention (heads_q = group x heads_kv, query head h reading
// K / V head h / group): a dK / dV workgroup sweeps the query tiles of every
// query head of its group in turn into the same accumulators, and a dQ
// workgroup reads its group's K and V. Every output still has one owner.
//
// All products are v_mfma_f32_32x32x16 (bf16 / f16 in, fp32 accumulate).
// LDS tiles whose rows become an MFMA A operand are stored with the
// kperm_inv row permutation, so the score accumulators feed the next
// contraction's k operand directly (see attn_common.h). Transposed copies
// (Q^T, dO^T, K^T) are formed in registers on the way into LDS.
// Masks: a masked score's probability is the row's pm (0 for any row with a
// live key) and carries no gradient (dS = 0), as the where() adjoint.
#include "attn_common.h"

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
    a.ws[a.rows + row] = lse2;
    a.ws[2 * a.rows + row] = pm;
  }
}

// Store a 32-row x D accumulator set held transposed (acc[db][i] is element
// (d = 32 db + 8(i/4) + 4g + i%4, row = r32)) to a row-major 16-bit output.
template <typename T, int D>
__device__ __forceinline__ void store_rows_t(uint16_t* base, int64_t ld, int r32, int g, const f32x16* acc,
                                             float mul) {
  const uint32_t off = static_cast<uint32_t>(r32 * ld * 2 + g * 8);
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4) {
      const int d0 = db * 32 + a4 * 8;
      const u32x2 wv = {pack2<T>(acc[db][4 * a4 + 0] * mul, acc[db][4 * a4 + 1] * mul),
                        pack2<T>(acc[db][4 * a4 + 2] * mul, acc[db][4 * a4 + 3] * mul)};
      gstore<u32x2>(base + d0, off, wv);
    }
  }
}

// A 32-row tile of a [rows, D] 16-bit operand in LDS: unpadded rows of D * 2
// bytes whose 16-byte slots are XOR-swizzled by swz_rt, filled by direct
// buffer loads (1 KB per wave instruction). The same tile is read as rows
// (b128, MFMA A operand) and transposed (ds_read_b64_tr_b16, MFMA A operand
// with the row index as k).
template <int D>
struct Tile32 {
  static constexpr int ROWB = D * 2, CPR = D / 8, BYTES = 32 * ROWB, RPK = 1024 / ROWB, NBLK = BYTES / 1024;
  static constexpr int KS = D / 16, DB = D / 32;
};

// Tiles staged per barrier: each stage holds kSub consecutive 32-row tiles,
// so a wave runs kSub tiles of MFMA / softmax work between barriers.
constexpr int kSub = 2;

// Per-lane offsets of the tile's three access patterns.
template <int D>
struct TileLane {
  using TT = Tile32<D>;
  uint32_t dma[(TT::NBLK + 3) / 4];  // direct-load offsets (4 waves share the blocks)
  int rowr[TT::KS];                 // row reads: row swap_bits23(r32), chunk 2 ks + g
  int tr[2][TT::DB];                // transposed reads, half h, feature block db (+ 16 s rows: immediate)

  __device__ __forceinline__ void init(int lane, int w, int r32, int g, uint32_t grb) {
    const int lrow = lane / TT::CPR, slot = lane % TT::CPR;
#pragma unroll
    for (int i = 0; i < (TT::NBLK + 3) / 4; ++i) {
      const int rho = (i * 4 + w) * TT::RPK + lrow;
      dma[i] = lrow * grb + ((slot ^ swz_rt<D>(rho)) << 4);
    }
    const int row = swap_bits23(r32);
#pragma unroll
    for (int ks = 0; ks < TT::KS; ++ks) rowr[ks] = row * TT::ROWB + (((2 * ks + g) ^ swz_rt<D>(row)) << 4);
    const int G = lane >> 4, kk = (lane >> 2) & 3, c4 = lane & 3;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int trow = 8 * (G >> 1) + 4 * h + kk;
#pragma unroll
      for (int db = 0; db < TT::DB; ++db)
        tr[h][db] = trow * TT::ROWB + (((4 * db + 2 * (G & 1) + (c4 >> 1)) ^ swz_rt<D>(trow)) << 4) + ((c4 & 1) << 3);
    }
  }
  // rows [row0, row0 + 32) of a buffer into an LDS tile (all 4 waves call this)
  __device__ __forceinline__ void stage(rsrc_t r, unsigned char* lds, uint32_t row0, uint32_t grb, int w) const {
#pragma unroll
    for (int i = 0; i < (TT::NBLK + 3) / 4; ++i) {
      const int blk = i * 4 + w;
      if (TT::NBLK % 4 != 0 && blk >= TT::NBLK) break;
      dma16(r, lds + blk * 1024, dma[i], (row0 + blk * TT::RPK) * grb);
    }
  }
  // MFMA A operand: 32 rows x 16 features (k-step ks) of the tile
  __device__ __forceinline__ u32x4 row_frag(const unsigned char* t, int ks) const {
    return *reinterpret_cast<const u32x4*>(t + rowr[ks]);
  }
  // MFMA A operand, transposed: features 32 db .. +32 x tile rows 16 s .. +16
  __device__ __forceinline__ u32x4 tr_frag(const unsigned char* t, int s, int db) const {
    const u32x2 lo = ds_read_tr16(t + 16 * s * TT::ROWB + tr[0][db]);
    const u32x2 hi = ds_read_tr16(t + 16 * s * TT::ROWB + tr[1][db]);
    return u32x4{lo.x, lo.y, hi.x, hi.y};
  }
};

// -------------------------------------------------------------------- dQ
//
// Workgroup: 4 waves x 32 query rows; key tiles of 32 rows (K, V) staged by
// direct loads kSub tiles per barrier, double buffered. Per wave and tile:
//   S^T = K Q^T, dP^T = V dO^T       (A = K / V rows, B = Q / dO in registers)
//   dS^T = P^T (dP^T - delta)        (lane = query row: lse, delta are scalars)
//   dQ^T += K^T dS^T                 (A = K transposed from LDS)

template <typename T, int D>
__device__ __forceinline__ void bwd_dq(const BwdArgs& a, int bid, unsigned char* smem) {  // smem: K[2], V[2]
  using TT = Tile32<D>;
  constexpr int KS = TT::KS, DB = TT::DB, BM = 128, BN = 32;
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id(), r32 = lane & 31, g = lane >> 5;
  const int64_t inst = bid / a.nqblk;
  const int qb = a.nqblk - 1 - (bid % a.nqblk);  // heavy (late) query blocks first
  const int64_t b = inst / a.heads, h = inst % a.heads, hkv = h / a.group;
  const uint16_t* qp = a.q + b * a.q_sb + h * a.q_sh;
  const uint16_t* kp = a.k + b * a.k_sb + hkv * a.k_sh;
  const uint16_t* vp = a.v + b * a.v_sb + hkv * a.v_sh;
  const uint16_t* dop = a.dout + b * a.o_sb + h * a.o_sh;
  const int64_t T_ = a.t, S_ = a.s;
  const int q0 = qb * BM;
  const int qw0 = q0 + 32 * w;
  const int qrow = qw0 + r32;

  u32x4 qreg[KS], doreg[KS];
  {
    const uint32_t qoff = static_cast<uint32_t>(r32 * a.q_st * 2 + g * 16);
    const uint32_t ooff = static_cast<uint32_t>(r32 * a.o_st * 2 + g * 16);
    const uint16_t* qbs = qp + static_cast<int64_t>(qw0) * a.q_st;
    const uint16_t* obs = dop + static_cast<int64_t>(qw0) * a.o_st;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qreg[ks] = qrow < T_ ? gload<u32x4>(qbs + ks * 16, qoff) : u32x4{0u, 0u, 0u, 0u};
      doreg[ks] = qrow < T_ ? gload<u32x4>(obs + ks * 16, ooff) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  const int64_t srow = inst * T_ + qrow;
  const float ndl = qrow < T_ ? a.ws[srow] : 0.f;  // -delta
  const float lse2 = qrow < T_ ? a.ws[a.rows + srow] : 0.f;

  const int ntiles = static_cast<int>((S_ + BN - 1) / BN);
  int kt_lo = 0, kt_hi = ntiles;
  if (a.masked && a.prune) {
    const int64_t qlast = (q0 + BM - 1 < T_ ? q0 + BM - 1 : T_ - 1);
    if (a.band_hi < INT64_MAX / 4) {
      const int64_t smax = qlast + a.band_hi;
      kt_hi = smax < 0 ? 0 : static_cast<int>(smax / BN + 1 < ntiles ? smax / BN + 1 : ntiles);
    }
    if (a.band_lo > INT64_MIN / 4) {
      const int64_t smin = q0 + a.band_lo;
      kt_lo = smin <= 0 ? 0 : static_cast<int>(smin / BN);
    }
  }

  const uint32_t grk = static_cast<uint32_t>(a.k_st * 2), grv = static_cast<uint32_t>(a.v_st * 2);
  const rsrc_t kr = make_rsrc(kp, static_cast<uint32_t>((S_ - 1) * a.k_st * 2 + D * 2));
  const rsrc_t vr = make_rsrc(vp, static_cast<uint32_t>((S_ - 1) * a.v_st * 2 + D * 2));
  TileLane<D> kl, vl;  // K and V tiles share the slot layout; only the source stride differs
  kl.init(lane, w, r32, g, grk);
  vl.init(lane, w, r32, g, grv);
  auto kbuf = [&](int buf, int sub) { return smem + (buf * kSub + sub) * TT::BYTES; };
  auto vbuf = [&](int buf, int sub) { return smem + ((2 + buf) * kSub + sub) * TT::BYTES; };
  auto stage = [&](int tile0, int buf) {  // tiles tile0 .. tile0 + kSub - 1 that the sweep reads
#pragma unroll
    for (int sub = 0; sub < kSub; ++sub) {
      if (tile0 + sub >= kt_hi) break;
      kl.stage(kr, kbuf(buf, sub), static_cast<uint32_t>((tile0 + sub) * BN), grk, w);
      vl.stage(vr, vbuf(buf, sub), static_cast<uint32_t>((tile0 + sub) * BN), grv, w);
    }
  };

  f32x16 dqacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) dqacc[db] = f32x16{};

  if (kt_lo < kt_hi) stage(kt_lo, 0);
  for (int kt0 = kt_lo; kt0 < kt_hi; kt0 += kSub) {
    const int buf = ((kt0 - kt_lo) / kSub) & 1;
    wait_vmcnt0();
    __syncthreads();
    if (kt0 + kSub < kt_hi) stage(kt0 + kSub, buf ^ 1);  // the next stage, into the idle buffers
#pragma unroll
    for (int sub = 0; sub < kSub; ++sub) {
      const int kt = kt0 + sub;
      if (kt >= kt_hi) break;
      const int64_t key0 = static_cast<int64_t>(kt) * BN;
      const int64_t dmin = key0 - (qw0 + 31), dmax = key0 + BN - 1 - qw0;
      bool dead = false, cut = key0 + BN > S_ || qw0 + 32 > T_;
      if (a.masked) {
        dead = a.prune && (dmin > a.band_hi || dmax < a.band_lo);
        cut = cut || dmin < a.band_lo || dmax > a.band_hi;
      }
      if (dead) continue;
      const unsigned char* kt_l = kbuf(buf, sub);
      const unsigned char* vt_l = vbuf(buf, sub);
      __builtin_amdgcn_s_setprio(1);
      f32x16 sacc = f32x16{};
      f32x16 pacc = ndl - f32x16{};  // dP^T - delta accumulates from -delta
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        sacc = mfma32<T>(kl.row_frag(kt_l, ks), qreg[ks], sacc);
        pacc = mfma32<T>(vl.row_frag(vt_l, ks), doreg[ks], pacc);
      }
      __builtin_amdgcn_s_setprio(0);
      // accumulator i of lane-half g: key key0 + 16 (i / 8) + 8 g + i % 8, query qrow
      if (cut) {
        const int64_t kl0 = key0 + 8 * g;
        const int rem = static_cast<int>(S_ - kl0 < 1024 ? S_ - kl0 : 1024);
        const int64_t dl0 = kl0 - qrow;
        auto clampi = [](int64_t x) { return static_cast<int>(x < -4096 ? -4096 : (x > 4096 ? 4096 : x)); };
        // an unbounded end (INT64_MIN / INT64_MAX) must not enter the subtraction: it would wrap
        const int lo = (a.masked && a.band_lo > INT64_MIN / 4) ? clampi(a.band_lo - dl0) : -4096;
        const int hi = (a.masked && a.band_hi < INT64_MAX / 4) ? clampi(a.band_hi - dl0) : 4096;
        const bool rowok = qrow < T_;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int c = (i >> 3) * 16 + (i & 7);
          const bool live = rowok && c < rem && c >= lo && c <= hi;
          pacc[i] = live ? fast_exp2(__builtin_fmaf(sacc[i], a.c2, -lse2)) * pacc[i] : 0.f;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) pacc[i] = fast_exp2(__builtin_fmaf(sacc[i], a.c2, -lse2)) * pacc[i];
      }
      const u32x4 ds0 = pack8<T>(pacc, 0), ds1 = pack8<T>(pacc, 1);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        dqacc[db] = mfma32<T>(kl.tr_frag(kt_l, 0, db), ds0, dqacc[db]);
        dqacc[db] = mfma32<T>(kl.tr_frag(kt_l, 1, db), ds1, dqacc[db]);
      }
      __builtin_amdgcn_s_setprio(0);
    }
  }
  wait_vmcnt0();

  if (qrow < T_)
    store_rows_t<T, D>(a.dq + b * a.q_sb + h * a.q_sh + static_cast<int64_t>(qw0) * a.q_st, a.q_st, r32, g, dqacc,
                       a.scale);
}

// ---------------------------------------------------------------- dK / dV
//
// Workgroup: 4 waves x 32 key rows (K, V in registers as B operands); query
// tiles of 32 rows (Q, dO and the rows' delta / lse2 / pm) staged by direct
// loads kSub tiles per barrier, double buffered. Per wave and tile:
//   S = Q K^T, dP = dO V^T           (A = Q / dO rows; lane = key, acc = query)
//   P = exp2(S c2 - lse2), dS = P (dP - delta)
//   dV^T += dO^T P, dK^T += Q^T dS   (A = dO / Q transposed from LDS)

template <typename T, int D>
__device__ __forceinline__ void bwd_dkdv(const BwdArgs& a, int bid, unsigned char* smem) {  // Q[2], dO[2], stats[2]
  using TT = Tile32<D>;
  constexpr int KS = TT::KS, DB = TT::DB, BK = 128, QT = 32;
  constexpr int STATB = 4 * kSub * TT::BYTES;  // [2][kSub][delta | lse2 | pm] x 32 floats
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id(), r32 = lane & 31, g = lane >> 5;
  const int64_t kinst = bid / a.nkblk;  // K / V instance
  const int kblk = bid % a.nkblk;  // early key blocks see the most queries under causal masks: launched first
  const int64_t b = kinst / a.heads_kv, hkv = kinst % a.heads_kv;
  const uint16_t* kp = a.k + b * a.k_sb + hkv * a.k_sh;
  const uint16_t* vp = a.v + b * a.v_sb + hkv * a.v_sh;
  const int64_t T_ = a.t, S_ = a.s;
  const int k0 = kblk * BK;
  const int kw0 = k0 + 32 * w;
  const int krow = kw0 + r32;
  auto clamp30 = [](int64_t x) { return static_cast<int>(x < -(1 << 30) ? -(1 << 30) : (x > (1 << 30) ? (1 << 30) : x)); };
  const int blo = a.masked ? clamp30(a.band_lo) : -(1 << 30);
  const int bhi = a.masked ? clamp30(a.band_hi) : (1 << 30);

  // this wave's K and V rows as B operands (lane: row r32, features 16 ks + 8 g .. +8)
  u32x4 kreg[KS], vreg[KS];
  {
    const uint32_t koff = static_cast<uint32_t>(r32 * a.k_st * 2 + g * 16);
    const uint32_t voff = static_cast<uint32_t>(r32 * a.v_st * 2 + g * 16);
    const uint16_t* kbs = kp + static_cast<int64_t>(kw0) * a.k_st;
    const uint16_t* vbs = vp + static_cast<int64_t>(kw0) * a.v_st;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kreg[ks] = krow < S_ ? gload<u32x4>(kbs + ks * 16, koff) : u32x4{0u, 0u, 0u, 0u};
      vreg[ks] = krow < S_ ? gload<u32x4>(vbs + ks * 16, voff) : u32x4{0u, 0u, 0u, 0u};
    }
  }

  const int nqt = static_cast<int>((T_ + QT - 1) / QT);
  int qt_lo = 0, qt_hi = nqt;
  if (a.masked && a.prune) {
    const int64_t klast = (k0 + BK - 1 < S_ ? k0 + BK - 1 : S_ - 1);
    if (a.band_hi < INT64_MAX / 4) {  // q >= key - hi
      const int64_t qmin = k0 - a.band_hi;
      qt_lo = qmin <= 0 ? 0 : static_cast<int>(qmin / QT < nqt ? qmin / QT : nqt);
    }
    if (a.band_lo > INT64_MIN / 4) {  // q <= key - lo
      const int64_t qmax = klast - a.band_lo;
      qt_hi = qmax < 0 ? 0 : static_cast<int>(qmax / QT + 1 < nqt ? qmax / QT + 1 : nqt);
    }
  }

  const uint32_t grq = static_cast<uint32_t>(a.q_st * 2), gro = static_cast<uint32_t>(a.o_st * 2);
  const rsrc_t sr = make_rsrc(a.ws, static_cast<uint32_t>(3 * a.rows * 4));
  TileLane<D> ql, ol;
  ql.init(lane, w, r32, g, grq);
  ol.init(lane, w, r32, g, gro);
  // The sweep runs over (query head of the group, query tile) items, head-major,
  // with two cursors kept by increments (no divisions): one staging a stage
  // ahead, one computing.
  struct Cursor {
    int gq, qt;
  };
  const int nqt_live = qt_hi - qt_lo;
  auto advance = [&](Cursor& c) {
    if (++c.qt == qt_hi) {
      c.qt = qt_lo;
      ++c.gq;
    }
  };
  // stats: wave 0 loads delta (lanes 0-31) and lse2 (32-63), then pm (0-31)
  const uint32_t st_lane0 = static_cast<uint32_t>(((lane >> 5) * a.rows + r32) * 4);
  const uint32_t st_lane1 = static_cast<uint32_t>((2 * a.rows + r32) * 4);
  const int64_t hq0 = hkv * a.group;  // the group's first query head
  auto qbuf = [&](int buf, int sub) { return smem + (buf * kSub + sub) * TT::BYTES; };
  auto obuf = [&](int buf, int sub) { return smem + ((2 + buf) * kSub + sub) * TT::BYTES; };
  auto sbuf = [&](int buf, int sub) {
    return reinterpret_cast<float*>(smem + STATB + (buf * kSub + sub) * 3 * QT * 4);
  };
  Cursor sc{0, qt_lo};  // the next item to stage
  auto stage = [&](int buf) {  // the next kSub items, into buffer buf
#pragma unroll
    for (int sub = 0; sub < kSub; ++sub) {
      if (sc.gq >= a.group) break;
      const int64_t hq = hq0 + sc.gq;
      const rsrc_t qr = make_rsrc(a.q + b * a.q_sb + hq * a.q_sh, static_cast<uint32_t>((T_ - 1) * a.q_st * 2 + D * 2));
      const rsrc_t orr =
          make_rsrc(a.dout + b * a.o_sb + hq * a.o_sh, static_cast<uint32_t>((T_ - 1) * a.o_st * 2 + D * 2));
      ql.stage(qr, qbuf(buf, sub), static_cast<uint32_t>(sc.qt * QT), grq, w);
      ol.stage(orr, obuf(buf, sub), static_cast<uint32_t>(sc.qt * QT), gro, w);
      if (w == 0) {
        unsigned char* sl = reinterpret_cast<unsigned char*>(sbuf(buf, sub));
        const uint32_t srow = static_cast<uint32_t>(((b * a.heads + hq) * T_ + sc.qt * QT) * 4);
        dma4(sr, sl, st_lane0, srow);
        if (lane < 32) dma4(sr, sl + 2 * QT * 4, st_lane1, srow);
      }
      advance(sc);
    }
  };

  f32x16 dkacc[DB], dvacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dkacc[db] = f32x16{};
    dvacc[db] = f32x16{};
  }

  Cursor cc{0, qt_lo};  // the next item to compute
  if (nqt_live > 0) stage(0);
  for (int buf = 0; nqt_live > 0 && cc.gq < a.group; buf ^= 1) {
    wait_vmcnt0();
    __syncthreads();
    if (sc.gq < a.group) stage(buf ^ 1);  // the next stage, into the idle buffers
#pragma unroll
    for (int sub = 0; sub < kSub; ++sub) {
      if (cc.gq >= a.group) break;
      const int qt = cc.qt;
      advance(cc);
      const int64_t q0 = static_cast<int64_t>(qt) * QT;
      const int64_t dmin = kw0 - (q0 + QT - 1), dmax = kw0 + 31 - q0;  // key - q over the tile
      bool dead = false, cut = q0 + QT > T_ || kw0 + 32 > S_;
      if (a.masked) {
        dead = a.prune && (dmin > a.band_hi || dmax < a.band_lo);
        cut = cut || dmin < a.band_lo || dmax > a.band_hi;
      }
      if (dead) continue;
      const unsigned char* q_l = qbuf(buf, sub);
      const unsigned char* o_l = obuf(buf, sub);
      const float* stl = sbuf(buf, sub);
      // accumulator i of lane-half g: query q0 + 16 (i / 8) + 8 g + i % 8, key krow.
      // dP - delta accumulates from the rows' -delta (the MFMA adds it).
      f32x16 sacc = f32x16{}, pacc;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int rb = 16 * hh + 8 * g;
        const f32x4 d0 = *reinterpret_cast<const f32x4*>(stl + rb);  // -delta
        const f32x4 d1 = *reinterpret_cast<const f32x4*>(stl + rb + 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) pacc[8 * hh + j] = j < 4 ? d0[j] : d1[j - 4];
      }
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        sacc = mfma32<T>(ql.row_frag(q_l, ks), kreg[ks], sacc);
        pacc = mfma32<T>(ol.row_frag(o_l, ks), vreg[ks], pacc);
      }
      __builtin_amdgcn_s_setprio(0);
      // masks in 32-bit offsets from the tile (band limits clamped to +-2^30)
      const int dk0 = static_cast<int>(krow - q0);
      const int qlim = krow < S_ ? static_cast<int>(T_ - q0 < (1 << 30) ? T_ - q0 : (1 << 30)) : 0;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int rb = 16 * hh + 8 * g;
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(stl + QT + rb);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(stl + QT + rb + 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int i = 8 * hh + j;
          const float lv = j < 4 ? l0[j] : l1[j - 4];
          const float p = fast_exp2(__builtin_fmaf(sacc[i], a.c2, -lv));
          pacc[i] = p * pacc[i];
          sacc[i] = p;
        }
      }
      // Masked tiles (uniform branch) fix up the probabilities with selects that
      // read the rows' pm values as vectors: no per-element branches, which
      // would split the tile into basic blocks the scheduler cannot interleave
      // with the MFMAs.
      if (cut) {
        asm volatile("" ::: "memory");  // keeps the branch: if-converted, every tile would pay the selects
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int rb = 16 * hh + 8 * g;
          const f32x4 m0 = *reinterpret_cast<const f32x4*>(stl + 2 * QT + rb);
          const f32x4 m1 = *reinterpret_cast<const f32x4*>(stl + 2 * QT + rb + 4);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int i = 8 * hh + j;
            const float pm = j < 4 ? m0[j] : m1[j - 4];  // the row's masked-score probability (0 unless fully masked)
            const int dd = dk0 - rb - j;                  // key - query
            const bool row_live = rb + j < qlim;
            const bool in_band = dd >= blo && dd <= bhi;
            sacc[i] = row_live ? (in_band ? sacc[i] : pm) : 0.f;
            pacc[i] = row_live && in_band ? pacc[i] : 0.f;
          }
        }
      }
      const u32x4 p0 = pack8<T>(sacc, 0), p1 = pack8<T>(sacc, 1);
      const u32x4 s0 = pack8<T>(pacc, 0), s1 = pack8<T>(pacc, 1);
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        dvacc[db] = mfma32<T>(ol.tr_frag(o_l, 0, db), p0, dvacc[db]);
        dvacc[db] = mfma32<T>(ol.tr_frag(o_l, 1, db), p1, dvacc[db]);
        dkacc[db] = mfma32<T>(ql.tr_frag(q_l, 0, db), s0, dkacc[db]);
        dkacc[db] = mfma32<T>(ql.tr_frag(q_l, 1, db), s1, dkacc[db]);
      }
      __builtin_amdgcn_s_setprio(0);
    }
  }
  wait_vmcnt0();

  if (krow < S_) {
    store_rows_t<T, D>(a.dk + b * a.k_sb + hkv * a.k_sh + static_cast<int64_t>(kw0) * a.k_st, a.k_st, r32, g, dkacc,
                       a.scale);
    store_rows_t<T, D>(a.dv + b * a.v_sb + hkv * a.v_sh + static_cast<int64_t>(kw0) * a.v_st, a.v_st, r32, g, dvacc,
                       1.0f);
  }
}

// dK/dV and dQ blocks share one launch (they depend only on the row
// statistics): logical blocks alternate between the two roles so the heavy
// causal blocks of both go first and each fills the other's tail.
template <typename T, int D>
__global__ __launch_bounds__(256, D == 64 ? 3 : 1) void bwd_main(BwdArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  int bid = blockIdx.x;
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
    if ((step & 1) == 0)
      bwd_dkdv<T, D>(a, inst * nb + (step >> 1), smem);
    else
      bwd_dq<T, D>(a, inst * nb + (step >> 1), smem);
    return;
  }
  if (a.xcd_remap) {  // consecutive logical blocks (one instance's) share an XCD's L2
    const int per = gridDim.x >> 3;
    bid = (bid & 7) * per + (bid >> 3);
  }
  const int nk = a.ninst_kv * a.nkblk, nq = a.ninst * a.nqblk;
  const int both = 2 * (nk < nq ? nk : nq);
  int role, idx;
  if (bid < both) {
    role = bid & 1;
    idx = bid >> 1;
  } else {
    role = nk > nq ? 0 : 1;
    idx = both / 2 + (bid - both);
  }
  if (role == 0)
    bwd_dkdv<T, D>(a, idx, smem);
  else
    bwd_dq<T, D>(a, idx, smem);
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
  constexpr int TB = Tile32<D>::BYTES;
  constexpr int lds = 4 * kSub * TB + 2 * kSub * 3 * 32 * 4;  // the larger of the two roles' needs (dK/dV)
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
  PDH_REQUIRE(G.t <= INT32_MAX / 2 && G.s <= INT32_MAX / 2, PDH_EINVAL, "pdh_flash_bwd: sequence too long");
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
  hipStream_t st = as_stream(stream);
  if (dtype == PDH_BF16)
    return G.e == 128 ? launch_bwd<__hip_bfloat16, 128>(a, st) : launch_bwd<__hip_bfloat16, 64>(a, st);
  return G.e == 128 ? launch_bwd<_Float16, 128>(a, st) : launch_bwd<_Float16, 64>(a, st);
}
