// Flash-attention backward — the closed form of the flash joint's gradients
// (autodiff.grad over the naive twin, autodiff.py:102-122; the reference
// executes it as a carved plan of contraction kernels, partition.py:586-607).
// Like the reference's carving, every output is owned by exactly one program
// (330 §7.8 ruling 4): no atomics.
//
//   bwd_stats : per query row: delta = sum_d dO O, the log2-domain statistic
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
  float* ws;            // [3][rows]: delta, lse2, pm
  int64_t rows;         // batch * heads * t
  int64_t heads, t, s;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
  float scale, c2, fill2;
  int masked;
  int64_t band_lo, band_hi;
  int prune;
  int nblk;  // blocks per instance (query blocks for dq, key blocks for dkdv)
};

// ---------------------------------------------------------------- row stats

template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_stats(BwdArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int64_t inst = row / a.t, tq = row % a.t;
  const int64_t b = inst / a.heads, h = inst % a.heads;
  const uint16_t* orow = a.o + b * a.o_sb + h * a.o_sh + tq * a.o_st;
  const uint16_t* drow = a.dout + b * a.o_sb + h * a.o_sh + tq * a.o_st;
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < D / 64; ++j)
    acc += Elem<T>::to_f32(orow[j * 64 + lane]) * Elem<T>::to_f32(drow[j * 64 + lane]);
  acc = wave_sum(acc);
  if (lane == 0) {
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
    a.ws[row] = acc;
    a.ws[a.rows + row] = lse2;
    a.ws[2 * a.rows + row] = pm;
  }
}

// ---------------------------------------------------------- tile staging

// A ROWS x D tile of 16-bit elements in registers: thread (rgrp, dgrp) holds
// rows [8 rgrp, 8 rgrp + 8) x features [DG dgrp, DG dgrp + DG).
template <int ROWS, int D>
struct TileT {
  static constexpr int DG = ROWS * D / 2048;
  static constexpr int NDG = D / DG;
  static_assert(DG == 2 || DG == 4, "tile shape");
  uint32_t r[8][DG / 2];
};

template <int ROWS, int D>
__device__ __forceinline__ void tload(TileT<ROWS, D>& t, const uint16_t* base, int64_t ld, int64_t nvalid,
                                      int tid) {
  constexpr int DG = TileT<ROWS, D>::DG, NDG = TileT<ROWS, D>::NDG;
  // Rows past nvalid (>= 1) re-read the last valid row and are zeroed by a
  // select: no divergent branches around the loads.
  const int dgrp = tid % NDG, rgrp = tid / NDG;
  const int last = static_cast<int>(nvalid < ROWS ? nvalid - 1 : ROWS - 1);
#pragma unroll
  for (int rr = 0; rr < 8; ++rr) {
    const int row = rgrp * 8 + rr;
    const bool ok = row <= last;
    const uint32_t off = static_cast<uint32_t>((ok ? row : last) * ld * 2 + dgrp * DG * 2);
    if constexpr (DG == 4) {
      const u32x2 x = gload<u32x2>(base, off);
      t.r[rr][0] = ok ? x.x : 0u;
      t.r[rr][1] = ok ? x.y : 0u;
    } else {
      const uint32_t x = gload<uint32_t>(base, off);
      t.r[rr][0] = ok ? x : 0u;
    }
  }
}

// Row-major copy, rows permuted by kperm_inv within each 32-row block.
template <int ROWS, int D>
__device__ __forceinline__ void tstore_rows(const TileT<ROWS, D>& t, unsigned char* lds, int rs, int tid) {
  constexpr int DG = TileT<ROWS, D>::DG, NDG = TileT<ROWS, D>::NDG;
  const int dgrp = tid % NDG, rgrp = tid / NDG;
#pragma unroll
  for (int rr = 0; rr < 8; ++rr) {
    const int row = rgrp * 8 + rr;
    unsigned char* dst = lds + ((row & ~31) + kperm_inv(row & 31)) * rs + dgrp * DG * 2;
    if constexpr (DG == 4)
      *reinterpret_cast<u32x2*>(dst) = u32x2{t.r[rr][0], t.r[rr][1]};
    else
      *reinterpret_cast<uint32_t*>(dst) = t.r[rr][0];
  }
}

// Transposed copy: LDS row d holds the tile's column d (ROWS elements).
template <int ROWS, int D>
__device__ __forceinline__ void tstore_trans(const TileT<ROWS, D>& t, unsigned char* lds, int ts, int tid) {
  constexpr int DG = TileT<ROWS, D>::DG, NDG = TileT<ROWS, D>::NDG;
  const int dgrp = tid % NDG, rgrp = tid / NDG;
#pragma unroll
  for (int d = 0; d < DG; ++d) {
    const uint32_t sel = (d & 1) ? 0x07060302u : 0x05040100u;
    const int c = d >> 1;
    const u32x4 w = {perm_halves(t.r[1][c], t.r[0][c], sel), perm_halves(t.r[3][c], t.r[2][c], sel),
                     perm_halves(t.r[5][c], t.r[4][c], sel), perm_halves(t.r[7][c], t.r[6][c], sel)};
    *reinterpret_cast<u32x4*>(lds + (dgrp * DG + d) * ts + rgrp * 16) = w;
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

// ---------------------------------------------------------------- dK / dV

template <int D>
struct DkdvCfg {
  static constexpr int KB = 128;               // keys per workgroup
  static constexpr int QT = D == 64 ? 64 : 32;  // query rows per tile
  static constexpr int RS = D * 2 + 16;        // row-major row stride (bytes)
  static constexpr int TS = QT * 2 + 16;       // transposed row stride
  static constexpr int QR = QT * RS;
  static constexpr int QTR = D * TS;
  static constexpr int OFF_QT = QR, OFF_DO = QR + QTR, OFF_DOT = 2 * QR + QTR, OFF_LSE = 2 * QR + 2 * QTR;
  static constexpr int OFF_DEL = OFF_LSE + QT * 4;
  static constexpr int OFF_PM = OFF_DEL + QT * 4;
  static constexpr int STAGE = OFF_PM + QT * 4;
  static constexpr int LDS = 2 * STAGE;
};

template <typename T, int D>
__global__ __launch_bounds__(256, 1) void bwd_dkdv(BwdArgs a) {
  using C = DkdvCfg<D>;
  constexpr int QT = C::QT, NQB = QT / 32;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id(), r32 = lane & 31, g = lane >> 5;
  const int64_t inst = blockIdx.x / a.nblk;
  const int kblk = blockIdx.x % a.nblk;  // early key blocks see the most queries: launched first
  const int64_t b = inst / a.heads, h = inst % a.heads;
  const uint16_t* qp = a.q + b * a.q_sb + h * a.q_sh;
  const uint16_t* kp = a.k + b * a.k_sb + h * a.k_sh;
  const uint16_t* vp = a.v + b * a.v_sb + h * a.v_sh;
  const uint16_t* dop = a.dout + b * a.o_sb + h * a.o_sh;
  const float* delp = a.ws + inst * a.t;
  const float* lsep = a.ws + a.rows + inst * a.t;
  const float* pmp = a.ws + 2 * a.rows + inst * a.t;
  const int64_t T_ = a.t, S_ = a.s;
  const int k0 = kblk * C::KB;
  const int kw0 = k0 + 32 * w;
  const int krow = kw0 + r32;

  // this wave's K and V rows as B operands (lane: row r32, features 16 ks + 8 g .. +8)
  u32x4 kreg[D / 16], vreg[D / 16];
  {
    const uint32_t koff = static_cast<uint32_t>(r32 * a.k_st * 2 + g * 16);
    const uint32_t voff = static_cast<uint32_t>(r32 * a.v_st * 2 + g * 16);
    const uint16_t* kb = kp + static_cast<int64_t>(kw0) * a.k_st;
    const uint16_t* vb = vp + static_cast<int64_t>(kw0) * a.v_st;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      kreg[ks] = krow < S_ ? gload<u32x4>(kb + ks * 16, koff) : u32x4{0u, 0u, 0u, 0u};
      vreg[ks] = krow < S_ ? gload<u32x4>(vb + ks * 16, voff) : u32x4{0u, 0u, 0u, 0u};
    }
  }

  const int nqt = static_cast<int>((T_ + QT - 1) / QT);
  int qt_lo = 0, qt_hi = nqt;
  if (a.masked && a.prune) {
    const int64_t klast = (k0 + C::KB - 1 < S_ ? k0 + C::KB - 1 : S_ - 1);
    if (a.band_hi < INT64_MAX / 4) {  // q >= key - hi
      const int64_t qmin = k0 - a.band_hi;
      qt_lo = qmin <= 0 ? 0 : static_cast<int>(qmin / QT < nqt ? qmin / QT : nqt);
    }
    if (a.band_lo > INT64_MIN / 4) {  // q <= key - lo
      const int64_t qmax = klast - a.band_lo;
      qt_hi = qmax < 0 ? 0 : static_cast<int>(qmax / QT + 1 < nqt ? qmax / QT + 1 : nqt);
    }
  }

  f32x16 dkacc[D / 32], dvacc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) {
    dkacc[db] = f32x16{};
    dvacc[db] = f32x16{};
  }

  TileT<QT, D> tq, tdo;
  float pl = 0.f, pd = 0.f, pq = 0.f;  // this thread's lse2 / delta / pm staging values (tid < QT)
  auto fetch = [&](int qt) {
    const int64_t q0 = static_cast<int64_t>(qt) * QT;
    const int64_t nv = T_ - q0;
    tload<QT, D>(tq, qp + q0 * a.q_st, a.q_st, nv, tid);
    tload<QT, D>(tdo, dop + q0 * a.o_st, a.o_st, nv, tid);
    if (tid < QT) {
      const bool ok = q0 + tid < T_;
      pl = ok ? lsep[q0 + tid] : 0.f;
      pd = ok ? delp[q0 + tid] : 0.f;
      pq = ok ? pmp[q0 + tid] : 0.f;
    }
  };
  auto stage_in = [&](unsigned char* st) {
    tstore_rows<QT, D>(tq, st, C::RS, tid);
    tstore_trans<QT, D>(tq, st + C::OFF_QT, C::TS, tid);
    tstore_rows<QT, D>(tdo, st + C::OFF_DO, C::RS, tid);
    tstore_trans<QT, D>(tdo, st + C::OFF_DOT, C::TS, tid);
    if (tid < QT) {
      reinterpret_cast<float*>(st + C::OFF_LSE)[tid] = pl;
      reinterpret_cast<float*>(st + C::OFF_DEL)[tid] = pd;
      reinterpret_cast<float*>(st + C::OFF_PM)[tid] = pq;
    }
  };

  if (qt_lo < qt_hi) {
    fetch(qt_lo);
    stage_in(smem);
  }
  for (int qt = qt_lo; qt < qt_hi; ++qt) {
    __syncthreads();
    unsigned char* st = smem + ((qt - qt_lo) & 1) * C::STAGE;
    const bool more = qt + 1 < qt_hi;
    if (more) fetch(qt + 1);

    const int64_t q0 = static_cast<int64_t>(qt) * QT;
    const int64_t dmin = kw0 - (q0 + QT - 1), dmax = kw0 + 31 - q0;  // key - q over the tile
    bool dead = false, cut = q0 + QT > T_ || kw0 + 32 > S_;
    if (a.masked) {
      dead = a.prune && (dmin > a.band_hi || dmax < a.band_lo);
      cut = cut || dmin < a.band_lo || dmax > a.band_hi;
    }
    if (!dead) {
      f32x16 sacc[NQB], pacc[NQB];
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        sacc[qb] = f32x16{};
        pacc[qb] = f32x16{};
      }
      const unsigned char* qrows = st + r32 * C::RS + g * 16;
      const unsigned char* drows = st + C::OFF_DO + r32 * C::RS + g * 16;
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
          sacc[qb] = mfma32<T>(*reinterpret_cast<const u32x4*>(qrows + qb * 32 * C::RS + ks * 32), kreg[ks], sacc[qb]);
          pacc[qb] = mfma32<T>(*reinterpret_cast<const u32x4*>(drows + qb * 32 * C::RS + ks * 32), vreg[ks], pacc[qb]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the phases' live ranges apart
      const float* lse_l = reinterpret_cast<const float*>(st + C::OFF_LSE);
      const float* del_l = reinterpret_cast<const float*>(st + C::OFF_DEL);
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int rbase = qb * 32 + hh * 16 + g * 8;  // tile rows of accumulators [8hh, 8hh+8)
          const f32x4 l0 = *reinterpret_cast<const f32x4*>(lse_l + rbase);
          const f32x4 l1 = *reinterpret_cast<const f32x4*>(lse_l + rbase + 4);
          const f32x4 d0 = *reinterpret_cast<const f32x4*>(del_l + rbase);
          const f32x4 d1 = *reinterpret_cast<const f32x4*>(del_l + rbase + 4);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int i = 8 * hh + j;
            const float lv = j < 4 ? l0[j] : l1[j - 4];
            const float dv = j < 4 ? d0[j] : d1[j - 4];
            float p = fast_exp2(sacc[qb][i] * a.c2 - lv);
            bool live = true;
            if (cut) {
              const int64_t qq = q0 + rbase + j;
              const int64_t dd = static_cast<int64_t>(krow) - qq;
              if (qq >= T_ || krow >= S_) {
                live = false;
                p = 0.f;
              } else if (a.masked && (dd < a.band_lo || dd > a.band_hi)) {
                live = false;
                p = reinterpret_cast<const float*>(st + C::OFF_PM)[rbase + j];
              }
            }
            sacc[qb][i] = p;
            pacc[qb][i] = live ? p * (pacc[qb][i] - dv) : 0.f;
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      const unsigned char* dot_l = st + C::OFF_DOT + r32 * C::TS + g * 16;
      const unsigned char* qt_l = st + C::OFF_QT + r32 * C::TS + g * 16;
#pragma unroll
      for (int s = 0; s < QT / 16; ++s) {
        const u32x4 pp = pack8<T>(sacc[s >> 1], s & 1);
        const u32x4 ds = pack8<T>(pacc[s >> 1], s & 1);
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
          dvacc[db] = mfma32<T>(*reinterpret_cast<const u32x4*>(dot_l + db * 32 * C::TS + s * 32), pp, dvacc[db]);
          dkacc[db] = mfma32<T>(*reinterpret_cast<const u32x4*>(qt_l + db * 32 * C::TS + s * 32), ds, dkacc[db]);
        }
      }
    }
    if (more) stage_in(smem + ((qt + 1 - qt_lo) & 1) * C::STAGE);
  }

  if (krow < S_) {
    store_rows_t<T, D>(a.dk + b * a.k_sb + h * a.k_sh + static_cast<int64_t>(kw0) * a.k_st, a.k_st, r32, g, dkacc,
                       a.scale);
    store_rows_t<T, D>(a.dv + b * a.v_sb + h * a.v_sh + static_cast<int64_t>(kw0) * a.v_st, a.v_st, r32, g, dvacc,
                       1.0f);
  }
}

// -------------------------------------------------------------------- dQ

template <int D>
struct DqCfg {
  static constexpr int BM = 128;  // query rows per workgroup
  static constexpr int BN = 64;   // keys per tile
  static constexpr int RS = D * 2 + 16;
  static constexpr int TS = BN * 2 + 16;
  static constexpr int KR = BN * RS;
  static constexpr int OFF_V = KR, OFF_KT = 2 * KR;
  static constexpr int STAGE = 2 * KR + D * TS;
  static constexpr int LDS = 2 * STAGE;
};

template <typename T, int D>
__global__ __launch_bounds__(256, D == 64 ? 2 : 1) void bwd_dq(BwdArgs a) {
  using C = DqCfg<D>;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id(), r32 = lane & 31, g = lane >> 5;
  const int64_t inst = blockIdx.x / a.nblk;
  const int qb = a.nblk - 1 - static_cast<int>(blockIdx.x % a.nblk);  // heavy (late) blocks first
  const int64_t b = inst / a.heads, h = inst % a.heads;
  const uint16_t* qp = a.q + b * a.q_sb + h * a.q_sh;
  const uint16_t* kp = a.k + b * a.k_sb + h * a.k_sh;
  const uint16_t* vp = a.v + b * a.v_sb + h * a.v_sh;
  const uint16_t* dop = a.dout + b * a.o_sb + h * a.o_sh;
  const int64_t T_ = a.t, S_ = a.s;
  const int q0 = qb * C::BM;
  const int qw0 = q0 + 32 * w;
  const int qrow = qw0 + r32;

  u32x4 qreg[D / 16], doreg[D / 16];
  {
    const uint32_t qoff = static_cast<uint32_t>(r32 * a.q_st * 2 + g * 16);
    const uint32_t ooff = static_cast<uint32_t>(r32 * a.o_st * 2 + g * 16);
    const uint16_t* qbs = qp + static_cast<int64_t>(qw0) * a.q_st;
    const uint16_t* obs = dop + static_cast<int64_t>(qw0) * a.o_st;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      qreg[ks] = qrow < T_ ? gload<u32x4>(qbs + ks * 16, qoff) : u32x4{0u, 0u, 0u, 0u};
      doreg[ks] = qrow < T_ ? gload<u32x4>(obs + ks * 16, ooff) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  const int64_t srow = inst * T_ + qrow;
  const float dl = qrow < T_ ? a.ws[srow] : 0.f;
  const float lse2 = qrow < T_ ? a.ws[a.rows + srow] : 0.f;

  const int ntiles = static_cast<int>((S_ + C::BN - 1) / C::BN);
  int kt_lo = 0, kt_hi = ntiles;
  if (a.masked && a.prune) {
    const int64_t qlast = (q0 + C::BM - 1 < T_ ? q0 + C::BM - 1 : T_ - 1);
    if (a.band_hi < INT64_MAX / 4) {
      const int64_t smax = qlast + a.band_hi;
      kt_hi = smax < 0 ? 0 : static_cast<int>(smax / C::BN + 1 < ntiles ? smax / C::BN + 1 : ntiles);
    }
    if (a.band_lo > INT64_MIN / 4) {
      const int64_t smin = q0 + a.band_lo;
      kt_lo = smin <= 0 ? 0 : static_cast<int>(smin / C::BN);
    }
  }

  f32x16 dqacc[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) dqacc[db] = f32x16{};

  TileT<64, D> tk, tv;
  auto fetch = [&](int kt) {
    const int64_t key0 = static_cast<int64_t>(kt) * C::BN;
    tload<64, D>(tk, kp + key0 * a.k_st, a.k_st, S_ - key0, tid);
    tload<64, D>(tv, vp + key0 * a.v_st, a.v_st, S_ - key0, tid);
  };
  auto stage_in = [&](unsigned char* st) {
    tstore_rows<64, D>(tk, st, C::RS, tid);
    tstore_rows<64, D>(tv, st + C::OFF_V, C::RS, tid);
    tstore_trans<64, D>(tk, st + C::OFF_KT, C::TS, tid);
  };

  if (kt_lo < kt_hi) {
    fetch(kt_lo);
    stage_in(smem);
  }
  for (int kt = kt_lo; kt < kt_hi; ++kt) {
    __syncthreads();
    unsigned char* st = smem + ((kt - kt_lo) & 1) * C::STAGE;
    const bool more = kt + 1 < kt_hi;
    if (more) fetch(kt + 1);

    const int64_t key0 = static_cast<int64_t>(kt) * C::BN;
    const int64_t dmin = key0 - (qw0 + 31), dmax = key0 + C::BN - 1 - qw0;
    bool dead = false, cut = key0 + C::BN > S_ || qw0 + 32 > T_;
    if (a.masked) {
      dead = a.prune && (dmin > a.band_hi || dmax < a.band_lo);
      cut = cut || dmin < a.band_lo || dmax > a.band_hi;
    }
    if (!dead) {
      f32x16 sacc[2] = {f32x16{}, f32x16{}}, pacc[2] = {f32x16{}, f32x16{}};
      const unsigned char* krows = st + r32 * C::RS + g * 16;
      const unsigned char* vrows = st + C::OFF_V + r32 * C::RS + g * 16;
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          sacc[kb] = mfma32<T>(*reinterpret_cast<const u32x4*>(krows + kb * 32 * C::RS + ks * 32), qreg[ks], sacc[kb]);
          pacc[kb] = mfma32<T>(*reinterpret_cast<const u32x4*>(vrows + kb * 32 * C::RS + ks * 32), doreg[ks], pacc[kb]);
        }
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float p = fast_exp2(sacc[kb][i] * a.c2 - lse2);
          bool live = true;
          if (cut) {
            const int64_t key = key0 + kb * 32 + acc_row(i, g);
            const int64_t dd = key - qrow;
            if (key >= S_ || qrow >= T_ || (a.masked && (dd < a.band_lo || dd > a.band_hi))) live = false;
          }
          pacc[kb][i] = live ? p * (pacc[kb][i] - dl) : 0.f;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      const unsigned char* kt_l = st + C::OFF_KT + r32 * C::TS + g * 16;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4 ds = pack8<T>(pacc[s >> 1], s & 1);
#pragma unroll
        for (int db = 0; db < D / 32; ++db)
          dqacc[db] = mfma32<T>(*reinterpret_cast<const u32x4*>(kt_l + db * 32 * C::TS + s * 32), ds, dqacc[db]);
      }
    }
    if (more) stage_in(smem + ((kt + 1 - kt_lo) & 1) * C::STAGE);
  }

  if (qrow < T_)
    store_rows_t<T, D>(a.dq + b * a.q_sb + h * a.q_sh + static_cast<int64_t>(qw0) * a.q_st, a.q_st, r32, g, dqacc,
                       a.scale);
}

bool band_has_empty_row(int64_t T, int64_t S, int64_t lo, int64_t hi) {
  if (lo > hi) return true;
  if (hi < 0) return true;
  if (lo > INT64_MIN / 4 && (T - 1) + lo > S - 1) return true;
  return false;
}

template <typename T, int D>
int launch_bwd(BwdArgs a, int64_t ninst, hipStream_t st) {
  bwd_stats<T, D><<<dim3(static_cast<unsigned>((a.rows + 3) / 4)), 256, 0, st>>>(a);
  int rc = check_launch("pdh_flash_bwd (row stats)");
  if (rc) return rc;
  {
    using C = DkdvCfg<D>;
    BwdArgs ak = a;
    ak.nblk = static_cast<int>((a.s + C::KB - 1) / C::KB);
    hipFuncSetAttribute(reinterpret_cast<const void*>(&bwd_dkdv<T, D>), hipFuncAttributeMaxDynamicSharedMemorySize,
                        C::LDS);
    bwd_dkdv<T, D><<<dim3(static_cast<unsigned>(ninst * ak.nblk)), 256, C::LDS, st>>>(ak);
    rc = check_launch("pdh_flash_bwd (dk, dv)");
    if (rc) return rc;
  }
  {
    using C = DqCfg<D>;
    BwdArgs aq = a;
    aq.nblk = static_cast<int>((a.t + C::BM - 1) / C::BM);
    hipFuncSetAttribute(reinterpret_cast<const void*>(&bwd_dq<T, D>), hipFuncAttributeMaxDynamicSharedMemorySize,
                        C::LDS);
    bwd_dq<T, D><<<dim3(static_cast<unsigned>(ninst * aq.nblk)), 256, C::LDS, st>>>(aq);
    rc = check_launch("pdh_flash_bwd (dq)");
  }
  return rc;
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
  PDH_REQUIRE(G.batch >= 0 && G.heads_q >= 1 && G.t >= 0 && G.s >= 1, PDH_EINVAL, "pdh_flash_bwd: bad shape");
  PDH_REQUIRE(G.heads_q == G.heads_kv, PDH_EUNSUPPORTED,
              "pdh_flash_bwd: grouped-query backward (heads_q %lld != heads_kv %lld) is not supported",
              (long long)G.heads_q, (long long)G.heads_kv);
  PDH_REQUIRE(dtype == PDH_BF16 || dtype == PDH_F16, PDH_EUNSUPPORTED, "pdh_flash_bwd: dtype must be bf16 or f16");
  PDH_REQUIRE(G.e == G.od && (G.e == 64 || G.e == 128), PDH_EUNSUPPORTED,
              "pdh_flash_bwd: need e == od in {64, 128} (got %lld, %lld)", (long long)G.e, (long long)G.od);
  PDH_REQUIRE(mask_kind == PDH_MASK_NONE || mask_kind == PDH_MASK_BAND, PDH_EINVAL,
              "pdh_flash_bwd: unknown mask kind %d", mask_kind);
  PDH_REQUIRE(q && k && v && o && dout && lse && dq && dk && dv && ws, PDH_EINVAL, "pdh_flash_bwd: null pointer");
  PDH_REQUIRE((m_in == nullptr) == (den_in == nullptr), PDH_EINVAL, "pdh_flash_bwd: pass both m and den, or neither");
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
  const int64_t ninst = G.batch * G.heads_q;
  if (ninst == 0 || G.t == 0) return PDH_OK;
  const int masked = mask_kind == PDH_MASK_BAND;
  const int prune_ok = masked && !band_has_empty_row(G.t, G.s, band_lo, band_hi);
  BwdArgs a{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
            static_cast<const uint16_t*>(o), static_cast<const uint16_t*>(dout), lse, m_in, den_in,
            static_cast<uint16_t*>(dq), static_cast<uint16_t*>(dk), static_cast<uint16_t*>(dv), ws,
            ninst * G.t, G.heads_q, G.t, G.s, G.q_sb, G.q_sh, G.q_st, G.k_sb, G.k_sh, G.k_st, G.v_sb, G.v_sh, G.v_st,
            G.o_sb, G.o_sh, G.o_st, scale, scale * kLog2e, fill * kLog2e, masked, band_lo, band_hi, prune_ok, 0};
  hipStream_t st = as_stream(stream);
  if (dtype == PDH_BF16)
    return G.e == 128 ? launch_bwd<__hip_bfloat16, 128>(a, ninst, st) : launch_bwd<__hip_bfloat16, 64>(a, ninst, st);
  return G.e == 128 ? launch_bwd<_Float16, 128>(a, ninst, st) : launch_bwd<_Float16, 64>(a, ninst, st);
}
