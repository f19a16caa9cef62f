// Flash-attention forward — the "flash" template row of the fusion registry
// (fusion.py:480-615): the online-softmax fold over key tiles, with the
// (out, m, den) artifacts of the artifact variant (fusion.py:611-613) and lse = m + log(den).
//
// MFMA kernel (bf16 / f16 in, fp32 accumulate), e == od == D in {64, 128}:
//   * workgroup = 4 waves x 32 query rows = 128 rows; key tiles of 32 rows,
//     double-buffered in LDS (32 KB at D = 128): three workgroups share a CU,
//     so three waves per SIMD overlap each other's LDS / MFMA / VALU latency;
//   * K and V tiles go HBM -> LDS by direct buffer loads (no VGPR staging, no
//     LDS write instructions) into unpadded rows whose 16-byte slots are
//     XOR-swizzled so every operand read is bank-conflict free;
//   * scores are computed TRANSPOSED, S^T = K Q^T with v_mfma_f32_16x16x32
//     (the matrix cores' faster shape on gfx950): lane 16 G + c owns query
//     rows c and 16 + c of its wave's 32, so the running max / denominator
//     live in registers; its eight keys of each 32-key tile are exactly the
//     B operand of O^T += V^T P^T (no register shuffles between the two
//     contractions; see the 16x16x32 section below);
//   * V stays row-major in LDS and is read transposed by ds_read_b64_tr_b16;
//     the LDS array is static and the key-tile loop runs in buffer pairs, so
//     every operand read is a lane offset plus an immediate (no per-tile
//     address arithmetic);
//   * exp runs as exp2 on log2(e)-scaled scores (v_exp_f32); the running max
//     is rescaled lazily (only when it grows by more than 2^8). Without the
//     (m, den) artifacts, full tiles skip the row max altogether: their
//     exponentials are referred to the running reference, and a tile takes
//     the exact path (row max, rescale, exponentials again) only when a lane's
//     partial sum leaves (0, 2^8]. On gfx950 VALU work adds to MFMA time
//     almost one for one once the matrix pipe is busy, so every VALU
//     instruction taken out of the tile body is time saved (a full tile is
//     32 products and 60 other VALU instructions per wave);
//   * causal / band masks prune dead tiles (the mask-derived bounds of
//     fusion.py:659-690) and mask only the tiles the band cuts;
//   * heavy (late) query blocks launch first, and the workgroup index is
//     remapped so each XCD works through whole (batch, head) instances — the
//     instance's K/V stays in that XCD's L2 — taking an instance's blocks in
//     groups of four of alternating direction, so each of an XCD's four
//     shader engines receives the same total work.
//
// Generic fp32 kernel (any e, od, t, s): one wave per query row, keys in
// chunks of 64 (one per lane), the same recurrence in fp32 — the column the
// reference's f32 Triton runner occupies (conformance/triton_tile.py:662-698).
#include "attn_common.h"

#include <type_traits>

namespace pdh {
namespace {

constexpr float kInf = __builtin_inff();

struct FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* m_out;
  float* den_out;
  float* lse_out;
  int64_t heads_q, heads_kv;
  int64_t t, s;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
  float scale;     // > 0
  float c2;        // scale * log2(e)
  float fill_raw;  // fill / scale: the masked raw score
  int masked;   // 0: no mask, 1: band
  int64_t band_lo, band_hi;
  int prune;    // skip dead tiles
  int nqb;      // query blocks per instance
  int xcd_remap;
  // split over the key axis (nsplit > 1): workgroup (block, split c) sweeps key
  // tiles [lo + c * split_tiles, ...) of its block's range and stores partial
  // (o referred to mused, mused, mtrue, den) to ws; flash_fwd_combine merges
  int nsplit, split_tiles;
  float* ws;      // [nsplit][plane][D] partial o, then [3][nsplit][plane] mused, mtrue, den
  int64_t plane;  // instances * t: rows per split
  // the band clamped to +-(2^29 + 64): with t, s <= 2^29 every key - row
  // difference compares the same against these as against the 64-bit band
  int band_lo32, band_hi32;
};

// Lazy rescaling: the running max used for the exponentials only moves when a
// row's max grows by more than 2^kTau (log2 units); probabilities then stay
// <= 2^kTau, the O accumulators are rescaled rarely, and the result is the
// same quotient (exact in real arithmetic).
constexpr float kTau = 8.0f;

// A workgroup's place in the grid and its key-tile ranges: the instance and
// query block it owns (heavy late blocks first, in an XCD- and shader-engine-
// aware order), the live key tiles [kt_lo, kt_hi) after the mask-derived
// prune, the run [kf_lo, kf_hi) of tiles live for every row of the block, and,
// for a split launch, this split's share of the range.
struct BlockPlan {
  int64_t inst;
  int qb, split;
  int kt_lo, kt_hi, kf_lo, kf_hi;
};

template <int BM, int BN>
__device__ __forceinline__ BlockPlan block_plan(const FwdArgs& a) {
  // workgroup -> (instance, query block); heavy (late) query blocks first
  int bid = blockIdx.x;
  int split = 0;
  if (a.nsplit > 1) {  // the splits of one query block are adjacent workgroups
    split = bid % a.nsplit;
    bid /= a.nsplit;
  }
  int64_t inst;
  int qb;
  if (a.xcd_remap == 3) {
    // Workgroups are dispatched round-robin over the 8 XCDs (bid % 8); each
    // XCD works through whole instances, heavy query blocks first. Its
    // workgroups go round-robin to its four shader engines (r % 4), so the
    // blocks are taken in groups of four whose direction alternates (31 30
    // 29 28, 24 25 26 27, 23 ...): over an instance every engine then draws
    // the same total work, and the XCD's L2 holds the K / V of the few
    // instances it is sweeping.
    const int per = gridDim.x >> 3;
    const int x = bid & 7, r = bid >> 3;
    const int64_t lin = static_cast<int64_t>(x) * per + r;
    inst = lin / a.nqb;
    const int j = static_cast<int>(lin % a.nqb), grp = j >> 2, e = j & 3;
    qb = a.nqb - 1 - (4 * grp + ((grp & 1) ? 3 - e : e));
  } else {
    if (a.xcd_remap) {
      const int per = gridDim.x >> 3;
      bid = (bid & 7) * per + (bid >> 3);
    }
    inst = bid / a.nqb;
    qb = a.nqb - 1 - (bid % a.nqb);
  }
  const int64_t T_ = a.t, S_ = a.s;
  const int q0 = qb * BM;
  // key-tile range of the workgroup (mask-derived prune, absolute tile grid)
  const int ntiles = static_cast<int>((S_ + BN - 1) / BN);
  int kt_lo = 0, kt_hi = ntiles;
  if (a.masked && a.prune) {
    const int64_t qlast = (q0 + BM - 1 < T_ ? q0 + BM - 1 : T_ - 1);
    if (a.band_hi < INT64_MAX / 4) {
      const int64_t smax = qlast + a.band_hi;  // last live key of the block
      kt_hi = smax < 0 ? 0 : static_cast<int>(smax / BN + 1 < ntiles ? smax / BN + 1 : ntiles);
    }
    if (a.band_lo > INT64_MIN / 4) {
      const int64_t smin = q0 + a.band_lo;  // first live key of the block
      kt_lo = smin <= 0 ? 0 : static_cast<int>(smin / BN);
    }
  }
  // Tiles fully live for every row of the workgroup form one run [kf_lo, kf_hi);
  // the tiles before it (a window's left edge) and after it (the diagonal, the
  // key tail) take the masked body.
  int kf_lo = kt_lo, kf_hi = kt_hi;
  {
    const int64_t full_end_keys = S_ / BN;
    kf_hi = kf_hi < full_end_keys ? kf_hi : static_cast<int>(full_end_keys);
    if (a.masked) {
      const int64_t qlo = q0, qhi = q0 + BM - 1;
      if (a.band_hi < INT64_MAX / 4) {  // key0 + BN - 1 - qlo <= hi
        const int64_t lim = qlo + a.band_hi - (BN - 1);
        const int64_t n = lim < 0 ? 0 : lim / BN + 1;
        kf_hi = kf_hi < n ? kf_hi : static_cast<int>(n);
      }
      if (a.band_lo > INT64_MIN / 4) {  // key0 - qhi >= lo
        const int64_t lim = qhi + a.band_lo;
        const int64_t n = lim <= 0 ? 0 : (lim + BN - 1) / BN;
        kf_lo = kf_lo > n ? kf_lo : static_cast<int>(n);
      }
    }
    if (kf_lo > kf_hi) kf_lo = kf_hi = kt_hi;
  }
  if (a.nsplit > 1) {  // this split's share of the range; the run boundaries clamp into it
    const int s_lo = kt_lo + split * a.split_tiles;
    const int lo2 = s_lo < kt_hi ? s_lo : kt_hi;
    const int hi2 = s_lo + a.split_tiles < kt_hi ? s_lo + a.split_tiles : kt_hi;
    kf_lo = kf_lo < lo2 ? lo2 : (kf_lo > hi2 ? hi2 : kf_lo);
    kf_hi = kf_hi < lo2 ? lo2 : (kf_hi > hi2 ? hi2 : kf_hi);
    kt_lo = lo2;
    kt_hi = hi2;
  }

  return BlockPlan{inst, qb, split, kt_lo, kt_hi, kf_lo, kf_hi};
}

// ------------------------------------------------ 16x16x32 MFMA forward
//
// The same sweep on v_mfma_f32_16x16x32 products. A wave still owns 32 query
// rows, as two 16-row halves: lane l = 16 G + c owns query rows c and 16 + c
// of the wave's 32, and within each 32-key tile the keys {4G .. 4G+3} and
// {16+4G .. 16+4G+3}. Those eight keys are exactly the B operand (k = 8G + j)
// of O^T += V^T P^T once the k index j is read as key 4G + j (j < 4) or
// 16 + 4G + j - 4 (j >= 4); the V operand follows the same k order, which the
// transposed LDS read gives for free (each 16-lane group names its own four
// rows). So, as in the 32x32x16 kernel, the score accumulators feed the
// second product with no register shuffle.

template <int D>
struct F16Cfg {
  static constexpr int WAVES = 4;
  static constexpr int THREADS = 64 * WAVES;
  static constexpr int BM = 32 * WAVES;    // query rows per workgroup (32 per wave)
  static constexpr int BN = 32;            // keys per tile
  static constexpr int ROWB = D * 2;       // LDS bytes per key row (swizzled, unpadded)
  static constexpr int CPR = D / 8;        // 16-byte chunks per row
  static constexpr int TILEB = BN * ROWB;  // one K or V tile
  static constexpr int KBUF = 0, VBUF = 2 * TILEB;
  static constexpr int LDS = 4 * TILEB;    // K and V, double buffered: 32 KB at D = 128
  static constexpr int RPK = 1024 / ROWB;  // rows per 1 KB direct-load block
  static constexpr int NBLK = TILEB / 1024;
  static constexpr int NDMA = (NBLK + WAVES - 1) / WAVES;
  static constexpr int KS = D / 32;        // k-steps of Q K^T (32 features each)
  static constexpr int FB = D / 16;        // 16-feature blocks of O
  static constexpr int PF = 2;             // V operands in flight ahead of their MFMA
  static constexpr int KPF = 3;            // K operands in flight
};

// K rows are read as A operands: lanes 16 G + c read row c (of a 16-row
// half) at chunk 4 ks + G. On gfx950 a ds_read_b128 serves 16 lanes per
// cycle over 256 bytes of banks (measured by an in-bounds probe): within
// each 32-lane half, the quads of even bit parity of lane / 4 ({0, 3, 5, 6})
// share a cycle and the odd ones ({1, 2, 4, 7}) another, so each cycle's 16
// slots (address / 16 mod 16) must differ. At D = 128 (256-byte rows) the
// row's own mask does it; at D = 64 rows 2 i and 2 i + 1 share 256 bytes
// (row & 1 picks the half) and the mask 4 ((i ^ (i >> 2)) & 1) +
// 2 ((i >> 1) & 1), i = row >> 1, gives each cycle's rows of one half distinct slots.
template <int D>
__device__ __forceinline__ int swz16_k(int row) {
  return D == 128 ? (row & 15) : (4 * (((row >> 1) ^ (row >> 3)) & 1) | 2 * ((row >> 2) & 1));
}

// V rows are read with ds_read_b64_tr_b16: 16-lane group G reads rows
// 4G .. 4G+3 (and 16 + those), 32 contiguous bytes each (two slots). An
// 8-byte read serves 32 lanes per cycle over 256 bytes of banks; even masks
// keep a slot pair adjacent and put lanes 0-31 (rows 0-7) on distinct banks.
template <int D>
__device__ __forceinline__ int swz16_v(int row) {
  return D == 128 ? 2 * (row & 7) : 2 * ((row & 3) ^ ((row >> 2) & 1));
}

// Row-wise combine across the four 16-lane groups (v_permlane32_swap and
// v_permlane16_swap exchange lane l with l ^ 32 and l ^ 16).
__device__ __forceinline__ float max4g(float m) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  m = __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
  return __builtin_fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

__device__ __forceinline__ float sum4g(float v) {
  v += __shfl_xor(v, 32, 64);
  return v + __shfl_xor(v, 16, 64);
}

// Stores a wave's 32 query rows (two halves of 16) from the 16x16 layout:
// o = oacc / den and the optional m, den and lse rows, or, for a split
// launch, the unnormalized partial state flash_fwd_combine merges.
template <typename T, int D>
__device__ __forceinline__ void fwd16_store(const FwdArgs& a, int64_t inst, int split, int qw0, int c, int G,
                                            uint16_t* op, const f32x4 (&oacc)[D / 16][2], const float (&mused)[2],
                                            const float (&mtrue)[2], const float (&lsum)[2]) {
  constexpr int FB = D / 16;
  const int64_t T_ = a.t;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int qrow = qw0 + 16 * h + c;
    const float den = sum4g(lsum[h]);
    if (qrow >= T_) continue;
    if (a.nsplit > 1) {  // the partial state, unnormalized, for flash_fwd_combine
      const int64_t srow = split * a.plane + inst * T_ + qrow;
      float* wo = a.ws + srow * D + 4 * G;
#pragma unroll
      for (int fb = 0; fb < FB; ++fb) *reinterpret_cast<f32x4*>(wo + 16 * fb) = oacc[fb][h];
      if (G == 0) {
        float* st = a.ws + a.nsplit * a.plane * D;
        st[srow] = mused[h];
        st[a.nsplit * a.plane + srow] = mtrue[h];
        st[2 * a.nsplit * a.plane + srow] = den;
      }
      continue;
    }
    const float inv = den > 0.f ? 1.0f / den : 0.f;
    uint16_t* obase = op + static_cast<int64_t>(qw0 + 16 * h) * a.o_st;  // wave-uniform
    const uint32_t o_lane = static_cast<uint32_t>(c * a.o_st * 2 + G * 8);
#pragma unroll
    for (int fb = 0; fb < FB; ++fb) {
      const f32x4 x = oacc[fb][h];
      gstore<u32x2>(obase + 16 * fb, o_lane, u32x2{pack2<T>(x[0] * inv, x[1] * inv), pack2<T>(x[2] * inv, x[3] * inv)});
    }
    if (G == 0) {
      const int64_t srow = inst * T_ + qrow;
      if (a.m_out) a.m_out[srow] = mtrue[h] * a.scale;
      if (a.den_out) a.den_out[srow] = den * fast_exp2((mused[h] - mtrue[h]) * a.c2);
      if (a.lse_out) a.lse_out[srow] = mused[h] * a.scale + __logf(den);
    }
  }
}

template <typename T, int D, bool ART>
__global__ __launch_bounds__(F16Cfg<D>::THREADS, 3) void flash_fwd_m16(FwdArgs a) {
  using C = F16Cfg<D>;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[C::LDS];
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id(), c = lane & 15, G = lane >> 4;

  const BlockPlan bp = block_plan<C::BM, C::BN>(a);
  const int64_t inst = bp.inst;
  const int kt_lo = bp.kt_lo, kt_hi = bp.kt_hi, kf_lo = bp.kf_lo, kf_hi = bp.kf_hi;
  const int64_t b = inst / a.heads_q, hq = inst % a.heads_q;
  const int64_t hk = hq / (a.heads_q / a.heads_kv);
  const uint16_t* qp = static_cast<const uint16_t*>(a.q) + b * a.q_sb + hq * a.q_sh;
  const uint16_t* kp = static_cast<const uint16_t*>(a.k) + b * a.k_sb + hk * a.k_sh;
  const uint16_t* vp = static_cast<const uint16_t*>(a.v) + b * a.v_sb + hk * a.v_sh;
  uint16_t* op = static_cast<uint16_t*>(a.o) + b * a.o_sb + hq * a.o_sh;
  // sequence lengths are bounded by 2^29 on the host: row / key arithmetic is 32-bit
  const int T_ = static_cast<int>(a.t), S_ = static_cast<int>(a.s);
  const int qw0 = bp.qb * C::BM + 32 * w;  // this wave's first row
  const int qr0 = qw0 + c, qr1 = qw0 + 16 + c;

  // Q as the B operand of S^T = K Q^T: lane holds q[row h][32 ks + 8 G .. +8]
  u32x4 qreg[2][C::KS];
  {
    const uint16_t* qbase = qp + static_cast<int64_t>(qw0) * a.q_st;  // wave-uniform
    const uint32_t q_lane = static_cast<uint32_t>(c * a.q_st * 2 + G * 16);
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int ks = 0; ks < C::KS; ++ks)
        qreg[h][ks] = (h ? qr1 : qr0) < T_ ? gload<u32x4>(qbase + 16 * h * a.q_st + ks * 32, q_lane)
                                           : u32x4{0u, 0u, 0u, 0u};
  }

  // ---- staging: 1 KB direct-load blocks; rows past the last key read as zero
  const uint32_t grk = static_cast<uint32_t>(a.k_st * 2), grv = static_cast<uint32_t>(a.v_st * 2);
  const rsrc_t kr = make_rsrc(kp, static_cast<uint32_t>((a.s - 1) * a.k_st * 2 + D * 2));
  const rsrc_t vr = make_rsrc(vp, static_cast<uint32_t>((a.s - 1) * a.v_st * 2 + D * 2));
  const int lrow = lane / C::CPR, slot = lane % C::CPR;
  uint32_t dk[C::NDMA], dv[C::NDMA];
#pragma unroll
  for (int i = 0; i < C::NDMA; ++i) {
    const int rho = (i * C::WAVES + w) * C::RPK + lrow;
    dk[i] = lrow * grk + ((slot ^ swz16_k<D>(rho)) << 4);
    dv[i] = lrow * grv + ((slot ^ swz16_v<D>(rho)) << 4);
  }
  auto stage = [&](int tile, int buf) {
#pragma unroll
    for (int i = 0; i < C::NDMA; ++i) {
      const int blk = i * C::WAVES + w;
      if (C::NBLK % C::WAVES != 0 && blk >= C::NBLK) break;
      const uint32_t row0 = static_cast<uint32_t>(tile * C::BN + blk * C::RPK);
      dma16(kr, smem + C::KBUF + buf * C::TILEB + blk * 1024, dk[i], row0 * grk);
      dma16(vr, smem + C::VBUF + buf * C::TILEB + blk * 1024, dv[i], row0 * grv);
    }
  };

  // ---- per-lane operand offsets (tile, buffer and 16-row half are immediates)
  int ka[C::KS];  // K row c, chunk 4 ks + G
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) ka[ks] = c * C::ROWB + (((4 * ks + G) ^ swz16_k<D>(c)) << 4);
  int va[C::FB];  // transposed V reads: row 4 G + k4 (+ 16), features 16 fb + 4 cc .. + 3
  {
    const int k4 = (lane >> 2) & 3, cc = lane & 3, row = 4 * G + k4;
#pragma unroll
    for (int fb = 0; fb < C::FB; ++fb)
      va[fb] = row * C::ROWB + (((2 * fb + (cc >> 1)) ^ swz16_v<D>(row)) << 4) + ((cc & 1) << 3);
  }

  float mused[2] = {-kInf, -kInf}, mtrue[2] = {-kInf, -kInf}, lsum[2] = {0.f, 0.f};
  f32x4 oacc[C::FB][2];
#pragma unroll
  for (int fb = 0; fb < C::FB; ++fb) oacc[fb][0] = oacc[fb][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto vfrag = [&](const unsigned char* vt, int fb) {
    const u32x2 lo = ds_read_tr16(vt + va[fb]);
    const u32x2 hi = ds_read_tr16(vt + 16 * C::ROWB + va[fb]);
    return u32x4{lo.x, lo.y, hi.x, hi.y};
  };

  auto tile = [&](auto bufc, int key0, auto cutc) {
    constexpr bool CUT = decltype(cutc)::value;
    constexpr int buf = decltype(bufc)::value;
    const unsigned char* kt = smem + C::KBUF + buf * C::TILEB;
    const unsigned char* vt = smem + C::VBUF + buf * C::TILEB;
    f32x4 sacc[2][2];  // [key half][query half]: S^T[16 kb + 4 G + i][16 h + c]
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) sacc[kb][0] = sacc[kb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    // K operands n = 2 ks + kb, read C::KPF ahead of their two products
    auto kfrag = [&](int n) { return *reinterpret_cast<const u32x4*>(kt + (n & 1) * 16 * C::ROWB + ka[n >> 1]); };
    u32x4 kf[C::KPF];
#pragma unroll
    for (int n = 0; n < C::KPF; ++n) kf[n] = kfrag(n);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int n = 0; n < 2 * C::KS; ++n) {
      const u32x4 kk = kf[n % C::KPF];
      if (n + C::KPF < 2 * C::KS) kf[n % C::KPF] = kfrag(n + C::KPF);
      const int ks = n >> 1, kb = n & 1;
      sacc[kb][0] = mfma16<T>(kk, qreg[0][ks], sacc[kb][0]);
      sacc[kb][1] = mfma16<T>(kk, qreg[1][ks], sacc[kb][1]);
    }
    u32x4 vf[C::PF];
#pragma unroll
    for (int n = 0; n < C::PF; ++n) vf[n] = vfrag(vt, n);
    __builtin_amdgcn_s_setprio(0);

    if constexpr (CUT) {
      // key of accumulator (kb, i) = kl + 16 kb + i; limits relative to it,
      // clamped to the tile (32-bit: |key - row| < 2^29 + 64)
      const int kl = key0 + 4 * G;
      const int rem = S_ - kl < 1024 ? S_ - kl : 1024;
      auto clampi = [](int x) { return x < -4096 ? -4096 : (x > 4096 ? 4096 : x); };
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int dl = kl - (h ? qr1 : qr0);
        const int lo = a.masked ? clampi(a.band_lo32 - dl) : -4096;
        const int hi = a.masked ? clampi(a.band_hi32 - dl) : 4096;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int cc = 16 * kb + i;
            const float x = (cc < lo || cc > hi) ? a.fill_raw : sacc[kb][h][i];
            sacc[kb][h][i] = cc >= rem ? -kInf : x;
          }
      }
    }
    u32x4 p[2];
    // the tile's exponentials of query half h into p[h]; returns their sum
    auto expo = [&](int h) {
      const float mc = mused[h] * a.c2;
      float e[8];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x = sacc[kb][h][i];
          e[4 * kb + i] = CUT ? fast_exp2((x - mused[h]) * a.c2) : fast_exp2(__builtin_fmaf(x, a.c2, -mc));
        }
      p[h] = u32x4{pack2<T>(e[0], e[1]), pack2<T>(e[2], e[3]), pack2<T>(e[4], e[5]), pack2<T>(e[6], e[7])};
      return ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
    };
    auto rowmax = [&](int h) {
      float m = -kInf;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) m = fmaxf(m, sacc[kb][h][i]);
      return max4g(m);
    };
    auto rescale = [&](int h, float mnew) {
      const float alpha = mnew == mused[h] ? 1.f : fast_exp2((mused[h] - mnew) * a.c2);
      mused[h] = mnew;
      lsum[h] *= alpha;
#pragma unroll
      for (int fb = 0; fb < C::FB; ++fb) oacc[fb][h] *= alpha;
    };
    if constexpr (!CUT && !ART) {
      float part0 = expo(0), part1 = expo(1);
      const float lim = static_cast<float>(1 << static_cast<int>(kTau));
      if (__builtin_amdgcn_ballot_w64(!(part0 <= lim) || !(part1 <= lim)) != 0) {
        rescale(0, fmaxf(mused[0], rowmax(0)));
        rescale(1, fmaxf(mused[1], rowmax(1)));
        part0 = expo(0);
        part1 = expo(1);
      }
      lsum[0] += part0;
      lsum[1] += part1;
    } else {
      const float m0 = rowmax(0), m1 = rowmax(1);
      mtrue[0] = fmaxf(mtrue[0], m0);
      mtrue[1] = fmaxf(mtrue[1], m1);
      if (__builtin_amdgcn_ballot_w64((m0 - mused[0]) * a.c2 > kTau || (m1 - mused[1]) * a.c2 > kTau) != 0) {
        rescale(0, fmaxf(mused[0], m0));
        rescale(1, fmaxf(mused[1], m1));
      }
      lsum[0] += expo(0);
      lsum[1] += expo(1);
    }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int fb = 0; fb < C::FB; ++fb) {
      const u32x4 vv = vf[fb % C::PF];
      if (fb + C::PF < C::FB) vf[fb % C::PF] = vfrag(vt, fb + C::PF);
      oacc[fb][0] = mfma16<T>(vv, p[0], oacc[fb][0]);
      oacc[fb][1] = mfma16<T>(vv, p[1], oacc[fb][1]);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  if (kt_lo < kt_hi) stage(kt_lo, 0);
  auto one = [&](int kt, auto bufc, auto cutc) {
    constexpr int buf = decltype(bufc)::value;
    wait_vmcnt0();
    __syncthreads();
    if (kt + 1 < kt_hi) stage(kt + 1, buf ^ 1);
    const int key0 = kt * C::BN;
    bool dead = false;
    if (decltype(cutc)::value && a.masked && a.prune) {  // this wave's rows see no live key here
      const int dmin = key0 - (qw0 + 31), dmax = key0 + C::BN - 1 - qw0;
      dead = dmin > a.band_hi32 || dmax < a.band_lo32;
    }
    if (!dead) tile(bufc, key0, cutc);
  };
  auto sweep = [&](int from, int to, auto cutc) {
    int kt = from;
    if (kt < to && ((kt - kt_lo) & 1)) one(kt++, std::integral_constant<int, 1>{}, cutc);
    for (; kt + 1 < to; kt += 2) {
      one(kt, std::integral_constant<int, 0>{}, cutc);
      one(kt + 1, std::integral_constant<int, 1>{}, cutc);
    }
    if (kt < to) one(kt, std::integral_constant<int, 0>{}, cutc);
  };
  sweep(kt_lo, kf_lo, std::true_type{});
  sweep(kf_lo, kf_hi, std::false_type{});
  sweep(kf_hi, kt_hi, std::true_type{});
  wait_vmcnt0();  // no load may be in flight into LDS when the workgroup exits

  const float mt[2] = {ART ? mtrue[0] : mused[0], ART ? mtrue[1] : mused[1]};
  fwd16_store<T, D>(a, inst, bp.split, qw0, c, G, op, oacc, mused, mt, lsum);
}

// ---------------------------------------------------------------- generic fp32

struct GenArgs {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  float* m_out;
  float* den_out;
  float* lse_out;
  int64_t heads_q, heads_kv, t, s, e, od;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st;
  float scale, fill;
  int masked;
  int64_t band_lo, band_hi;
  int prune;
};

constexpr int kGenOdPerLane = 8;  // od <= 512 handled in registers

// One wave per (instance, query row); keys in absolute chunks of 64.
__global__ __launch_bounds__(256) void flash_fwd_generic_f32(GenArgs a, int64_t nrows) {
  const int lane = threadIdx.x & 63;
  const int64_t grow = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (grow >= nrows) return;
  const int64_t inst = grow / a.t, t = grow % a.t;
  const int64_t b = inst / a.heads_q, hq = inst % a.heads_q, hk = hq / (a.heads_q / a.heads_kv);
  const float* qr = a.q + b * a.q_sb + hq * a.q_sh + t * a.q_st;
  const float* kp = a.k + b * a.k_sb + hk * a.k_sh;
  const float* vp = a.v + b * a.v_sb + hk * a.v_sh;
  float* orow = a.o + b * a.o_sb + hq * a.o_sh + t * a.o_st;

  int64_t c_lo = 0, c_hi = (a.s + 63) / 64;
  if (a.masked && a.prune) {
    if (a.band_hi < INT64_MAX / 4) {
      const int64_t smax = t + a.band_hi;
      c_hi = smax < 0 ? 0 : (smax / 64 + 1 < c_hi ? smax / 64 + 1 : c_hi);
    }
    if (a.band_lo > INT64_MIN / 4) {
      const int64_t smin = t + a.band_lo;
      c_lo = smin <= 0 ? 0 : smin / 64;
    }
  }
  float m = -kInf, l = 0.f;
  float acc[kGenOdPerLane];
#pragma unroll
  for (int j = 0; j < kGenOdPerLane; ++j) acc[j] = 0.f;
  for (int64_t c = c_lo; c < c_hi; ++c) {
    const int64_t key = c * 64 + lane;
    float sc = -kInf;
    if (key < a.s) {
      const float* kr = kp + key * a.k_st;
      float dot = 0.f;
      for (int64_t e = 0; e < a.e; ++e) dot = __builtin_fmaf(qr[e], kr[e], dot);
      sc = dot * a.scale;
      if (a.masked) {
        const int64_t d = key - t;
        if (d < a.band_lo || d > a.band_hi) sc = a.fill;
      }
    }
    const float mnew = fmaxf(m, wave_max(sc));
    const float alpha = __expf(m - mnew);
    const float p = key < a.s ? __expf(sc - mnew) : 0.f;
    l = l * alpha + wave_sum(p);
    m = mnew;
#pragma unroll
    for (int j = 0; j < kGenOdPerLane; ++j) acc[j] *= alpha;
    const int64_t nk = (a.s - c * 64) < 64 ? (a.s - c * 64) : 64;
    for (int kk = 0; kk < nk; ++kk) {
      const float pk = __shfl(p, kk, 64);
      const float* vr = vp + (c * 64 + kk) * a.v_st;
#pragma unroll
      for (int j = 0; j < kGenOdPerLane; ++j) {
        const int64_t d = j * 64 + lane;
        if (d < a.od) acc[j] = __builtin_fmaf(pk, vr[d], acc[j]);
      }
    }
  }
  const float inv = 1.0f / l;
#pragma unroll
  for (int j = 0; j < kGenOdPerLane; ++j) {
    const int64_t d = j * 64 + lane;
    if (d < a.od) orow[d] = acc[j] * inv;
  }
  if (lane == 0) {
    if (a.m_out) a.m_out[grow] = m;
    if (a.den_out) a.den_out[grow] = l;
    if (a.lse_out) a.lse_out[grow] = m + __logf(l);
  }
}

// The fp32 kernel for heads of E = OD = 32 or 64 features: lane = query
// row, 64 rows per workgroup, so each lane runs its own row's recurrence with
// no cross-lane reduction, and a key's K and V rows are the same for every
// lane. The workgroup copies each 64-key chunk of K and V (coalesced rows,
// zero past the range) into LDS and the waves read their keys' rows as
// broadcast LDS reads; eight keys per step give eight independent score
// chains. The chunk's groups of eight keys (on the absolute key grid) go
// round-robin to the NW waves (eight on grids under one workgroup per
// compute unit, four otherwise), and the NW partial states (m, l, o) merge
// through LDS with the associative combine (zoo/attention.py:40-46); the
// chunk buffers become the merge slots once every wave is done with them.
// Each row keeps the generic kernel's semantics: with pruning it sees exactly
// the 64-key chunks the band leaves it, a masked score inside them is the
// fill, and keys past s take no part. A group the prune skips holds only fill
// scores, whose exponentials vanish against the row's live maximum, and the
// assignment of groups to waves does not move with the range: pruned and
// unpruned sweeps agree bit for bit. Measured against the same recurrence on
// wave-uniform scalar loads (bit-equal results): 1.35-2.4x faster; loading
// the next chunk during the sweep needs registers this kernel does not have
// (it spilled and ran 10-15% slower).
template <int E, int OD, int NW>
__global__ __launch_bounds__(64 * NW) void flash_fwd_rows_f32_lds(GenArgs a, int nqb) {
  constexpr int CH = 64;
  static_assert(NW == 4 || NW == 8, "a chunk's eight groups split evenly over the waves");
  constexpr int KS = CH * E, VS = CH * OD;       // floats of one staged chunk
  constexpr int MS = (NW - 1) * (OD + 2) * 64;   // floats of the merge slots
  constexpr int SM = KS + VS > MS ? KS + VS : MS;
  constexpr int KPT = KS / (64 * NW), VPT = VS / (64 * NW);
  static_assert(KS % (64 * NW) == 0 && VS % (64 * NW) == 0, "a chunk splits evenly over the threads");
  __shared__ __attribute__((aligned(16))) float sm[SM];
  float* ks = sm;
  float* vs = sm + KS;
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int64_t inst = blockIdx.x / nqb;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x % nqb) * 64;
  const int64_t t = row0 + lane;
  const bool rin = t < a.t;
  const int64_t tc = rin ? t : a.t - 1;
  const int64_t b = inst / a.heads_q, hq = inst % a.heads_q, hk = hq / (a.heads_q / a.heads_kv);
  const float* __restrict__ qr = a.q + b * a.q_sb + hq * a.q_sh + tc * a.q_st;
  const float* __restrict__ kp = a.k + b * a.k_sb + hk * a.k_sh;
  const float* __restrict__ vp = a.v + b * a.v_sb + hk * a.v_sh;

  auto chunks = [&](int64_t row, int64_t& lo, int64_t& hi) {
    lo = 0;
    hi = (a.s + 63) / 64;
    if (a.masked && a.prune) {
      if (a.band_hi < INT64_MAX / 4) {
        const int64_t smax = row + a.band_hi;
        hi = smax < 0 ? 0 : (smax / 64 + 1 < hi ? smax / 64 + 1 : hi);
      }
      if (a.band_lo > INT64_MIN / 4) {
        const int64_t smin = row + a.band_lo;
        lo = smin <= 0 ? 0 : smin / 64;
      }
    }
  };
  int64_t rlo, rhi, blo, bhi, tmp;
  chunks(tc, rlo, rhi);
  chunks(row0, blo, tmp);
  chunks((row0 + 63 < a.t ? row0 + 63 : a.t - 1), tmp, bhi);
  const int64_t klo = blo * 64, khi = (bhi * 64 < a.s ? bhi * 64 : a.s);
  const int64_t kr_lo = rlo * 64, kr_hi = rhi * 64;

  float q[E];
#pragma unroll
  for (int e = 0; e < E; ++e) q[e] = qr[e];
  float m = -kInf, l = 0.f, acc[OD];
#pragma unroll
  for (int f = 0; f < OD; ++f) acc[f] = 0.f;

  // thread tid stages floats tid, tid + 512, ... of the chunk's K rows (and V
  // rows): consecutive threads read consecutive features of a row
  float kreg[KPT], vreg[VPT];
  auto fetch = [&](int64_t c0) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int idx = tid + 64 * NW * i;
      const int64_t key = c0 + idx / E;
      kreg[i] = key < khi ? kp[key * a.k_st + idx % E] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int idx = tid + 64 * NW * i;
      const int64_t key = c0 + idx / OD;
      vreg[i] = key < khi ? vp[key * a.v_st + idx % OD] : 0.f;
    }
  };
  const int64_t nch = khi > klo ? (khi - klo + CH - 1) / CH : 0;  // klo is a multiple of 64
  for (int64_t ci = 0; ci < nch; ++ci) {
    const int64_t c0 = klo + ci * CH;
    fetch(c0);
    __syncthreads();  // every wave is done with the previous chunk
#pragma unroll
    for (int i = 0; i < KPT; ++i) ks[tid + 64 * NW * i] = kreg[i];
#pragma unroll
    for (int i = 0; i < VPT; ++i) vs[tid + 64 * NW * i] = vreg[i];
    __syncthreads();  // the chunk is in LDS
    for (int gi = w; gi < CH / 8; gi += NW) {  // this wave's groups of the chunk
    const int64_t k0 = c0 + 8 * gi;
    if (k0 >= khi) continue;
    const float* __restrict__ kw = ks + 8 * gi * E;
    const float* __restrict__ vw = vs + 8 * gi * OD;
    float sc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) sc[j] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e)
#pragma unroll
      for (int j = 0; j < 8; ++j) sc[j] = __builtin_fmaf(q[e], kw[j * E + e], sc[j]);
    float mx = m;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t key = k0 + j;
      float x = sc[j] * a.scale;
      if (a.masked) {
        const int64_t d = key - tc;
        if (d < a.band_lo || d > a.band_hi) x = a.fill;
      }
      const bool in = key < khi && key >= kr_lo && key < kr_hi;
      sc[j] = in ? x : -kInf;
      mx = fmaxf(mx, sc[j]);
    }
    if (mx == -kInf) continue;
    const float alpha = m == -kInf ? 0.f : __expf(m - mx);
    float p[8], ps = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p[j] = sc[j] == -kInf ? 0.f : __expf(sc[j] - mx);
      ps += p[j];
    }
    l = l * alpha + ps;
    m = mx;
#pragma unroll
    for (int f = 0; f < OD; ++f) {
      float s_ = acc[f] * alpha;
#pragma unroll
      for (int j = 0; j < 8; ++j) s_ = __builtin_fmaf(p[j], vw[j * OD + f], s_);
      acc[f] = s_;
    }
    }
  }
  __syncthreads();  // the chunk buffers become the merge slots

  float (*part)[OD + 2][64] = reinterpret_cast<float (*)[OD + 2][64]>(sm);
  if (w > 0) {
#pragma unroll
    for (int f = 0; f < OD; ++f) part[w - 1][f][lane] = acc[f];
    part[w - 1][OD][lane] = m;
    part[w - 1][OD + 1][lane] = l;
  }
  __syncthreads();
  if (w != 0) return;
  float mw[NW - 1], M = m;
#pragma unroll
  for (int i = 0; i < NW - 1; ++i) {
    mw[i] = part[i][OD][lane];
    M = fmaxf(M, mw[i]);
  }
  float wt[NW];
  wt[0] = m == -kInf ? 0.f : __expf(m - M);
#pragma unroll
  for (int i = 0; i < NW - 1; ++i) wt[i + 1] = mw[i] == -kInf ? 0.f : __expf(mw[i] - M);
  float L = l * wt[0];
#pragma unroll
  for (int i = 0; i < NW - 1; ++i) L += part[i][OD + 1][lane] * wt[i + 1];
  if (!rin) return;
  const float inv = 1.0f / L;
  float* orow = a.o + b * a.o_sb + hq * a.o_sh + t * a.o_st;
#pragma unroll
  for (int f = 0; f < OD; ++f) {
    float v = acc[f] * wt[0];
#pragma unroll
    for (int i = 0; i < NW - 1; ++i) v += part[i][f][lane] * wt[i + 1];
    orow[f] = v * inv;
  }
  const int64_t grow = inst * a.t + t;
  if (a.m_out) a.m_out[grow] = M;
  if (a.den_out) a.den_out[grow] = L;
  if (a.lse_out) a.lse_out[grow] = M + __logf(L);
}

// The splits of a key-split forward merged per row (the associative
// online-softmax combine of zoo/attention.py:40-46): with M the largest of the
// splits' mused, o = sum_c o_c 2^((mused_c - M) c2) / den and den = sum_c den_c
// 2^((mused_c - M) c2); the artifacts as the unsplit kernel stores them. One
// thread per (row, 4 features).
template <typename T, int D>
__global__ __launch_bounds__(256) void flash_fwd_combine(FwdArgs a) {
  constexpr int TPR = D / 4;
  const int64_t gt = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t row = gt / TPR;
  const int f4 = static_cast<int>(gt % TPR);
  if (row >= a.plane) return;
  const int64_t P = a.plane, NS = a.nsplit;
  const float* mu = a.ws + NS * P * D;
  const float* mt = mu + NS * P;
  const float* dn = mt + NS * P;
  float M = -kInf, MT = -kInf;
  for (int c = 0; c < a.nsplit; ++c) {
    M = fmaxf(M, mu[c * P + row]);
    MT = fmaxf(MT, mt[c * P + row]);
  }
  float den = 0.f;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < a.nsplit; ++c) {
    const float m_c = mu[c * P + row];
    const float w = m_c > -kInf ? fast_exp2((m_c - M) * a.c2) : 0.f;  // an empty split adds nothing
    den += dn[c * P + row] * w;
    const f32x4 oc = *reinterpret_cast<const f32x4*>(a.ws + (c * P + row) * D + 4 * f4);
    acc += oc * w;
  }
  const float inv = den > 0.f ? 1.0f / den : 0.f;
  const int64_t inst = row / a.t, tq = row % a.t;
  const int64_t b = inst / a.heads_q, hq = inst % a.heads_q;
  uint16_t* orow = static_cast<uint16_t*>(a.o) + b * a.o_sb + hq * a.o_sh + tq * a.o_st + 4 * f4;
  *reinterpret_cast<u32x2*>(orow) = u32x2{pack2<T>(acc[0] * inv, acc[1] * inv), pack2<T>(acc[2] * inv, acc[3] * inv)};
  if (f4 == 0) {
    if (a.m_out) a.m_out[row] = MT * a.scale;
    if (a.den_out) a.den_out[row] = den * fast_exp2((M - MT) * a.c2);
    if (a.lse_out) a.lse_out[row] = M * a.scale + __logf(den);
  }
}

bool band_has_empty_row(int64_t T, int64_t S, int64_t lo, int64_t hi) {
  // row t has a live key iff max(0, t + lo) <= min(S - 1, t + hi); the
  // tightest rows are t = 0 (needs hi >= 0) and t = T - 1 (needs T-1+lo <= S-1)
  if (lo > hi) return true;
  if (hi < 0) return true;
  if (lo > INT64_MIN / 4 && (T - 1) + lo > S - 1) return true;
  return false;
}


template <typename T, int D>
void fwd_kernel(const FwdArgs& a, unsigned nblocks, hipStream_t st) {
  if (a.m_out || a.den_out)
    flash_fwd_m16<T, D, true><<<dim3(nblocks), F16Cfg<D>::THREADS, 0, st>>>(a);
  else
    flash_fwd_m16<T, D, false><<<dim3(nblocks), F16Cfg<D>::THREADS, 0, st>>>(a);
}

template <typename T, int D>
int launch_mfma(const FwdArgs& a, int64_t ninst, hipStream_t st) {
  using C = F16Cfg<D>;
  static_assert(C::LDS <= 64 * 1024, "the forward's static LDS fits one workgroup's limit");
  const int64_t nblk = ninst * a.nqb;
  PDH_REQUIRE(nblk <= INT32_MAX, PDH_EINVAL, "pdh_flash_fwd: grid too large (%lld workgroups)", (long long)nblk);
  FwdArgs aa = a;
  if (a.nsplit > 1) {
    const int64_t ntiles = (a.s + C::BN - 1) / C::BN;
    aa.split_tiles = static_cast<int>((ntiles + a.nsplit - 1) / a.nsplit);
    aa.xcd_remap = 0;
    PDH_REQUIRE(nblk * a.nsplit <= INT32_MAX, PDH_EINVAL, "pdh_flash_fwd_split: grid too large");
    fwd_kernel<T, D>(aa, static_cast<unsigned>(nblk * a.nsplit), st);
    int rc = check_launch("pdh_flash_fwd_split");
    if (rc) return rc;
    const int64_t nthr = a.plane * (D / 4);
    PDH_REQUIRE((nthr + 255) / 256 <= INT32_MAX, PDH_EINVAL, "pdh_flash_fwd_split: too many rows");
    flash_fwd_combine<T, D><<<dim3(static_cast<unsigned>((nthr + 255) / 256)), 256, 0, st>>>(aa);
    return check_launch("pdh_flash_fwd_split (combine)");
  }
  aa.xcd_remap = (nblk % 32 == 0 && a.nqb % 8 == 0) ? 3 : ((nblk % 8 == 0) ? 1 : 0);
  fwd_kernel<T, D>(aa, static_cast<unsigned>(nblk), st);
  return check_launch("pdh_flash_fwd");
}

}  // namespace
}  // namespace pdh

using namespace pdh;

namespace {

int flash_fwd_impl(const void* q, const void* k, const void* v, void* o, float* m_out, float* den_out,
                   float* lse_out, const pdh_attn_geom* gm, int dtype, float scale, float fill, int mask_kind,
                   int64_t band_lo, int64_t band_hi, int prune, int nsplit, void* ws, size_t ws_bytes,
                   void* stream) {
  PDH_REQUIRE(gm != nullptr, PDH_EINVAL, "pdh_flash_fwd: null geometry");
  const pdh_attn_geom G = *gm;
  PDH_REQUIRE(G.batch >= 0 && G.heads_q >= 1 && G.heads_kv >= 1 && G.t >= 0 && G.s >= 1 && G.e >= 1 && G.od >= 1,
              PDH_EINVAL, "pdh_flash_fwd: bad shape (batch %lld heads %lld/%lld t %lld s %lld e %lld od %lld)",
              (long long)G.batch, (long long)G.heads_q, (long long)G.heads_kv, (long long)G.t, (long long)G.s,
              (long long)G.e, (long long)G.od);
  PDH_REQUIRE(G.heads_q % G.heads_kv == 0, PDH_EINVAL,
              "pdh_flash_fwd: heads_q (%lld) must be a multiple of heads_kv (%lld)", (long long)G.heads_q,
              (long long)G.heads_kv);
  PDH_REQUIRE(mask_kind == PDH_MASK_NONE || mask_kind == PDH_MASK_BAND, PDH_EINVAL,
              "pdh_flash_fwd: unknown mask kind %d", mask_kind);
  PDH_REQUIRE(q && k && v && o, PDH_EINVAL, "pdh_flash_fwd: null tensor pointer");
  const int64_t ninst = G.batch * G.heads_q;
  if (ninst == 0 || G.t == 0) return PDH_OK;
  const int masked = mask_kind == PDH_MASK_BAND;
  const int prune_ok = prune && masked && !band_has_empty_row(G.t, G.s, band_lo, band_hi);
  hipStream_t st = as_stream(stream);

  if (dtype == PDH_F32) {
    PDH_REQUIRE(G.od <= 64 * kGenOdPerLane, PDH_EUNSUPPORTED, "pdh_flash_fwd: fp32 od > %d not supported",
                64 * kGenOdPerLane);
    GenArgs ga{static_cast<const float*>(q), static_cast<const float*>(k), static_cast<const float*>(v),
               static_cast<float*>(o), m_out, den_out, lse_out, G.heads_q, G.heads_kv, G.t, G.s, G.e, G.od,
               G.q_sb, G.q_sh, G.q_st, G.k_sb, G.k_sh, G.k_st, G.v_sb, G.v_sh, G.v_st, G.o_sb, G.o_sh, G.o_st,
               scale, fill, masked, band_lo, band_hi, prune_ok};
    const int64_t nrows = ninst * G.t;
    if (G.e == G.od && (G.e == 32 || G.e == 64)) {  // lanes are rows, K / V rows uniform
      const int64_t nqb = (G.t + 63) / 64;
      PDH_REQUIRE(ninst * nqb <= INT32_MAX && nqb <= INT32_MAX, PDH_EINVAL, "pdh_flash_fwd: too many rows");
      const dim3 grid(static_cast<unsigned>(ninst * nqb));
      static int cus = 0;  // compute units, read once (one device per process)
      if (cus == 0) cus = pdh_device_cus() > 0 ? pdh_device_cus() : 256;
      const bool small = ninst * nqb < cus;  // under one workgroup per compute unit
      if (G.e == 64 && small)
        flash_fwd_rows_f32_lds<64, 64, 8><<<grid, 512, 0, st>>>(ga, static_cast<int>(nqb));
      else if (G.e == 64)
        flash_fwd_rows_f32_lds<64, 64, 4><<<grid, 256, 0, st>>>(ga, static_cast<int>(nqb));
      else if (small)
        flash_fwd_rows_f32_lds<32, 32, 8><<<grid, 512, 0, st>>>(ga, static_cast<int>(nqb));
      else
        flash_fwd_rows_f32_lds<32, 32, 4><<<grid, 256, 0, st>>>(ga, static_cast<int>(nqb));
      return check_launch("pdh_flash_fwd");
    }
    PDH_REQUIRE((nrows + 3) / 4 <= INT32_MAX, PDH_EINVAL, "pdh_flash_fwd: too many rows");
    flash_fwd_generic_f32<<<dim3(static_cast<unsigned>((nrows + 3) / 4)), 256, 0, st>>>(ga, nrows);
    return check_launch("pdh_flash_fwd");
  }
  PDH_REQUIRE(dtype == PDH_BF16 || dtype == PDH_F16, PDH_EINVAL, "pdh_flash_fwd: unknown dtype %d", dtype);
  PDH_REQUIRE(scale > 0.f, PDH_EINVAL, "pdh_flash_fwd: the 16-bit kernels need scale > 0 (got %g)", (double)scale);
  PDH_REQUIRE(G.e == G.od && (G.e == 64 || G.e == 128), PDH_EUNSUPPORTED,
              "pdh_flash_fwd: 16-bit kernels need e == od in {64, 128} (got e %lld od %lld)", (long long)G.e,
              (long long)G.od);
  PDH_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o), PDH_EINVAL,
              "pdh_flash_fwd: q/k/v/o must be 16-byte aligned");
  PDH_REQUIRE(G.q_st % 8 == 0 && G.k_st % 8 == 0 && G.v_st % 8 == 0 && G.o_st % 8 == 0 && G.q_sh % 8 == 0 &&
                  G.k_sh % 8 == 0 && G.v_sh % 8 == 0 && G.o_sh % 8 == 0 && G.q_sb % 8 == 0 && G.k_sb % 8 == 0 &&
                  G.v_sb % 8 == 0 && G.o_sb % 8 == 0,
              PDH_EINVAL, "pdh_flash_fwd: 16-bit strides must be multiples of 8 elements");
  PDH_REQUIRE(G.t <= (1 << 29) && G.s <= (1 << 29), PDH_EINVAL, "pdh_flash_fwd: sequence too long (t, s <= 2^29)");
  PDH_REQUIRE(G.q_st < (1 << 24) && G.k_st < (1 << 24) && G.v_st < (1 << 24) && G.o_st < (1 << 24), PDH_EINVAL,
              "pdh_flash_fwd: row strides must be < 2^24 elements");
  PDH_REQUIRE(G.s * G.k_st * 2 < INT32_MAX && G.s * G.v_st * 2 < INT32_MAX, PDH_EINVAL,
              "pdh_flash_fwd: one instance's K / V rows must span < 2 GiB");
  FwdArgs a{q, k, v, o, m_out, den_out, lse_out, G.heads_q, G.heads_kv, G.t, G.s,
            G.q_sb, G.q_sh, G.q_st, G.k_sb, G.k_sh, G.k_st, G.v_sb, G.v_sh, G.v_st, G.o_sb, G.o_sh, G.o_st,
            scale, scale * kLog2e, fill / scale, masked, band_lo, band_hi, prune_ok,
            static_cast<int>((G.t + F16Cfg<128>::BM - 1) / F16Cfg<128>::BM), 0};
  {
    constexpr int64_t kBand32 = (int64_t{1} << 29) + 64;
    auto clamp32 = [](int64_t x) { return static_cast<int>(x < -kBand32 ? -kBand32 : (x > kBand32 ? kBand32 : x)); };
    a.band_lo32 = clamp32(band_lo);
    a.band_hi32 = clamp32(band_hi);
  }
  a.nsplit = 1;
  if (nsplit > 1) {
    const size_t need = pdh_flash_fwd_workspace(gm, nsplit);
    PDH_REQUIRE(ws != nullptr && ws_bytes >= need && aligned16(ws), PDH_EINVAL,
                "pdh_flash_fwd_split: ws must be 16-byte aligned and hold %zu bytes (got %zu)", need, ws_bytes);
    a.nsplit = nsplit;
    a.ws = static_cast<float*>(ws);
    a.plane = ninst * G.t;
  }
  if (dtype == PDH_BF16) {
    return G.e == 128 ? launch_mfma<__hip_bfloat16, 128>(a, ninst, st) : launch_mfma<__hip_bfloat16, 64>(a, ninst, st);
  }
  return G.e == 128 ? launch_mfma<_Float16, 128>(a, ninst, st) : launch_mfma<_Float16, 64>(a, ninst, st);
}

}  // namespace

extern "C" size_t pdh_flash_fwd_workspace(const pdh_attn_geom* gm, int nsplit) {
  if (gm == nullptr || nsplit <= 1) return 0;
  const int64_t rows = gm->batch * gm->heads_q * gm->t;
  return static_cast<size_t>(nsplit) * static_cast<size_t>(rows) * static_cast<size_t>(gm->od + 3) * sizeof(float);
}

extern "C" int pdh_flash_fwd(const void* q, const void* k, const void* v, void* o, float* m_out, float* den_out,
                             float* lse_out, const pdh_attn_geom* gm, int dtype, float scale, float fill,
                             int mask_kind, int64_t band_lo, int64_t band_hi, int prune, void* stream) {
  return flash_fwd_impl(q, k, v, o, m_out, den_out, lse_out, gm, dtype, scale, fill, mask_kind, band_lo, band_hi,
                        prune, 1, nullptr, 0, stream);
}

extern "C" int pdh_flash_fwd_split(const void* q, const void* k, const void* v, void* o, float* m_out,
                                   float* den_out, float* lse_out, const pdh_attn_geom* gm, int dtype, float scale,
                                   float fill, int mask_kind, int64_t band_lo, int64_t band_hi, int prune,
                                   int nsplit, void* ws, size_t ws_bytes, void* stream) {
  PDH_REQUIRE(nsplit >= 1 && nsplit <= 64, PDH_EINVAL, "pdh_flash_fwd_split: nsplit %d outside [1, 64]", nsplit);
  return flash_fwd_impl(q, k, v, o, m_out, den_out, lse_out, gm, dtype, scale, fill, mask_kind, band_lo, band_hi,
                        prune, nsplit, ws, ws_bytes, stream);
}
