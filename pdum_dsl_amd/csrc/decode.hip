// Decode attention, split over the key axis — the flash row at a handful of
// query rows per head, where the work is reading the key/value cache once.
//
// Pass 1 (decode_split): one workgroup per (batch, kv head, split). The
// heads_q / heads_kv query heads of the group (x t query rows) are packed
// into the workgroup, so every cache byte is read from HBM exactly once.
// Each wave sweeps 64-key blocks of its split: the block's K rows arrive with
// 128-bit coalesced loads into a wave-private LDS tile, each lane then owns
// one key and forms its scores with v_dot2 bf16/f16 dot products against the
// queries (LDS broadcast reads); the P V update runs with lanes owning feature
// pairs and each key's probability broadcast by v_readlane. Each wave carries
// its own online-softmax state; the four waves combine through LDS and the
// workgroup writes one partial (m, den, o) per query row.
//
// Pass 2 (decode_merge): one wave per query row folds the splits' partials
// with the associative online-softmax combine (flashsm, zoo/attention.py:40-46):
//   m = max(mL, mR); den = denL e^(mL-m) + denR e^(mR-m); o likewise.
#include "common.h"

namespace pdh {
namespace {

constexpr float kInf = __builtin_inff();
constexpr int kMaxNq = 8;  // query rows per workgroup (heads_q / heads_kv * t)

struct DecArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t heads_q, heads_kv, t, s;
  int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st;
  float c2;  // scale * log2(e)
  int nsplit;
  int64_t chunk;  // keys per split (multiple of 64)
  float* ws;      // [batch*heads_q*t][nsplit][2 + D]
};

template <typename T>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c);

template <>
__device__ __forceinline__ float dot2<__hip_bfloat16>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

template <>
__device__ __forceinline__ float dot2<_Float16>(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

template <int D>
struct DecCfg {
  static constexpr int KROW = D * 2 + 16;  // LDS bytes per K row (16 B pad)
  static constexpr int WAVE_LDS = 64 * KROW;
  static constexpr int DPL = D / 64;  // value features per lane in the P V update
};

template <typename T, int D, int NQ>
__global__ __launch_bounds__(256, 2) void decode_split(DecArgs a) {
  using C = DecCfg<D>;
  extern __shared__ __attribute__((aligned(16))) unsigned char dsm[];
  unsigned char* kl = dsm;                                         // 4 wave-private K tiles
  uint32_t* ql = reinterpret_cast<uint32_t*>(dsm + 4 * C::WAVE_LDS);  // staged query rows
  float* pl = reinterpret_cast<float*>(dsm + 4 * C::WAVE_LDS + kMaxNq * D * 2);  // [wave][NQ][64] probabilities
  float* red = reinterpret_cast<float*>(dsm);                      // reuses the K tiles at the end

  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const int R = static_cast<int>(a.heads_q / a.heads_kv);
  const int64_t nsplit = a.nsplit;
  const int64_t split = blockIdx.x % nsplit;
  const int64_t grp = blockIdx.x / nsplit;  // (batch, kv head)
  const int64_t b = grp / a.heads_kv, hk = grp % a.heads_kv;
  const uint16_t* kp = a.k + b * a.k_sb + hk * a.k_sh;
  const uint16_t* vp = a.v + b * a.v_sb + hk * a.v_sh;

  // stage the group's query rows (row qi = r * t + tq) in LDS as 16-bit pairs
  const int nq = R * static_cast<int>(a.t);
  for (int c = tid; c < NQ * D / 8; c += 256) {
    const int qi = c / (D / 8), ch = c % (D / 8);
    u32x4 val = {0u, 0u, 0u, 0u};
    if (qi < nq) {
      const int64_t hq = hk * R + qi / a.t, tq = qi % a.t;
      val = *reinterpret_cast<const u32x4*>(a.q + b * a.q_sb + hq * a.q_sh + tq * a.q_st + ch * 8);
    }
    *reinterpret_cast<u32x4*>(&ql[qi * D / 2 + ch * 4]) = val;
  }
  __syncthreads();

  const int64_t k_begin = split * a.chunk;
  const int64_t k_end = (k_begin + a.chunk < a.s) ? k_begin + a.chunk : a.s;
  unsigned char* kw = kl + w * C::WAVE_LDS;
  constexpr int CPR = D / 8;  // 16-byte chunks per K row

  float m[NQ], lp[NQ], o[NQ][C::DPL];
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    m[qi] = -kInf;
    lp[qi] = 0.f;
#pragma unroll
    for (int j = 0; j < C::DPL; ++j) o[qi][j] = 0.f;
  }

  // K block of 64 keys: global (coalesced, 64/CPR rows per instruction) -> registers -> LDS
  constexpr int RPI = 64 / CPR;  // rows per load instruction
  const uint32_t k_lane = static_cast<uint32_t>((lane / CPR) * a.k_st * 2 + (lane % CPR) * 16);
  const int k_lds = (lane / CPR) * C::KROW + (lane % CPR) * 16;
  u32x4 kreg[CPR];
  auto load_k = [&](int64_t kb0) {
#pragma unroll
    for (int i = 0; i < CPR; ++i) {
      const int64_t row0 = kb0 + i * RPI;  // uniform
      const bool ok = row0 + lane / CPR < k_end;
      kreg[i] = ok ? gload<u32x4>(kp + row0 * a.k_st, k_lane) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_k = [&]() {
#pragma unroll
    for (int i = 0; i < CPR; ++i) *reinterpret_cast<u32x4*>(kw + i * RPI * C::KROW + k_lds) = kreg[i];
  };

  const uint32_t v_lane = static_cast<uint32_t>(lane * C::DPL * 2);
  for (int64_t kb = k_begin + 64 * w; kb < k_end; kb += 256) {
    // this block's K rows and value rows in flight together; K lands in LDS first
    load_k(kb);
    uint32_t vreg[64];
    const int nk = (k_end - kb) < 64 ? static_cast<int>(k_end - kb) : 64;
    const uint16_t* vblk = vp + kb * a.v_st;
#pragma unroll
    for (int kk = 0; kk < 64; ++kk) {
      if constexpr (C::DPL == 2)
        vreg[kk] = kk < nk ? gload<uint32_t>(vblk + kk * a.v_st, v_lane) : 0u;
      else
        vreg[kk] = kk < nk ? static_cast<uint32_t>(gload<uint16_t>(vblk + kk * a.v_st, v_lane)) : 0u;
    }
    store_k();
    __builtin_amdgcn_wave_barrier();

    // lane = key: scores against every query row (K row from LDS, q broadcast).
    // The query offset is laundered each iteration so the compiler re-reads the
    // (loop-invariant) query rows from LDS instead of pinning them in registers.
    int qoff = 0;
    asm volatile("" : "+v"(qoff));
    const int64_t key = kb + lane;
    float sc[NQ];
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) sc[qi] = 0.f;
#pragma unroll 2
    for (int ch = 0; ch < CPR; ++ch) {
      const u32x4 kv = *reinterpret_cast<const u32x4*>(kw + lane * C::KROW + ch * 16);
#pragma unroll
      for (int qi = 0; qi < NQ; ++qi) {
        const u32x4 qv = *reinterpret_cast<const u32x4*>(&ql[qoff + qi * D / 2 + ch * 4]);
        float acc = sc[qi];
        acc = dot2<T>(kv.x, qv.x, acc);
        acc = dot2<T>(kv.y, qv.y, acc);
        acc = dot2<T>(kv.z, qv.z, acc);
        acc = dot2<T>(kv.w, qv.w, acc);
        sc[qi] = acc;
      }
    }
    float* pw = pl + w * NQ * 64;
#pragma unroll
    for (int qi = 0; qi < NQ; ++qi) {
      const float x = key < k_end ? sc[qi] * a.c2 : -kInf;
      const float mnew = fmaxf(m[qi], wave_max(x));
      const float alpha = fast_exp2(m[qi] - mnew);
      const float p = fast_exp2(x - mnew);
      pw[qi * 64 + lane] = p;
      lp[qi] = lp[qi] * alpha + p;
      m[qi] = mnew;
#pragma unroll
      for (int j = 0; j < C::DPL; ++j) o[qi][j] *= alpha;
    }
    __builtin_amdgcn_wave_barrier();
    // P V: lanes own features; each key's probability is an LDS broadcast read
#pragma unroll
    for (int k4 = 0; k4 < 64; k4 += 4) {
#pragma unroll
      for (int qi = 0; qi < NQ; ++qi) {
        const f32x4 pk = *reinterpret_cast<const f32x4*>(pw + qi * 64 + k4);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t vw = vreg[k4 + u];
          if constexpr (C::DPL == 2) {
            o[qi][0] = __builtin_fmaf(pk[u], lo_f32<T>(vw), o[qi][0]);
            o[qi][1] = __builtin_fmaf(pk[u], hi_f32<T>(vw), o[qi][1]);
          } else {
            o[qi][0] = __builtin_fmaf(pk[u], lo_f32<T>(vw), o[qi][0]);
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // per-wave state -> LDS (over the K tiles), then combine the four waves
  __syncthreads();
  constexpr int RS = 2 + D;  // floats per (wave, query row) record
#pragma unroll
  for (int qi = 0; qi < NQ; ++qi) {
    const float l = wave_sum(lp[qi]);
    float* rec = red + (w * NQ + qi) * RS;
    if (lane == 0) {
      rec[0] = m[qi];
      rec[1] = l;
    }
#pragma unroll
    for (int j = 0; j < C::DPL; ++j) rec[2 + lane * C::DPL + j] = o[qi][j];
  }
  __syncthreads();
  const int64_t q_row0 = (b * a.heads_q + hk * R) * a.t;  // first stats row of the group
  for (int c = tid; c < nq * RS; c += 256) {
    const int qi = c / RS, f = c % RS;
    float mm = -kInf;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) mm = fmaxf(mm, red[(ww * NQ + qi) * RS]);
    float val = 0.f;
    if (f == 0) {
      val = mm;
    } else {
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        const float mw = red[(ww * NQ + qi) * RS];
        const float sc = mw == -kInf ? 0.f : fast_exp2(mw - mm);
        val += red[(ww * NQ + qi) * RS + f] * sc;
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
int launch_decode(const DecArgs& a, int nq, int64_t nrows, uint16_t* o, float* lse, int64_t o_sb, int64_t o_sh,
                  int64_t o_st, int64_t groups, hipStream_t st) {
  const int64_t nblk = groups * a.nsplit;
  PDH_REQUIRE(nblk <= INT32_MAX, PDH_EINVAL, "pdh_attn_decode: grid too large");
  const dim3 grid(static_cast<unsigned>(nblk));
  const int lds = 4 * DecCfg<D>::WAVE_LDS + kMaxNq * D * 2 + 4 * kMaxNq * 64 * 4;
  auto go = [&](auto kern) {
    hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    kern<<<grid, 256, lds, st>>>(a);
  };
  if (nq <= 1)
    go(decode_split<T, D, 1>);
  else if (nq <= 2)
    go(decode_split<T, D, 2>);
  else if (nq <= 4)
    go(decode_split<T, D, 4>);
  else
    go(decode_split<T, D, 8>);
  int rc = check_launch("pdh_attn_decode (split)");
  if (rc) return rc;
  decode_merge<T, D><<<dim3(static_cast<unsigned>((nrows + 3) / 4)), 256, 0, st>>>(
      a.ws, o, lse, nrows, a.nsplit, a.heads_q, a.t, o_sb, o_sh, o_st);
  return check_launch("pdh_attn_decode (merge)");
}

}  // namespace
}  // namespace pdh

using namespace pdh;

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
  chunk = (chunk + 63) / 64 * 64;
  DecArgs a{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
            G.heads_q, G.heads_kv, G.t, G.s, G.q_sb, G.q_sh, G.q_st, G.k_sb, G.k_sh, G.k_st, G.v_sb, G.v_sh,
            G.v_st, scale * kLog2e, nsplit, chunk, static_cast<float*>(ws)};
  const int64_t nrows = G.batch * G.heads_q * G.t;
  const int64_t groups = G.batch * G.heads_kv;
  hipStream_t st = as_stream(stream);
  uint16_t* op = static_cast<uint16_t*>(o);
  if (dtype == PDH_BF16)
    return G.e == 128 ? launch_decode<__hip_bfloat16, 128>(a, (int)nq, nrows, op, lse_out, G.o_sb, G.o_sh, G.o_st,
                                                           groups, st)
                      : launch_decode<__hip_bfloat16, 64>(a, (int)nq, nrows, op, lse_out, G.o_sb, G.o_sh, G.o_st,
                                                          groups, st);
  return G.e == 128
             ? launch_decode<_Float16, 128>(a, (int)nq, nrows, op, lse_out, G.o_sb, G.o_sh, G.o_st, groups, st)
             : launch_decode<_Float16, 64>(a, (int)nq, nrows, op, lse_out, G.o_sb, G.o_sh, G.o_st, groups, st);
}
