// Kernel bodies of the map-chain and contraction-epilogue templates,
// parameterized on the element type (DT) and on the evaluator policy (Eval)
// that runs the pointwise program: the interpreter (ew.h) in the library
// build, or a generated straight-line evaluator in the kernels the library
// specializes at run time (hipRTC compiles this same header).
//
//   map_chain_body     one lane = EPT consecutive elements of the output's
//                      last dim
//   contract_mfma_body bf16 / f16: 4 waves of WM x WM (WM = 64: 2 x 2
//                      v_mfma_f32_32x32x16 per wave, 128 x 128 workgroup
//                      tiles; WM = 32: one product per wave, 64 x 64 tiles
//                      for grids too small to fill the chip), 64-wide k tiles
//                      copied HBM -> LDS by direct buffer loads, double
//                      buffered; XOR-swizzled 16-byte slots keep the b128
//                      operand reads conflict-free for 32- and 64-bank LDS;
//                      a and bt are read through batch and row strides
//   contract_f32_body  the fp32 column: 64 x 64 tiles, 4 x 4 outputs per
//                      lane, VALU fma, k tiles of 16 through LDS
// The epilogue program runs on the accumulators before the one store:
// out = epi(acc, operands); the output never makes an HBM round trip.
#pragma once

#include "ew.h"

namespace pdh {

struct ContractArgs {
  const void* a;
  const void* bt;
  void* out;
  int batch, m, n, k, kp;  // kp: the k extent read (a multiple of 64; columns k..kp-1 read as zero)
  int tiles_m, tiles_n;
  int dtype;
  long long sa_b, sa_r, sb_b, sb_r;  // element strides of a and bt: per batch, per row (k is contiguous)
};

constexpr int kBK = 64;
constexpr int kRowB = kBK * 2;  // LDS bytes per tile row (64 16-bit k values)
constexpr int kFT = 64, kFK = 16;  // fp32 column tiles

// k tiles in flight: the 128 x 128 variant double buffers (two workgroups
// per CU hide the load latency), the 64 x 64 one, which serves grids of
// under one workgroup per CU, keeps four k tiles in flight instead.
template <int WM>
constexpr int contract_stages() {
  return WM == 64 ? 2 : 4;
}

// LDS bytes of the WM variant: the operand tiles of 2 WM rows of every stage,
// or (epilogue) each wave's WM x WM accumulators with rows padded by 4 floats.
template <int WM>
constexpr int contract_lds() {
  return 2 * contract_stages<WM>() * (2 * WM) * kRowB > 4 * WM * (WM + 4) * 4
             ? 2 * contract_stages<WM>() * (2 * WM) * kRowB
             : 4 * WM * (WM + 4) * 4;
}

// s_waitcnt vmcnt(N) with the other counters at their maxima (N < 64).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

// ---------------------------------------------------------------- map chain

template <int DT, int EPT, typename Eval>
__device__ __forceinline__ void map_chain_body(const pdh_ew_program& p, const EwOperands& ops, void* out,
                                               uint32_t total) {
  const int ndim = p.ndim;
  // Rows that are whole multiples of a wave's 64 EPT elements: lane l takes
  // columns l, l + 64, ... of its wave's chunk, so every load and store
  // instruction covers 64 consecutive elements. Otherwise a lane takes EPT
  // consecutive columns.
  const bool wide = EPT > 1 && p.shape[ndim - 1] % (64 * EPT) == 0;
  const uint32_t gt = static_cast<uint32_t>(blockIdx.x) * 256u + threadIdx.x;
  const uint32_t i0 = wide ? (gt & ~63u) * EPT + (gt & 63u) : gt * EPT;
  const int es = wide ? 64 : 1;
  if (i0 >= total) return;
  int c[PDH_EW_MAX_DIMS] = {0, 0, 0, 0};
  uint32_t rem = i0;
#pragma unroll
  for (int d = PDH_EW_MAX_DIMS - 1; d >= 0; --d) {
    if (d < ndim) {
      const uint32_t ext = static_cast<uint32_t>(p.shape[d]);
      c[d] = static_cast<int>(rem % ext);
      rem /= ext;
    }
  }
  float acc[EPT], res[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) acc[e] = 0.f;
  Eval::template run<EPT>(p, ops, DT, c, acc, res, es);
  int off = 0;
#pragma unroll
  for (int d = 0; d < PDH_EW_MAX_DIMS; ++d)
    if (d < ndim) off += c[d] * static_cast<int>(p.out_stride[d]);
  const int step = es * static_cast<int>(p.out_stride[ndim - 1]);
#pragma unroll
  for (int e = 0; e < EPT; ++e) st_dt<DT>(out, off + e * step, res[e]);
}

// ------------------------------------------------------------- row reduce

// The ROWSUM and PLAIN contraction shapes: out[r] = epi(sum_k s(r, k)) where
// the summand program s runs over the lattice (row dims..., k dims...) (the
// last nk dims are reduced) and the epilogue program over the row dims with
// ACC = the sum. One wave per output element; with one k dim a lane takes
// k = lane, lane + 64, ... four at a time (every load covers 64 consecutive
// k), otherwise one k at a time with its coordinates decoded. The sum is fp32.
template <int DT, typename EvalS, typename EvalE>
__device__ __forceinline__ void reduce_rows_body(const pdh_ew_program& ps, const pdh_ew_program& pe,
                                                 const EwOperands& ops, void* out, int nk, int rows, int reducer) {
  const int lane = threadIdx.x & 63;
  const int r = static_cast<int>(blockIdx.x) * 4 + wave_id();
  if (r >= rows) return;
  const int nr = pe.ndim;
  int c[PDH_EW_MAX_DIMS] = {0, 0, 0, 0};
  int rem = r;
  for (int d = nr - 1; d >= 0; --d) {  // the row's coordinates (a unit lattice when nr = 0)
    const int ext = static_cast<int>(pe.shape[d]);
    c[d] = rem % ext;
    rem /= ext;
  }
  int ktot = 1;
  for (int d = nr; d < nr + nk; ++d) ktot *= static_cast<int>(ps.shape[d]);
  // reducer 0: sum; 1: max; 2: min (wave-uniform, so the branches do not diverge)
  auto comb = [reducer](float x, float y) { return reducer == 0 ? x + y : (reducer == 1 ? nan_max(x, y) : nan_min(x, y)); };
  float sum = reducer == 0 ? 0.f : (reducer == 1 ? -__builtin_inff() : __builtin_inff());
  if (nk == 1) {
    const float zero4[4] = {0.f, 0.f, 0.f, 0.f};
    int base = 0;
    for (; base + 256 <= ktot; base += 256) {
      c[nr] = base + lane;
      float res[4];
      EvalS::template run<4>(ps, ops, DT, c, zero4, res, 64);
      sum = comb(sum, comb(comb(res[0], res[1]), comb(res[2], res[3])));
    }
    for (int kk = base + lane; kk < ktot; kk += 64) {
      c[nr] = kk;
      const float z1[1] = {0.f};
      float r1[1];
      EvalS::template run<1>(ps, ops, DT, c, z1, r1, 1);
      sum = comb(sum, r1[0]);
    }
  } else {
    for (int kk = lane; kk < ktot; kk += 64) {
      int q = kk;
      for (int d = nr + nk - 1; d >= nr; --d) {
        const int ext = static_cast<int>(ps.shape[d]);
        c[d] = q % ext;
        q /= ext;
      }
      const float z1[1] = {0.f};
      float r1[1];
      EvalS::template run<1>(ps, ops, DT, c, z1, r1, 1);
      sum = comb(sum, r1[0]);
    }
  }
  if (reducer == 0) {
    sum = wave_total(sum);
  } else {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum = comb(sum, __shfl_xor(sum, off, 64));
  }
  if (lane == 0) {
    const float a1[1] = {sum};
    float r1[1];
    int co[PDH_EW_MAX_DIMS] = {c[0], c[1], c[2], c[3]};
    for (int d = nr; d < PDH_EW_MAX_DIMS; ++d) co[d] = 0;
    EvalE::template run<1>(pe, ops, DT, co, a1, r1, 1);
    long long off = 0;
    for (int d = 0; d < nr; ++d) off += static_cast<long long>(co[d]) * pe.out_stride[d];
    st_dt<DT>(out, off, r1[0]);
  }
}

// ------------------------------------------------------------ contraction

// 16-byte slot of chunk c (0..7) of tile row r is c ^ swz_gemm(r): conflict
// free for the b128 reads below (16 lanes = rows r0..r0+15 at one chunk on
// 64 banks, 8 lanes on 32 banks).
__device__ __forceinline__ int swz_gemm(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Epilogue for EPT consecutive columns col0.. of one row. Elements past the
// output are neither computed nor stored, so every operand read stays inside
// its view: a full group runs once for all EPT columns, a ragged right edge
// one column at a time.
template <int DT, int EPT, typename Eval>
__device__ __forceinline__ void contract_epilogue(const pdh_ew_program& p, const EwOperands& ops, const ContractArgs& a,
                                                  int b, int row, int col0, const float (&acc)[EPT]) {
  if (row >= a.m) return;
  const long long rbase = static_cast<long long>(b) * p.out_stride[0] + static_cast<long long>(row) * p.out_stride[1];
  if (col0 + EPT <= a.n) {
    const int c0[PDH_EW_MAX_DIMS] = {b, row, col0, 0};
    float res[EPT];
    Eval::template run<EPT>(p, ops, DT, c0, acc, res, 1);
    if constexpr (EPT == 4) {
      const long long o0 = rbase + col0;
      if (p.out_stride[2] == 1 && (o0 & 3) == 0 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0) {
        // four consecutive, aligned outputs: one 16-byte (fp32) or 8-byte (16-bit) store
        if constexpr (DT == PDH_F32) {
          *reinterpret_cast<f32x4*>(static_cast<float*>(a.out) + o0) = f32x4{res[0], res[1], res[2], res[3]};
        } else {
          uint16_t h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = DT == PDH_BF16 ? f32_to_bf16(res[e]) : f32_to_f16(res[e]);
          *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.out) + o0) =
              u32x2{h[0] | (static_cast<uint32_t>(h[1]) << 16), h[2] | (static_cast<uint32_t>(h[3]) << 16)};
        }
        return;
      }
    }
#pragma unroll
    for (int e = 0; e < EPT; ++e) st_dt<DT>(a.out, rbase + static_cast<long long>(col0 + e) * p.out_stride[2], res[e]);
    return;
  }
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    if (col0 + e >= a.n) break;
    const int c1[PDH_EW_MAX_DIMS] = {b, row, col0 + e, 0};
    const float a1[1] = {acc[e]};
    float r1[1];
    Eval::template run<1>(p, ops, DT, c1, a1, r1, 1);
    st_dt<DT>(a.out, rbase + static_cast<long long>(col0 + e) * p.out_stride[2], r1[0]);
  }
}

template <int DT, int WM, typename Eval>
__device__ __forceinline__ void contract_mfma_body(const ContractArgs& a, const pdh_ew_program& p,
                                                   const EwOperands& ops, unsigned char* smem) {
  constexpr int BM = 2 * WM;          // workgroup tile (rows of a and of bt)
  constexpr int TI = WM / 32;         // 32 x 32 products per wave and dim
  constexpr int TILEB = BM * kRowB;   // LDS bytes per operand tile
  constexpr int BLK = BM / 8 / 4;     // 8-row direct-load blocks per wave and operand
  constexpr int ACCP = WM + 4;        // accumulator row pitch in LDS (floats)
  constexpr int NS = contract_stages<WM>();
  constexpr int PER_STAGE = 2 * BLK;  // direct loads per wave and k tile
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id(), r32 = lane & 31, g = lane >> 5;
  (void)tid;
  const int wy = w >> 1, wx = w & 1;  // the wave's WM x WM quadrant
  const int per = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x / per, rest = blockIdx.x % per;
  const int m0 = (rest / a.tiles_n) * BM, n0 = (rest % a.tiles_n) * BM;
  const uint32_t rowa = static_cast<uint32_t>(a.sa_r) * 2u, rowbb = static_cast<uint32_t>(a.sb_r) * 2u;
  const uint16_t* abase = static_cast<const uint16_t*>(a.a) + b * a.sa_b;
  const uint16_t* bbase = static_cast<const uint16_t*>(a.bt) + b * a.sb_b;
  // the buffers end after the batch slice's last row: rows past m (n) read as zero
  const rsrc_t ar = make_rsrc(abase, (static_cast<uint32_t>(a.m) - 1u) * rowa + static_cast<uint32_t>(a.kp) * 2u);
  const rsrc_t br = make_rsrc(bbase, (static_cast<uint32_t>(a.n) - 1u) * rowbb + static_cast<uint32_t>(a.kp) * 2u);

  // direct loads: 1 KB = 8 tile rows; lane i -> row i / 8, slot i % 8 holds chunk slot ^ swz(row)
  const int lrow = lane >> 3, slot = lane & 7;
  uint32_t offa[2], offb[2];  // tile-row parity of the 8-row block decides the swizzle of row 8 j + lrow
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const uint32_t sl = static_cast<uint32_t>((slot ^ swz_gemm(8 * par + lrow)) << 4);
    offa[par] = lrow * rowa + sl;
    offb[par] = lrow * rowbb + sl;
  }
  auto stage = [&](int kt, int buf) {  // stage buf: a tile at 2 buf, bt tile at 2 buf + 1
    unsigned char* at = smem + (2 * buf) * TILEB;
    unsigned char* bt = smem + (2 * buf + 1) * TILEB;
    const uint32_t koff = static_cast<uint32_t>(kt) * kBK * 2u;
#pragma unroll
    for (int i = 0; i < BLK; ++i) {
      const int blk = 4 * i + w;  // BM / 8 blocks of 8 rows per operand tile
      dma16(ar, at + blk * 1024, offa[blk & 1], static_cast<uint32_t>(m0 + 8 * blk) * rowa + koff);
      dma16(br, bt + blk * 1024, offb[blk & 1], static_cast<uint32_t>(n0 + 8 * blk) * rowbb + koff);
    }
  };
  // operand reads: row (WM q + 32 t + r32) of a tile, chunk 2 ks + g
  int rd[TI][4];
#pragma unroll
  for (int t = 0; t < TI; ++t)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int row = 32 * t + r32;  // + WM q: a multiple of 16 rows, so the swizzle is unchanged
      rd[t][ks] = row * kRowB + (((2 * ks + g) ^ swz_gemm(row)) << 4);
    }

  f32x16 acc[TI][TI];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TI; ++j) acc[i][j] = f32x16{};

  const int nkt = a.kp / kBK;
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (s < nkt) stage(s, s);
  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = kt % NS;
    // tile kt has landed when at most the NS - 2 later tiles' loads are outstanding
    if (kt + NS - 2 < nkt)
      wait_vmcnt<(NS - 2) * PER_STAGE>();
    else
      wait_vmcnt0();
    __syncthreads();  // every wave's loads of tile kt are done; everyone finished tile kt - 1
    if (kt + NS - 1 < nkt) stage(kt + NS - 1, (kt + NS - 1) % NS);
    const unsigned char* at = smem + (2 * buf) * TILEB + WM * wy * kRowB;
    const unsigned char* bt = smem + (2 * buf + 1) * TILEB + WM * wx * kRowB;
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 af[TI], bf[TI];
#pragma unroll
      for (int t = 0; t < TI; ++t) {
        af[t] = *reinterpret_cast<const u32x4*>(at + rd[t][ks]);
        bf[t] = *reinterpret_cast<const u32x4*>(bt + rd[t][ks]);
      }
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TI; ++j) acc[i][j] = mfma32_dt<DT>(af[i], bf[j], acc[i][j]);
    }
    __builtin_amdgcn_s_setprio(0);
  }
  wait_vmcnt0();

  // The epilogue reads the accumulators back from LDS (each wave its own
  // WM x WM block, rows padded by 4 floats): one runtime loop, four
  // consecutive columns per lane, so one copy of the program's code.
  // Accumulator v of tile (i, j) is row 32 i + 8 (v / 4) + 4 g + v % 4,
  // column 32 j + r32 of the wave's block.
  __syncthreads();  // every wave is done with the operand tiles
  float* blkf = reinterpret_cast<float*>(smem) + w * WM * ACCP;
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TI; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) blkf[(32 * i + 8 * (v >> 2) + 4 * g + (v & 3)) * ACCP + 32 * j + r32] = acc[i][j][v];
  __builtin_amdgcn_wave_barrier();  // the block is wave-private: in-order LDS, no workgroup barrier
  for (int it = 0; it < WM * WM / 256; ++it) {
    const int idx = it * 256 + lane * 4;
    const int row = idx / WM, col = idx % WM;
    const f32x4 av4 = *reinterpret_cast<const f32x4*>(blkf + row * ACCP + col);
    const float av[4] = {av4[0], av4[1], av4[2], av4[3]};
    contract_epilogue<DT, 4, Eval>(p, ops, a, b, m0 + WM * wy + row, n0 + WM * wx + col, av);
  }
}

template <typename Eval>
__device__ __forceinline__ void contract_f32_body(const ContractArgs& a, const pdh_ew_program& p,
                                                  const EwOperands& ops) {
  __shared__ float as[kFK][kFT + 4];  // k-major copies of the two 64-row tiles
  __shared__ float bs[kFK][kFT + 4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int per = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x / per, rest = blockIdx.x % per;
  const int m0 = (rest / a.tiles_n) * kFT, n0 = (rest % a.tiles_n) * kFT;
  const float* abase = static_cast<const float*>(a.a) + b * a.sa_b;
  const float* bbase = static_cast<const float*>(a.bt) + b * a.sb_b;
  const int lr = tid >> 2, lc = (tid & 3) * 4;  // this lane's tile row and 4 k values per load
  float acc[4][4] = {};
  for (int k0 = 0; k0 < a.kp; k0 += kFK) {
    const int am = m0 + lr, bn = n0 + lr;
    f32x4 av = {0.f, 0.f, 0.f, 0.f}, bv = {0.f, 0.f, 0.f, 0.f};
    if (am < a.m) av = *reinterpret_cast<const f32x4*>(abase + am * a.sa_r + k0 + lc);
    if (bn < a.n) bv = *reinterpret_cast<const f32x4*>(bbase + bn * a.sb_r + k0 + lc);
    __syncthreads();  // the previous tile's reads are done
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      as[lc + j][lr] = av[j];
      bs[lc + j][lr] = bv[j];
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kFK; ++kk) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(&as[kk][4 * ty]);
      const f32x4 y = *reinterpret_cast<const f32x4*>(&bs[kk][4 * tx]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(x[i], y[j], acc[i][j]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float av[4] = {acc[i][0], acc[i][1], acc[i][2], acc[i][3]};
    contract_epilogue<PDH_F32, 4, Eval>(p, ops, a, b, m0 + 4 * ty + i, n0 + 4 * tx, av);
  }
}

}  // namespace pdh
