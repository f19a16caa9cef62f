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
//   contract_split_body fp32 on the bf16 matrix cores: the same tiles, fp32
//                      k tiles of 32 loaded to registers, split into two or
//                      three bf16 planes in LDS, and the cross products of
//                      the planes summed by v_mfma_f32_32x32x16_bf16 (3 or 6
//                      products per term; 6 is fp32 grade)
//   contract_f32_body  fp32 by VALU fma: 64 x 64 tiles, 4 x 4 outputs per
//                      lane, k tiles of 16 through LDS
// The epilogue program runs on the accumulators before the one store:
// out = epi(acc, operands); the output never makes an HBM round trip.
#pragma once

#include "ew.h"

namespace pdh {

struct ContractArgs {
  const void* a;
  const void* bt;
  void* out;
  // k: the k columns of a batch entry that hold data; kp: the columns one k
  // slice reads (a multiple of 64). The fp32 bodies read columns at or past k
  // as zero; the 16-bit body reads them, so its operands are zero-padded.
  int batch, m, n, k, kp;
  int tiles_m, tiles_n;
  int dtype;
  long long sa_b, sa_r, sb_b, sb_r;  // element strides of a and bt: per batch, per row
  // k slices per batch entry: batch index bb is (bb / ksplit, slice bb % ksplit),
  // and slice s reads k columns [s kp, (s + 1) kp) (1: no split)
  int ksplit;
  // element strides along k: 1 (k contiguous), or, for the fp32 bodies only,
  // any stride of an operand whose rows are contiguous (row stride 1)
  long long sa_k, sb_k;
  // -1: out receives the epilogue's values. 0 / 1 / 2 (fp32 bodies only): out
  // receives their sum / max / min over each run of 32 output columns, fp32
  // [batch][m][ceil(n / 32)] (row partials; columns past n take no part)
  int rowred;
  // nonzero: a (pro_a) / bt (pro_b) is not read but computed in the k loop by
  // its prologue program (ContractPro; the split and VALU bodies of a prologue
  // kernel only; with 16-bit storage both operands are computed, their LOADs
  // reading 16-bit values, and the split body runs with one bf16 plane)
  int pro_a, pro_b;
};

// An operand prologue: the program whose value at lattice point
// (batch entry, row, k column) is the operand's element there (rows are the
// m rows for a, the n rows for bt; k counts from the entry's first column,
// across k slices), and the pointer table its LOADs index.
struct ContractPro {
  pdh_ew_program p;
  EwOperands ops;
};

template <typename A, typename B>
struct SameT {
  static constexpr bool value = false;
};
template <typename A>
struct SameT<A, A> {
  static constexpr bool value = true;
};

// Four values of a computed operand at (batch entry, row rc, k columns
// k0 .. k0 + 3 from the entry's first), those at or past kend zero; every
// evaluated coordinate is clamped below kend, so every LOAD stays inside the
// views the host checked. Whole runs take one evaluator call of four.
template <typename PE>
__device__ __forceinline__ void pro_run4(const ContractPro& pr, int dt, int be, int rc, int k0, int kend,
                                         float (&x)[4]) {
  int c0[PDH_EW_MAX_DIMS] = {be, rc, k0, 0};
  if (k0 + 3 < kend) {
    const float zacc[4] = {0.f, 0.f, 0.f, 0.f};
    PE::template run<4>(pr.p, pr.ops, dt, c0, zacc, x, 1);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c0[2] = k0 + j < kend ? k0 + j : kend - 1;
      float y[1];
      const float z1[1] = {0.f};
      PE::template run<1>(pr.p, pr.ops, dt, c0, z1, y, 1);
      x[j] = k0 + j < kend ? y[0] : 0.f;
    }
  }
}

// The interpreter's form, called rather than inlined: the interpreter is a
// large switch, and the prologue kernels call it from many places.
static __device__ __attribute__((noinline)) void pro_interp4(const ContractPro& pr, int dt, int be, int rc, int k0,
                                                              int kend, float (&x)[4]) {
  pro_run4<InterpEval>(pr, dt, be, rc, k0, kend, x);
}

// Four operand values of one row, k columns kk .. kk + 3 of batch index bb's
// slice, by prologue evaluator PE; columns at or past kin and rows at or past
// rows are zero (the row is clamped into the lattice for the evaluation).
template <typename PE>
__device__ __forceinline__ f32x4 pro_eval4(const ContractPro& pr, const ContractArgs& a, int bb, int row, int rows,
                                           int kk, int kin) {
  const int rc = row < rows ? row : rows - 1;
  const int kbase = (bb % a.ksplit) * a.kp;
  float x[4];
  if constexpr (SameT<PE, InterpEval>::value)
    pro_interp4(pr, a.dtype, bb / a.ksplit, rc, kbase + kk, kbase + kin, x);
  else
    pro_run4<PE>(pr, a.dtype, bb / a.ksplit, rc, kbase + kk, kbase + kin, x);
  const bool rin = row < rows;
  return f32x4{rin ? x[0] : 0.f, rin ? x[1] : 0.f, rin ? x[2] : 0.f, rin ? x[3] : 0.f};
}

// Element offsets of batch index bb's a and bt rows (the batch entry's, moved
// to its k slice).
__device__ __forceinline__ long long contract_off_a(const ContractArgs& a, int bb) {
  return static_cast<long long>(bb / a.ksplit) * a.sa_b + static_cast<long long>(bb % a.ksplit) * a.kp * a.sa_k;
}
__device__ __forceinline__ long long contract_off_b(const ContractArgs& a, int bb) {
  return static_cast<long long>(bb / a.ksplit) * a.sb_b + static_cast<long long>(bb % a.ksplit) * a.kp * a.sb_k;
}

// Columns of batch index bb's k slice that hold data (kp or fewer; <= 0 past k).
__device__ __forceinline__ int contract_kvalid(const ContractArgs& a, int bb) {
  return a.k - (bb % a.ksplit) * a.kp;
}

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
  // (An evaluator that reads fp32 operands four at a time, Eval::kVec, takes
  // EPT consecutive columns per lane instead: one 16-byte access per operand.)
  const bool wide = !Eval::kVec && EPT > 1 && p.shape[ndim - 1] % (64 * EPT) == 0;
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
  if constexpr (Eval::kVec && DT == PDH_F32 && EPT == 4) {
    if (step == 1) {
      *reinterpret_cast<f32x4u*>(static_cast<float*>(out) + off) = f32x4u{res[0], res[1], res[2], res[3]};
      return;
    }
  }
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

// The same reduce when the summand's operands run along the outputs, not
// along k (a bias gradient: sum over tokens of dy[t, f], f contiguous). A
// workgroup of 1024 lanes takes 16 consecutive outputs: lane (q, c), c the
// output column, q = 0..63 its k lane, sums k = 4 q' + ... in runs of four
// (k = kk, kk + 64, kk + 128, kk + 192 per evaluation, four loads in flight),
// so every load instruction covers 16 consecutive outputs at 4 consecutive
// k. The 64 partials of each output are combined in LDS in a fixed order.
// nk is 1.
constexpr int kColOut = 16, kColK = 64;  // outputs per workgroup, k lanes per output

template <int DT, typename EvalS, typename EvalE>
__device__ __forceinline__ void reduce_cols_body(const pdh_ew_program& ps, const pdh_ew_program& pe,
                                                 const EwOperands& ops, void* out, int rows, int reducer,
                                                 float* part) {
  const int tid = threadIdx.x, col = tid % kColOut, q = tid / kColOut;
  const int r = static_cast<int>(blockIdx.x) * kColOut + col;
  const int nr = pe.ndim;
  auto comb = [reducer](float x, float y) { return reducer == 0 ? x + y : (reducer == 1 ? nan_max(x, y) : nan_min(x, y)); };
  const float ident = reducer == 0 ? 0.f : (reducer == 1 ? -__builtin_inff() : __builtin_inff());
  float sum = ident;
  int c[PDH_EW_MAX_DIMS] = {0, 0, 0, 0};
  if (r < rows) {
    int rem = r;
    for (int d = nr - 1; d >= 0; --d) {
      const int ext = static_cast<int>(pe.shape[d]);
      c[d] = rem % ext;
      rem /= ext;
    }
    const int ktot = static_cast<int>(ps.shape[nr]);
    const float zero4[4] = {0.f, 0.f, 0.f, 0.f};
    int base = 0;
    for (; base + 4 * kColK <= ktot; base += 4 * kColK) {
      c[nr] = base + q;
      float res[4];
      EvalS::template run<4>(ps, ops, DT, c, zero4, res, kColK);
      sum = comb(sum, comb(comb(res[0], res[1]), comb(res[2], res[3])));
    }
    const float z1[1] = {0.f};
    for (int kk = base + q; kk < ktot; kk += kColK) {
      c[nr] = kk;
      float r1[1];
      EvalS::template run<1>(ps, ops, DT, c, z1, r1, 1);
      sum = comb(sum, r1[0]);
    }
  }
  part[tid] = sum;
  __syncthreads();
  if (q == 0 && r < rows) {
    float tot = part[col];
    for (int j = 1; j < kColK; ++j) tot = comb(tot, part[col + kColOut * j]);
    const float a1[1] = {tot};
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

// Four fp32 as four 16-bit elements, round to nearest even by the hardware
// conversion (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32: one instruction a pair).
template <int DT>
__device__ __forceinline__ u32x2 pack4_16(const float (&r)[4]) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  if constexpr (DT == PDH_BF16) {
    typedef __bf16 h2 __attribute__((ext_vector_type(2)));
    return u32x2{__builtin_bit_cast(uint32_t, __builtin_convertvector(f2{r[0], r[1]}, h2)),
                 __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{r[2], r[3]}, h2))};
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return u32x2{__builtin_bit_cast(uint32_t, __builtin_convertvector(f2{r[0], r[1]}, h2)),
                 __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{r[2], r[3]}, h2))};
  }
}

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
    if constexpr (EPT % 4 == 0) {
      const long long o0 = rbase + col0;
      if (p.out_stride[2] == 1 && (o0 & 3) == 0 && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0) {
        // runs of four consecutive, aligned outputs: one 16-byte (fp32) or
        // 8-byte (16-bit) store each; 16-bit runs of eight that start on a
        // multiple of 8: one 16-byte store each
        if constexpr (DT == PDH_F32) {
#pragma unroll
          for (int q = 0; q < EPT / 4; ++q)
            *reinterpret_cast<f32x4*>(static_cast<float*>(a.out) + o0 + 4 * q) =
                f32x4{res[4 * q], res[4 * q + 1], res[4 * q + 2], res[4 * q + 3]};
        } else {
          uint16_t* o = static_cast<uint16_t*>(a.out) + o0;
          u32x2 pk[EPT / 4];
#pragma unroll
          for (int q = 0; q < EPT / 4; ++q) {
            const float r4[4] = {res[4 * q], res[4 * q + 1], res[4 * q + 2], res[4 * q + 3]};
            pk[q] = pack4_16<DT>(r4);
          }
          if (EPT % 8 == 0 && (o0 & 7) == 0) {
#pragma unroll
            for (int q = 0; q < EPT / 8; ++q)
              *reinterpret_cast<u32x4*>(o + 8 * q) = u32x4{pk[2 * q][0], pk[2 * q][1], pk[2 * q + 1][0], pk[2 * q + 1][1]};
          } else {
#pragma unroll
            for (int q = 0; q < EPT / 4; ++q) *reinterpret_cast<u32x2*>(o + 4 * q) = pk[q];
          }
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

// Row partials. RED is the reduction (0 sum, 1 max, 2 min, as reduce_rows:
// NaN-propagating), or kRedRuntime to read it from the arguments (the
// interpreter kernels serve both stores).
constexpr int kRedRuntime = 3;

template <int RED>
__device__ __forceinline__ int red_kind(const ContractArgs& a) {
  return RED == kRedRuntime ? a.rowred : RED;
}

__device__ __forceinline__ float red_identity(int r) {
  return r == 0 ? 0.f : (r == 1 ? -__builtin_inff() : __builtin_inff());
}

__device__ __forceinline__ float red_combine(int r, float x, float y) {
  return r == 0 ? x + y : (r == 1 ? nan_max(x, y) : nan_min(x, y));
}

// The reduction r of the epilogue's values at columns col0 .. col0 + 3 of one
// row; the identity for a row past m and for columns past n (whose operands
// are never read).
template <int DT, typename Eval>
__device__ __forceinline__ float epilogue_reduced4(const pdh_ew_program& p, const EwOperands& ops,
                                                   const ContractArgs& a, int r, int b, int row, int col0,
                                                   const float (&acc)[4]) {
  float v = red_identity(r);
  if (row >= a.m) return v;
  if (col0 + 4 <= a.n) {
    const int c0[PDH_EW_MAX_DIMS] = {b, row, col0, 0};
    float res[4];
    Eval::template run<4>(p, ops, DT, c0, acc, res, 1);
#pragma unroll
    for (int e = 0; e < 4; ++e) v = red_combine(r, v, res[e]);
    return v;
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (col0 + e >= a.n) break;
    const int c1[PDH_EW_MAX_DIMS] = {b, row, col0 + e, 0};
    const float a1[1] = {acc[e]};
    float r1[1];
    Eval::template run<1>(p, ops, DT, c1, a1, r1, 1);
    v = red_combine(r, v, r1[0]);
  }
  return v;
}

// Eight consecutive lanes that hold 32 consecutive columns of one row
// (columns col0.., col0 of the first a multiple of 32) combine their values by
// a fixed butterfly, and the first writes the run's partial. Every lane of
// the wave calls this (cross-lane moves).
__device__ __forceinline__ void store_row_partial(const ContractArgs& a, int r, int b, int row, int col0, float v) {
  v = red_combine(r, v, __shfl_xor(v, 1, 64));
  v = red_combine(r, v, __shfl_xor(v, 2, 64));
  v = red_combine(r, v, __shfl_xor(v, 4, 64));
  if ((threadIdx.x & 7) == 0 && row < a.m && col0 < a.n) {
    const long long nblk = (a.n + 31) / 32;
    static_cast<float*>(a.out)[(static_cast<long long>(b) * a.m + row) * nblk + col0 / 32] = v;
  }
}

// The epilogue of a WM x WM-per-wave workgroup tile: the accumulators go
// through LDS (each wave its own WM x WM block, rows padded by 4 floats) and
// come back four consecutive columns per lane, so one runtime loop holds one
// copy of the program's code. Accumulator v of tile (i, j) is row
// 32 i + 8 (v / 4) + 4 g + v % 4, column 32 j + r32 of the wave's block. The
// caller has passed a barrier after its last read of the operand tiles.
template <int DT, int WM, typename Eval, int RED = -1>
__device__ __forceinline__ void contract_store(const ContractArgs& a, const pdh_ew_program& p, const EwOperands& ops,
                                               unsigned char* smem, const f32x16 (&acc)[WM / 32][WM / 32], int b,
                                               int m0, int n0) {
  constexpr int TI = WM / 32, ACCP = WM + 4;
  const int lane = threadIdx.x & 63, w = wave_id(), r32 = lane & 31, g = lane >> 5;
  const int wy = w >> 1, wx = w & 1;
  float* blkf = reinterpret_cast<float*>(smem) + w * WM * ACCP;
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TI; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) blkf[(32 * i + 8 * (v >> 2) + 4 * g + (v & 3)) * ACCP + 32 * j + r32] = acc[i][j][v];
  __builtin_amdgcn_wave_barrier();  // the block is wave-private: in-order LDS, no workgroup barrier
  if constexpr (RED < 0) {
    // EPT consecutive outputs of one row per lane and evaluator call: the
    // call issues every operand load of its EPT outputs before it waits, so
    // a wave waits on operand latency WM * WM / (64 EPT) times, not WM * WM / 256.
    // fp32 outputs keep runs of four: a lane's 16 bytes, so eight lanes write a
    // row's 128 bytes with one instruction (longer fp32 runs split every store
    // instruction into 32-byte pieces of 32 rows, measured 30-40% slower).
    constexpr int RUN = DT == PDH_F32 ? 4 : Eval::kStoreRun;
    constexpr int EPT = RUN < WM * WM / 64 ? RUN : WM * WM / 64;
    static_assert(WM % EPT == 0 && WM * WM % (64 * EPT) == 0, "runs stay in one row and cover the block");
    for (int it = 0; it < WM * WM / (64 * EPT); ++it) {
      const int idx = it * 64 * EPT + lane * EPT;
      const int row = idx / WM, col = idx % WM;
      float av[EPT];
#pragma unroll
      for (int q = 0; q < EPT / 4; ++q) {
        const f32x4 v4 = *reinterpret_cast<const f32x4*>(blkf + row * ACCP + col + 4 * q);
        av[4 * q] = v4[0];
        av[4 * q + 1] = v4[1];
        av[4 * q + 2] = v4[2];
        av[4 * q + 3] = v4[3];
      }
      contract_epilogue<DT, EPT, Eval>(p, ops, a, b, m0 + WM * wy + row, n0 + WM * wx + col, av);
    }
  } else {
    for (int it = 0; it < WM * WM / 256; ++it) {
      const int idx = it * 256 + lane * 4;
      const int row = idx / WM, col = idx % WM;
      const f32x4 av4 = *reinterpret_cast<const f32x4*>(blkf + row * ACCP + col);
      const float av[4] = {av4[0], av4[1], av4[2], av4[3]};
      // row partials: lanes 8 q .. 8 q + 7 hold 32 consecutive columns of one row
      const int r = red_kind<RED>(a);
      if (r >= 0) {
        const int grow = m0 + WM * wy + row, gcol = n0 + WM * wx + col;
        store_row_partial(a, r, b, grow, gcol, epilogue_reduced4<DT, Eval>(p, ops, a, r, b, grow, gcol, av));
      } else {
        contract_epilogue<DT, 4, Eval>(p, ops, a, b, m0 + WM * wy + row, n0 + WM * wx + col, av);
      }
    }
  }
}

template <int DT, int WM, typename Eval>
__device__ __forceinline__ void contract_mfma_body(const ContractArgs& a, const pdh_ew_program& p,
                                                   const EwOperands& ops, unsigned char* smem) {
  constexpr int BM = 2 * WM;          // workgroup tile (rows of a and of bt)
  constexpr int TI = WM / 32;         // 32 x 32 products per wave and dim
  constexpr int TILEB = BM * kRowB;   // LDS bytes per operand tile
  constexpr int BLK = BM / 8 / 4;     // 8-row direct-load blocks per wave and operand
  constexpr int NS = contract_stages<WM>();
  constexpr int PER_STAGE = 2 * BLK;  // direct loads per wave and k tile
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id(), r32 = lane & 31, g = lane >> 5;
  (void)tid;
  const int wy = w >> 1, wx = w & 1;  // the wave's WM x WM quadrant
  const int per = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x / per, rest = blockIdx.x % per;
  const int m0 = (rest / a.tiles_n) * BM, n0 = (rest % a.tiles_n) * BM;
  const uint32_t rowa = static_cast<uint32_t>(a.sa_r) * 2u, rowbb = static_cast<uint32_t>(a.sb_r) * 2u;
  const uint16_t* abase = static_cast<const uint16_t*>(a.a) + contract_off_a(a, b);
  const uint16_t* bbase = static_cast<const uint16_t*>(a.bt) + contract_off_b(a, b);
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
  static_assert(contract_lds<WM>() >= 2 * NS * TILEB, "operand stages fit the LDS block");
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
    u32x4 af[4][TI], bf[4][TI];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int t = 0; t < TI; ++t) {
        af[ks][t] = *reinterpret_cast<const u32x4*>(at + rd[t][ks]);
        bf[ks][t] = *reinterpret_cast<const u32x4*>(bt + rd[t][ks]);
      }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TI; ++j) acc[i][j] = mfma32_dt<DT>(af[ks][i], bf[ks][j], acc[i][j]);
    }
    __builtin_amdgcn_s_setprio(0);
  }
  wait_vmcnt0();
  __syncthreads();  // every wave is done with the operand tiles
  contract_store<DT, WM, Eval>(a, p, ops, smem, acc, b, m0, n0);
}

// One 64 x 64 block (rows m0.., columns n0..) of batch b by fp32 VALU fma,
// 4 x 4 outputs per lane, k tiles of 16 staged k-major through LDS (as, bs:
// kFK x (kFT + 4) floats each), and the epilogue applied. Every lane of the
// workgroup takes part (barriers inside).
template <typename Eval, int RED = -1, typename ProA = InterpEval, typename ProB = InterpEval, bool PRO = false,
          int ODT = PDH_F32>
__device__ __forceinline__ void f32_valu_block(const ContractArgs& a, const pdh_ew_program& p, const EwOperands& ops,
                                               int b, int m0, int n0, float (*as)[kFT + 4], float (*bs)[kFT + 4],
                                               const ContractPro* pra = nullptr, const ContractPro* prb = nullptr) {
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const float* abase = static_cast<const float*>(a.a) + contract_off_a(a, b);
  const float* bbase = static_cast<const float*>(a.bt) + contract_off_b(a, b);
  const int lr = tid >> 2, lc = (tid & 3) * 4;  // this lane's tile row and 4 k values per load
  const int kin = contract_kvalid(a, b) < a.kp ? contract_kvalid(a, b) : a.kp;  // columns past it read as zero
  float acc[4][4] = {};
  for (int k0 = 0; k0 < a.kp; k0 += kFK) {
    const int am = m0 + lr, bn = n0 + lr;
    f32x4 av = {0.f, 0.f, 0.f, 0.f}, bv = {0.f, 0.f, 0.f, 0.f};
    if (PRO && (a.pro_a || a.pro_b)) {  // computed operands (the other one read in place)
      if (a.pro_a)
        av = pro_eval4<ProA>(*pra, a, b, am, a.m, k0 + lc, kin);
      else
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const long long kk = k0 + lc + j;
          if (am < a.m && kk < kin) av[j] = abase[am * a.sa_r + kk * a.sa_k];
        }
      if (a.pro_b)
        bv = pro_eval4<ProB>(*prb, a, b, bn, a.n, k0 + lc, kin);
      else
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const long long kk = k0 + lc + j;
          if (bn < a.n && kk < kin) bv[j] = bbase[bn * a.sb_r + kk * a.sb_k];
        }
    } else if (a.sa_k == 1 && a.sb_k == 1 && k0 + kFK <= kin) {  // k contiguous, whole tile
      if (am < a.m) av = *reinterpret_cast<const f32x4u*>(abase + am * a.sa_r + k0 + lc);
      if (bn < a.n) bv = *reinterpret_cast<const f32x4u*>(bbase + bn * a.sb_r + k0 + lc);
    } else {  // any strides, one element at a time
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const long long kk = k0 + lc + j;
        if (am < a.m && kk < kin) av[j] = abase[am * a.sa_r + kk * a.sa_k];
        if (bn < a.n && kk < kin) bv[j] = bbase[bn * a.sb_r + kk * a.sb_k];
      }
    }
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
  __syncthreads();  // as / bs may be reused by the caller
  const int r = RED < 0 ? -1 : red_kind<RED>(a);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float av[4] = {acc[i][0], acc[i][1], acc[i][2], acc[i][3]};
    if (r >= 0)  // lanes 16 ty + 8 h .. + 7 hold columns 32 h .. 32 h + 31 of row 4 ty + i
      store_row_partial(a, r, b, m0 + 4 * ty + i, n0 + 4 * tx,
                        epilogue_reduced4<PDH_F32, Eval>(p, ops, a, r, b, m0 + 4 * ty + i, n0 + 4 * tx, av));
    else
      contract_epilogue<ODT, 4, Eval>(p, ops, a, b, m0 + 4 * ty + i, n0 + 4 * tx, av);
  }
}

template <typename Eval, int RED = kRedRuntime, typename ProA = InterpEval, typename ProB = InterpEval, bool PRO = false>
__device__ __forceinline__ void contract_f32_body(const ContractArgs& a, const pdh_ew_program& p,
                                                  const EwOperands& ops, const ContractPro* pra = nullptr,
                                                  const ContractPro* prb = nullptr) {
  __shared__ float as[kFK][kFT + 4];  // k-major copies of the two 64-row tiles
  __shared__ float bs[kFK][kFT + 4];
  const int per = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x / per, rest = blockIdx.x % per;
  f32_valu_block<Eval, RED, ProA, ProB, PRO>(a, p, ops, b, (rest / a.tiles_n) * kFT, (rest % a.tiles_n) * kFT, as, bs,
                                         pra, prb);
}

// ------------------------------------------- fp32 on the bf16 matrix cores

// An fp32 value as a sum of bf16 terms, each the round-to-nearest of what the
// previous ones leave: x = x1 + x2 + x3 + r with |x2| <= 2^-8 |x1|,
// |x3| <= 2^-16 |x1|, |r| <= 2^-24 |x1| (each difference is exact in fp32).
// The contraction keeps the cross products above 2^-24 |a b|: NSPLIT = 3
// takes (1,1) (1,2) (2,1), about 2^-16 of each product; NSPLIT = 6 adds
// (2,2) (1,3) (3,1), about 2^-24: fp32 grade. NSPLIT = 1 keeps x1 alone:
// bf16-rounded operands with fp32 accumulation and fp32 storage (the
// numerics of a bf16 autocast). A non-finite x1 (x itself non-finite, or
// |x| above the largest bf16) is taken alone.
template <int NSPLIT>
constexpr int split_planes() {
  static_assert(NSPLIT == 1 || NSPLIT == 3 || NSPLIT == 6, "NSPLIT is 1, 3 or 6");
  return NSPLIT == 1 ? 1 : (NSPLIT == 3 ? 2 : 3);
}
constexpr int kSBK = 32;          // fp32 k values per k tile
constexpr int kSRowB = kSBK * 2;  // bytes per row of one bf16 plane: four 16-byte slots of 8 k values

// LDS bytes of the split variant: PL planes of both operand tiles, or the
// epilogue's accumulator blocks.
template <int WM, int NSPLIT>
constexpr int split_lds() {
  return split_planes<NSPLIT>() * 2 * (2 * WM) * kSRowB > 4 * WM * (WM + 4) * 4
             ? split_planes<NSPLIT>() * 2 * (2 * WM) * kSRowB
             : 4 * WM * (WM + 4) * 4;
}

// Tile row r of a plane is stored as plane row r ^ swz_split(r) (a
// permutation within each aligned group of 16 rows), its slot s (0..3) at
// s ^ swz_split(r). The b128 operand reads of 16 consecutive rows at one slot
// then cover all 64 banks once, and so do the 8-byte writes of both load
// layouts: (rows 8 w .. 8 w + 7 (+ 32 c), all 8 chunks) for a k-contiguous
// operand and (rows 4 q + c, q = 8 w .. 8 w + 7, all 8 chunks) for a
// rows-contiguous one.
__device__ __forceinline__ int swz_split(int r) { return (r >> 2) & 3; }
template <bool B>
struct BoolC {  // a compile-time flag passed to generic lambdas
  static constexpr bool value = B;
};
template <typename T>
struct TypeC {  // a type passed to generic lambdas
  using type = T;
};
__device__ __forceinline__ int split_off(int r, int ch) {  // byte offset of (row r, 8-byte chunk ch) in a plane
  return (r ^ swz_split(r)) * kSRowB + (((ch >> 1) ^ swz_split(r)) << 4) + ((ch & 1) << 3);
}

typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
typedef float f32x2_v __attribute__((ext_vector_type(2)));

// Two fp32 as two bf16 (lo = x, hi = y), round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t rne_bf16x2(float x, float y) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_v{x, y}, bf16x2_v));
}

// Four consecutive fp32 of one row -> PL planes of four bf16 each. The
// leading terms' magnitude bits (bf16, so an unsigned 16-bit compare orders
// them as values) are folded into two packed running extrema per lane: big,
// the largest (0x7f80 and above: an inf or NaN, x itself non-finite or above
// the largest bf16), and low, the smallest of (bits - 1) (wrapping, so an
// exact zero is 0xffff): below 0x0d7f is a nonzero term under 2^-100, whose
// lower planes would fall into the subnormal range and lose the bits that make
// the split fp32 grade. split_odd reads the verdict off the pair once per
// block. The planes of such values are not used (the block recomputes in
// fp32), so the remainders are formed without guards.
typedef unsigned short u16x2_v __attribute__((ext_vector_type(2)));
template <int PL>
__device__ __forceinline__ void split4(u32x4 v, u32x2 (&out)[PL], u16x2_v& big, u16x2_v& low) {
  float r[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float x0 = __uint_as_float(v[2 * j]), x1 = __uint_as_float(v[2 * j + 1]);
    const uint32_t h = rne_bf16x2(x0, x1);
    out[0][j] = h;
    const u16x2_v mag = __builtin_bit_cast(u16x2_v, h & 0x7fff7fffu);
    big = __builtin_elementwise_max(big, mag);
    if constexpr (PL > 1) {
      low = __builtin_elementwise_min(low, mag - u16x2_v{1, 1});
      r[2 * j] = x0 - __uint_as_float(h << 16);
      r[2 * j + 1] = x1 - __uint_as_float(h & 0xffff0000u);
    }
  }
#pragma unroll
  for (int p = 1; p < PL; ++p)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t h = rne_bf16x2(r[2 * j], r[2 * j + 1]);
      out[p][j] = h;
      if (p + 1 < PL) {
        r[2 * j] -= __uint_as_float(h << 16);
        r[2 * j + 1] -= __uint_as_float(h & 0xffff0000u);
      }
    }
}

template <int PL>
__device__ __forceinline__ bool split_odd(u16x2_v big, u16x2_v low) {
  const bool nonfinite = big[0] >= 0x7f80 || big[1] >= 0x7f80;
  return PL > 1 ? nonfinite || low[0] < 0x0d7f || low[1] < 0x0d7f : nonfinite;
}

// LAY bit 0: a is rows-contiguous (k strided), bit 1: bt is; otherwise k is
// contiguous. The host picks LAY from the strides (sa_k, sb_k != 1).
// PRO: a prologue kernel (ContractArgs::pro_a / pro_b name the operands its
// evaluators ProA / ProB compute; such an operand takes the k-contiguous lane
// layout, its LAY bit clear).
template <int DT, int WM, int NSPLIT, int LAY, typename Eval, int RED = kRedRuntime, typename ProA = InterpEval,
          typename ProB = InterpEval, bool PRO = false>
__device__ __forceinline__ void contract_split_body(const ContractArgs& a, const pdh_ew_program& p,
                                                    const EwOperands& ops, unsigned char* smem,
                                                    const ContractPro* pra = nullptr,
                                                    const ContractPro* prb = nullptr) {
  constexpr int BM = 2 * WM, TI = WM / 32, PL = split_planes<NSPLIT>();
  constexpr int PLANEB = BM * kSRowB;  // one plane of one operand tile
  constexpr int CH = BM / 32;          // 16-byte fp32 chunks per lane and operand: rows (tid / 8) + 32 c
  static_assert(split_lds<WM, NSPLIT>() >= PL * 2 * PLANEB, "planes fit the LDS block");
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id(), r32 = lane & 31, g = lane >> 5;
  const int wy = w >> 1, wx = w & 1;
  const int per = a.tiles_m * a.tiles_n;
  const int b = blockIdx.x / per, rest = blockIdx.x % per;
  const int m0 = (rest / a.tiles_n) * BM, n0 = (rest % a.tiles_n) * BM;
  const float* abase = static_cast<const float*>(a.a) + contract_off_a(a, b);
  const float* bbase = static_cast<const float*>(a.bt) + contract_off_b(a, b);
  // Columns at or past kin read as zero, and so do rows past m (n): such
  // loads take the lane offset kOOB, past every buffer's extent (the host
  // keeps every in-bounds byte offset under 2^31), so the hardware returns
  // zero without a memory access.
  constexpr uint32_t kOOB = 0x80000000u;
  constexpr bool mna = (LAY & 1) != 0, mnb = (LAY & 2) != 0;
  int kin = contract_kvalid(a, b);
  kin = kin < 0 ? 0 : (kin > a.kp ? a.kp : kin);
  const uint32_t rowa = static_cast<uint32_t>(a.sa_r) * 4u, rowbb = static_cast<uint32_t>(a.sb_r) * 4u;
  const uint32_t ka = static_cast<uint32_t>(a.sa_k) * 4u, kb = static_cast<uint32_t>(a.sb_k) * 4u;
  auto extent = [&](bool mn, int rows, uint32_t rowb, uint32_t kbs) -> uint32_t {
    if (kin == 0) return 0u;
    return mn ? static_cast<uint32_t>(kin - 1) * kbs + static_cast<uint32_t>(rows) * 4u
              : static_cast<uint32_t>(rows - 1) * rowb + static_cast<uint32_t>(kin) * 4u;
  };
  const rsrc_t ar = make_rsrc(abase, extent(mna, a.m, rowa, ka));
  const rsrc_t br = make_rsrc(bbase, extent(mnb, a.n, rowbb, kb));

  // A lane holds four consecutive k values (columns 4 ch .. 4 ch + 3 of the
  // tile) of CH rows. k-contiguous: lane tid = 8 q + ch, rows q + 32 c, one
  // 16-byte load each (8 lanes read a row's 128-byte line). Rows-contiguous:
  // rows CH q + c, four loads of CH consecutive rows (one per column),
  // re-paired in registers; with CH = 4, lane tid = 8 q + ch as before, with
  // CH = 2, 16 lanes of a wave cover 32 rows (so every load instruction reads
  // whole 128-byte lines): q = 16 (w % 2) + lane % 16, ch = 4 (w / 2) + lane / 16.
  const int lq = tid >> 3, lch = tid & 7;
  const int mq = CH == 4 ? lq : 16 * (w & 1) + (lane & 15), mch = CH == 4 ? lch : 4 * (w >> 1) + (lane >> 4);
  int wra[CH], wrb[CH];  // where chunk c lands in a plane
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    wra[c] = mna ? split_off(CH * mq + c, mch) : split_off(lq + 32 * c, lch);
    wrb[c] = mnb ? split_off(CH * mq + c, mch) : split_off(lq + 32 * c, lch);
  }
  // operand reads: row 32 t + r32 (+ WM q) of a plane, slot 2 ks + g
  int rd[TI][2];
#pragma unroll
  for (int t = 0; t < TI; ++t)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {  // + WM q rows: a multiple of 32, which the permutation keeps
      const int row = 32 * t + r32;
      rd[t][ks] = (row ^ swz_split(row)) * kSRowB + (((2 * ks + g) ^ swz_split(row)) << 4);
    }

  typedef uint32_t u32xCH __attribute__((ext_vector_type(CH)));
  auto fetch1 = [&](auto mn_c, auto edge_c, const rsrc_t& r, uint32_t rowb, uint32_t kbs, int r0, int rows, int kt,
                    u32x4(&v)[CH]) {
    constexpr bool MN = decltype(mn_c)::value, EDGE = decltype(edge_c)::value;
    const int k0 = kt * kSBK;
    if constexpr (!MN) {
      const uint32_t vo = static_cast<uint32_t>(lq) * rowb + static_cast<uint32_t>(lch) * 16u;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const bool rin = r0 + lq + 32 * c < rows;
        const uint32_t so = static_cast<uint32_t>(r0 + 32 * c) * rowb + static_cast<uint32_t>(k0) * 4u;
        if constexpr (!EDGE) {
          v[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, rin ? vo : kOOB, so, 0));
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            v[c][j] = __builtin_amdgcn_raw_buffer_load_b32(
                r, (rin && k0 + 4 * lch + j < kin) ? vo + 4u * j : kOOB, so, 0);
        }
      }
    } else {
      const int rv = rows - (r0 + CH * mq);  // rows of this lane's group inside the operand
      const uint32_t vo = static_cast<uint32_t>(CH * mq) * 4u + static_cast<uint32_t>(4 * mch) * kbs;
      u32xCH ld[4];
      if (rv >= CH) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t so = static_cast<uint32_t>(r0) * 4u + static_cast<uint32_t>(k0 + j) * kbs;
          const bool ok = !EDGE || k0 + 4 * mch + j < kin;
          if constexpr (CH == 4)
            ld[j] = __builtin_bit_cast(u32xCH, __builtin_amdgcn_raw_buffer_load_b128(r, ok ? vo : kOOB, so, 0));
          else
            ld[j] = __builtin_bit_cast(u32xCH, __builtin_amdgcn_raw_buffer_load_b64(r, ok ? vo : kOOB, so, 0));
        }
      } else {  // the last rows of the operand: one element at a time
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t so = static_cast<uint32_t>(r0) * 4u + static_cast<uint32_t>(k0 + j) * kbs;
          const bool ok = !EDGE || k0 + 4 * mch + j < kin;
#pragma unroll
          for (int i = 0; i < CH; ++i)
            ld[j][i] = __builtin_amdgcn_raw_buffer_load_b32(r, (ok && i < rv) ? vo + 4u * i : kOOB, so, 0);
        }
      }
#pragma unroll
      for (int c = 0; c < CH; ++c) v[c] = u32x4{ld[0][c], ld[1][c], ld[2][c], ld[3][c]};
    }
  };
  u32x4 va[CH], vb[CH];
  // a computed operand: the lane's k-contiguous chunks (rows r0 + lq + 32 c,
  // columns 4 lch .. 4 lch + 3 of the k tile) by its prologue
  auto compute1 = [&](auto pe_c, const ContractPro& pr, int r0, int rows, int kt, u32x4(&v)[CH]) {
    using PE = typename decltype(pe_c)::type;
#pragma unroll
    for (int c = 0; c < CH; ++c)
      v[c] = __builtin_bit_cast(u32x4, pro_eval4<PE>(pr, a, b, r0 + lq + 32 * c, rows, kt * kSBK + 4 * lch, kin));
  };
  auto fetch = [&](int kt, auto edge_c) {
    if (PRO && a.pro_a)
      compute1(TypeC<ProA>{}, *pra, m0, a.m, kt, va);
    else
      fetch1(BoolC<mna>{}, edge_c, ar, rowa, ka, m0, a.m, kt, va);
    if (PRO && a.pro_b)
      compute1(TypeC<ProB>{}, *prb, n0, a.n, kt, vb);
    else
      fetch1(BoolC<mnb>{}, edge_c, br, rowbb, kb, n0, a.n, kt, vb);
  };

  f32x16 acc[TI][TI];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TI; ++j) acc[i][j] = f32x16{};

  // the k tiles that hold data; the last one masked per element when ragged
  const int nkt = (kin + kSBK - 1) / kSBK;
  const bool ragged = kin % kSBK != 0;
  auto fetch_tile = [&](int kt) {
    if (ragged && kt == nkt - 1)
      fetch(kt, BoolC<true>{});
    else
      fetch(kt, BoolC<false>{});
  };
  // the extrema of this lane's leading terms (split4): a non-finite one (an
  // inf, a NaN, |x| above the largest bf16), or with lower planes a nonzero
  // one below 2^-100, sends the block to the fp32 path
  u16x2_v big = u16x2_v{0, 0}, low = u16x2_v{0xffff, 0xffff};
  if (nkt > 0) fetch_tile(0);
  for (int kt = 0; kt < nkt; ++kt) {
    __syncthreads();  // every wave is done reading the planes of tile kt - 1
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      u32x2 pa[PL], pb[PL];
      split4<PL>(va[c], pa, big, low);
      split4<PL>(vb[c], pb, big, low);
#pragma unroll
      for (int pl = 0; pl < PL; ++pl) {
        *reinterpret_cast<u32x2*>(smem + (2 * pl) * PLANEB + wra[c]) = pa[pl];
        *reinterpret_cast<u32x2*>(smem + (2 * pl + 1) * PLANEB + wrb[c]) = pb[pl];
      }
    }
    if (kt + 1 < nkt) fetch_tile(kt + 1);  // in flight under this tile's products
    __syncthreads();                  // the planes of tile kt are in LDS
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x4 af[PL][TI], bf[PL][TI];
#pragma unroll
      for (int pl = 0; pl < PL; ++pl)
#pragma unroll
        for (int t = 0; t < TI; ++t) {
          af[pl][t] = *reinterpret_cast<const u32x4*>(smem + (2 * pl) * PLANEB + WM * wy * kSRowB + rd[t][ks]);
          bf[pl][t] = *reinterpret_cast<const u32x4*>(smem + (2 * pl + 1) * PLANEB + WM * wx * kSRowB + rd[t][ks]);
        }
      // smallest terms first; (pa, pb) plane pairs
      constexpr int NP = NSPLIT;
      constexpr int PA[6] = {NSPLIT == 6 ? 2 : (NSPLIT == 3 ? 1 : 0), 0, NSPLIT == 6 ? 1 : 0, 1, 0, 0};
      constexpr int PB[6] = {0, NSPLIT == 6 ? 2 : 1, NSPLIT == 6 ? 1 : 0, 0, 1, 0};
#pragma unroll
      for (int q = 0; q < NP; ++q)
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int j = 0; j < TI; ++j) acc[i][j] = mfma32_dt<PDH_BF16>(af[PA[q]][i], bf[PB[q]][j], acc[i][j]);
    }
    __builtin_amdgcn_s_setprio(0);
  }
  __syncthreads();  // every wave is done with the planes
  // A plane product of an inf with an exact zero of the other operand's
  // lower plane is NaN where IEEE arithmetic gives the inf: a workgroup that
  // loaded any non-finite (or bf16-overflowing) value recomputes its tile by
  // fp32 VALU fma instead, so such values behave as in fp32.
  int* flags = reinterpret_cast<int*>(smem);
  const bool wave_odd = __builtin_amdgcn_ballot_w64(split_odd<PL>(big, low)) != 0;  // every lane votes
  if (lane == 0) flags[w] = wave_odd ? 1 : 0;
  __syncthreads();
  const bool slow = (flags[0] | flags[1] | flags[2] | flags[3]) != 0;
  __syncthreads();  // every wave has read the flags before the LDS is reused
  if (slow) {
    float(*as)[kFT + 4] = reinterpret_cast<float(*)[kFT + 4]>(smem);
    float(*bs)[kFT + 4] = reinterpret_cast<float(*)[kFT + 4]>(smem + kFK * (kFT + 4) * 4);
#pragma unroll 1
    for (int ij = 0; ij < (BM / kFT) * (BM / kFT); ++ij)  // one copy of the block's code
      f32_valu_block<Eval, RED, ProA, ProB, PRO, DT>(a, p, ops, b, m0 + kFT * (ij / (BM / kFT)),
                                                 n0 + kFT * (ij % (BM / kFT)), as, bs, pra, prb);
    return;
  }
  contract_store<DT, WM, Eval, RED>(a, p, ops, smem, acc, b, m0, n0);
}

}  // namespace pdh
