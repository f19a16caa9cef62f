// The map-chain and contraction-epilogue templates (fusion.py:844-854 and
// fusion.py:159-324): the C ABI, its validation, and the launch of either
// the runtime-specialized kernels (jit.hip) or the interpreter kernels
// (the bodies of contract_core.h with the program interpreter of ew.h).
#include <atomic>
#include <type_traits>

#include "common.h"
#include "contract_core.h"
#include "jit.h"

namespace pdh {
namespace {

// The interpreter kernels: the bodies of contract_core.h with InterpEval.

template <int DT, int EPT>
__global__ __launch_bounds__(256) void map_chain_kernel(pdh_ew_program p, EwOperands ops, void* out, uint32_t total) {
  map_chain_body<DT, EPT, InterpEval>(p, ops, out, total);
}

template <int DT>
__global__ __launch_bounds__(256, 2) void contract_mfma(ContractArgs a, pdh_ew_program p, EwOperands ops) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[contract_lds<64>()];
  contract_mfma_body<DT, 64, InterpEval>(a, p, ops, smem);
}

template <int DT>
__global__ __launch_bounds__(256, 2) void contract_mfma_small(ContractArgs a, pdh_ew_program p, EwOperands ops) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[contract_lds<32>()];
  contract_mfma_body<DT, 32, InterpEval>(a, p, ops, smem);
}

__global__ __launch_bounds__(256) void contract_f32(ContractArgs a, pdh_ew_program p, EwOperands ops) {
  contract_f32_body<InterpEval>(a, p, ops);
}

template <int NSPLIT, int LAY>
__global__ __launch_bounds__(256, 2) void contract_split(ContractArgs a, pdh_ew_program p, EwOperands ops) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[split_lds<64, NSPLIT>()];
  contract_split_body<PDH_F32, 64, NSPLIT, LAY, InterpEval>(a, p, ops, smem);
}

template <int NSPLIT, int LAY>
__global__ __launch_bounds__(256, 2) void contract_split_small(ContractArgs a, pdh_ew_program p, EwOperands ops) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[split_lds<32, NSPLIT>()];
  contract_split_body<PDH_F32, 32, NSPLIT, LAY, InterpEval>(a, p, ops, smem);
}

// The prologue kernels: the same bodies with operands computed in the k
// loop by the interpreter (ContractArgs::pro_a / pro_b say which).
__global__ __launch_bounds__(256) void contract_f32_pro(ContractArgs a, pdh_ew_program p, EwOperands ops,
                                                        ContractPro pa, ContractPro pb) {
  contract_f32_body<InterpEval, kRedRuntime, InterpEval, InterpEval, true>(a, p, ops, &pa, &pb);
}

template <int NSPLIT, int LAY>
__global__ __launch_bounds__(256, 2) void contract_split_pro(ContractArgs a, pdh_ew_program p, EwOperands ops,
                                                             ContractPro pa, ContractPro pb) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[split_lds<64, NSPLIT>()];
  contract_split_body<PDH_F32, 64, NSPLIT, LAY, InterpEval, kRedRuntime, InterpEval, InterpEval, true>(a, p, ops, smem,
                                                                                                        &pa, &pb);
}

template <int NSPLIT, int LAY>
__global__ __launch_bounds__(256, 2) void contract_split_pro_small(ContractArgs a, pdh_ew_program p, EwOperands ops,
                                                                   ContractPro pa, ContractPro pb) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[split_lds<32, NSPLIT>()];
  contract_split_body<PDH_F32, 32, NSPLIT, LAY, InterpEval, kRedRuntime, InterpEval, InterpEval, true>(a, p, ops, smem,
                                                                                                        &pa, &pb);
}

// 16-bit storage with computed operands: the split body with one bf16 plane
// (the operands' values rounded to bf16, as a materialized 16-bit operand is),
// both operands computed by prologues that read 16-bit leaves.
template <int DT>
__global__ __launch_bounds__(256, 2) void contract_split16_pro(ContractArgs a, pdh_ew_program p, EwOperands ops,
                                                               ContractPro pa, ContractPro pb) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[split_lds<64, 1>()];
  contract_split_body<DT, 64, 1, 0, InterpEval, -1, InterpEval, InterpEval, true>(a, p, ops, smem, &pa, &pb);
}

template <int DT>
__global__ __launch_bounds__(256, 2) void contract_split16_pro_small(ContractArgs a, pdh_ew_program p, EwOperands ops,
                                                                     ContractPro pa, ContractPro pb) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[split_lds<32, 1>()];
  contract_split_body<DT, 32, 1, 0, InterpEval, -1, InterpEval, InterpEval, true>(a, p, ops, smem, &pa, &pb);
}

// The interpreter's split kernel for (mode, operand layouts), by value; with
// prologues (pro non-null) the prologue kernel.
template <int NSPLIT>
void launch_split(bool small, int lay, dim3 grid, hipStream_t st, const ContractArgs& ca, const pdh_ew_program& epi,
                  const EwOperands& ops, const ContractPro* pro = nullptr) {
  auto go = [&](auto lay_c) {
    constexpr int L = decltype(lay_c)::value;
    if (pro != nullptr) {
      if (small)
        contract_split_pro_small<NSPLIT, L><<<grid, 256, 0, st>>>(ca, epi, ops, pro[0], pro[1]);
      else
        contract_split_pro<NSPLIT, L><<<grid, 256, 0, st>>>(ca, epi, ops, pro[0], pro[1]);
    } else if (small)
      contract_split_small<NSPLIT, L><<<grid, 256, 0, st>>>(ca, epi, ops);
    else
      contract_split<NSPLIT, L><<<grid, 256, 0, st>>>(ca, epi, ops);
  };
  if (lay == 0)
    go(std::integral_constant<int, 0>{});
  else if (lay == 1)
    go(std::integral_constant<int, 1>{});
  else if (lay == 2)
    go(std::integral_constant<int, 2>{});
  else
    go(std::integral_constant<int, 3>{});
}

template <int DT>
__global__ __launch_bounds__(256) void reduce_rows_kernel(pdh_ew_program ps, pdh_ew_program pe, EwOperands ops,
                                                          void* out, int nk, int rows, int reducer) {
  reduce_rows_body<DT, InterpEval, InterpEval>(ps, pe, ops, out, nk, rows, reducer);
}

template <int DT>
__global__ __launch_bounds__(1024) void reduce_cols_kernel(pdh_ew_program ps, pdh_ew_program pe, EwOperands ops,
                                                           void* out, int nk, int rows, int reducer) {
  __shared__ float part[kColOut * kColK];
  (void)nk;
  reduce_cols_body<DT, InterpEval, InterpEval>(ps, pe, ops, out, rows, reducer, part);
}

// The column variant pays when k is the strided dim: one reduced dim, every
// summand operand strided (or broadcast) along it, and one of them
// contiguous along the last output dim.
bool reduce_by_columns(const pdh_ew_program& ps, int nk, int nr, int64_t rows) {
  if (nk != 1 || nr < 1 || rows < kColOut || ps.n_operands < 1) return false;
  bool contiguous = false;
  for (int i = 0; i < ps.n_operands; ++i) {
    if (ps.in_stride[i][nr] == 1) return false;
    contiguous |= ps.in_stride[i][nr - 1] == 1;
  }
  return contiguous;
}

// -------------------------------------------------------------- validation

// A program is checked in full on the host before any launch: opcodes,
// register numbers, operand slots and dims in range.
int check_program(const pdh_ew_program* p, int ndim, bool allow_acc, const char* fn) {
  PDH_REQUIRE(p != nullptr, PDH_EINVAL, "%s: null program", fn);
  PDH_REQUIRE(p->n_insns >= 1 && p->n_insns <= PDH_EW_MAX_INSNS, PDH_EINVAL, "%s: %d instructions (1..%d)", fn,
              p->n_insns, PDH_EW_MAX_INSNS);
  PDH_REQUIRE(p->n_operands >= 0 && p->n_operands <= PDH_EW_MAX_OPERANDS, PDH_EINVAL, "%s: %d operands (max %d)", fn,
              p->n_operands, PDH_EW_MAX_OPERANDS);
  PDH_REQUIRE(p->ndim >= 1 && p->ndim <= PDH_EW_MAX_DIMS && (ndim < 0 || p->ndim == ndim), PDH_EINVAL,
              "%s: program ndim %d", fn, p->ndim);
  PDH_REQUIRE(p->out_reg >= 0 && p->out_reg < PDH_EW_MAX_REGS, PDH_EINVAL, "%s: out_reg %d", fn, p->out_reg);
  for (int d = 0; d < p->ndim; ++d) PDH_REQUIRE(p->shape[d] >= 1, PDH_EINVAL, "%s: shape[%d] = %lld", fn, d, (long long)p->shape[d]);
  for (int i = 0; i < p->n_insns; ++i) {
    const pdh_ew_insn& in = p->insns[i];
    PDH_REQUIRE(in.op < PDH_EW_NOPS, PDH_EINVAL, "%s: instruction %d: opcode %d", fn, i, in.op);
    PDH_REQUIRE(in.dst < PDH_EW_MAX_REGS && in.a < PDH_EW_MAX_REGS && in.b < PDH_EW_MAX_REGS && in.c < PDH_EW_MAX_REGS,
                PDH_EINVAL, "%s: instruction %d: register out of range", fn, i);
    if (in.op == PDH_EW_LOAD)
      PDH_REQUIRE(in.a < p->n_operands, PDH_EINVAL, "%s: instruction %d loads operand %d of %d", fn, i, in.a,
                  p->n_operands);
    if (in.op == PDH_EW_IOTA)
      PDH_REQUIRE(in.a < p->ndim, PDH_EINVAL, "%s: instruction %d: iota over dim %d of %d", fn, i, in.a, p->ndim);
    if (in.op == PDH_EW_ACC) PDH_REQUIRE(allow_acc, PDH_EINVAL, "%s: instruction %d reads an accumulator", fn, i);
  }
  return PDH_OK;
}

// A view of the program's lattice with these strides: non-negative strides,
// and its largest element offset under 2^31 (the interpreter's offsets are
// 32-bit).
int check_view(const pdh_ew_program* p, const int64_t* stride, const char* fn, const char* what) {
  int64_t reach = 0;
  for (int d = 0; d < p->ndim; ++d) {
    PDH_REQUIRE(stride[d] >= 0 && stride[d] <= INT32_MAX, PDH_EINVAL, "%s: %s stride[%d] = %lld", fn, what, d,
                (long long)stride[d]);
    reach += (p->shape[d] - 1) * stride[d];
    PDH_REQUIRE(reach <= INT32_MAX, PDH_EINVAL, "%s: the %s view spans more than 2^31 elements", fn, what);
  }
  return PDH_OK;
}

int dtype_ok(int dtype) { return dtype == PDH_F32 || dtype == PDH_BF16 || dtype == PDH_F16; }

}  // namespace
}  // namespace pdh

using namespace pdh;

extern "C" int pdh_map_chain(const pdh_ew_program* prog, const void* const* operands, void* out, int dtype,
                             void* stream) {
  int rc = check_program(prog, -1, false, "pdh_map_chain");
  if (rc) return rc;
  PDH_REQUIRE(dtype_ok(dtype), PDH_EUNSUPPORTED, "pdh_map_chain: dtype %d", dtype);
  PDH_REQUIRE(out != nullptr, PDH_EINVAL, "pdh_map_chain: null output");
  PDH_REQUIRE(prog->n_operands == 0 || operands != nullptr, PDH_EINVAL, "pdh_map_chain: null operand table");
  int64_t total = 1;
  for (int d = 0; d < prog->ndim; ++d) total *= prog->shape[d];
  PDH_REQUIRE(total <= INT32_MAX, PDH_EINVAL, "pdh_map_chain: %lld elements (at most 2^31 - 1 per call)",
              (long long)total);
  if ((rc = check_view(prog, prog->out_stride, "pdh_map_chain", "output"))) return rc;
  EwOperands ops{};
  for (int i = 0; i < prog->n_operands; ++i) {
    PDH_REQUIRE(operands[i] != nullptr, PDH_EINVAL, "pdh_map_chain: operand %d is null", i);
    if ((rc = check_view(prog, prog->in_stride[i], "pdh_map_chain", "operand"))) return rc;
    ops.p[i] = operands[i];
  }
  hipStream_t st = as_stream(stream);
  const bool four = prog->shape[prog->ndim - 1] % 4 == 0;  // four consecutive elements per lane
  const int64_t nthreads = four ? total / 4 : total;
  const dim3 grid(static_cast<unsigned>((nthreads + 255) / 256));
  uint32_t tot = static_cast<uint32_t>(total);
  hipFunction_t fns[2];
  if (jit_get(JitKind::MapChain, *prog, dtype, fns)) {
    pdh_ew_program pa = *prog;
    void* args[] = {&pa, &ops, &out, &tot};
    if (hipModuleLaunchKernel(four ? fns[0] : fns[1], grid.x, 1, 1, 256, 1, 1, 0, st, args, nullptr) != hipSuccess)
      PDH_REQUIRE(false, PDH_ELAUNCH, "pdh_map_chain: specialized launch failed");
    jit_count_launch();
    return PDH_OK;
  }
  auto go = [&](auto dt) {
    constexpr int DT = decltype(dt)::value;
    if (four)
      map_chain_kernel<DT, 4><<<grid, 256, 0, st>>>(*prog, ops, out, tot);
    else
      map_chain_kernel<DT, 1><<<grid, 256, 0, st>>>(*prog, ops, out, tot);
  };
  if (dtype == PDH_F32)
    go(std::integral_constant<int, PDH_F32>{});
  else if (dtype == PDH_BF16)
    go(std::integral_constant<int, PDH_BF16>{});
  else
    go(std::integral_constant<int, PDH_F16>{});
  return check_launch("pdh_map_chain");
}

namespace pdh {
namespace {

int g_cus = 0;  // compute units of the device, read once
std::atomic<int> g_f32_mode{6};  // fp32 contractions: 6 bf16 products per term (fp32 grade) by default

// Validation shared by the entry points, then the launch: the 128 x 128
// tiles, or the 64 x 64 ones when the big tiles would not give every compute
// unit a workgroup, an output side is 64 or under, or k is 128 or under.
int contract_launch(ContractArgs ca, const pdh_ew_program* epi, const void* const* operands, int64_t esize,
                    hipStream_t st, const char* fn, const ContractPro* pro = nullptr) {
  int rc = check_program(epi, 3, true, fn);
  if (rc) return rc;
  const int64_t batch = ca.batch, m = ca.m, n = ca.n;
  PDH_REQUIRE(epi->shape[0] == batch && epi->shape[1] == m && epi->shape[2] == n, PDH_EINVAL,
              "%s: epilogue shape must be {batch, m, n}", fn);
  PDH_REQUIRE(epi->n_operands == 0 || operands != nullptr, PDH_EINVAL, "%s: null operand table", fn);
  if ((rc = check_view(epi, epi->out_stride, fn, "output"))) return rc;
  EwOperands ops{};
  for (int i = 0; i < epi->n_operands; ++i) {
    PDH_REQUIRE(operands[i] != nullptr, PDH_EINVAL, "%s: operand %d is null", fn, i);
    if ((rc = check_view(epi, epi->in_stride[i], fn, "operand"))) return rc;
    ops.p[i] = operands[i];
  }
  // every 32-bit buffer offset (rows up to m + 128, k up to kp) stays under
  // 2^31, the offset that masked loads take
  PDH_REQUIRE((m + 128) * ca.sa_r * esize + ca.kp * ca.sa_k * esize < (int64_t{1} << 31) &&
                  (n + 128) * ca.sb_r * esize + ca.kp * ca.sb_k * esize < (int64_t{1} << 31),
              PDH_EINVAL, "%s: one k slice of a / bt must span under 2 GiB", fn);
  hipFunction_t fns[2];
  // operand layouts of the fp32 split kernels: bit 0 a, bit 1 bt rows-contiguous
  // (a computed operand takes the k-contiguous layout)
  const int lay = (ca.sa_k != 1 && !ca.pro_a ? 1 : 0) | (ca.sb_k != 1 && !ca.pro_b ? 2 : 0);
  PDH_REQUIRE(lay == 0 || ca.dtype == PDH_F32, PDH_EUNSUPPORTED, "%s: 16-bit operands must have k contiguous", fn);
  PDH_REQUIRE(ca.rowred < 0 || ca.dtype == PDH_F32, PDH_EUNSUPPORTED, "%s: row partials of fp32 contractions only", fn);
  PDH_REQUIRE(pro == nullptr || (ca.rowred < 0 && (ca.dtype == PDH_F32 || (ca.pro_a && ca.pro_b))), PDH_EUNSUPPORTED,
              "%s: operand prologues: no row partials, and with 16-bit storage both operands computed", fn);
  const bool spec = pro != nullptr ? jit_get_pro(*epi, ca.pro_a ? &pro[0].p : nullptr, ca.pro_b ? &pro[1].p : nullptr,
                                                 fns, lay, ca.dtype)
                                   : jit_get(JitKind::Contract, *epi, ca.dtype, fns, lay, ca.rowred);
  pdh_ew_program pe = *epi;
  ContractPro pro_a = pro != nullptr ? pro[0] : ContractPro{}, pro_b = pro != nullptr ? pro[1] : ContractPro{};
  void* args3[] = {&ca, &pe, &ops};
  void* args5[] = {&ca, &pe, &ops, &pro_a, &pro_b};
  void** args = pro != nullptr ? args5 : args3;
  auto launch_spec = [&](hipFunction_t f, int64_t nblk) {
    PDH_REQUIRE(nblk <= INT32_MAX, PDH_EINVAL, "%s: grid too large", fn);
    PDH_REQUIRE(hipModuleLaunchKernel(f, static_cast<unsigned>(nblk), 1, 1, 256, 1, 1, 0, st, args, nullptr) ==
                    hipSuccess,
                PDH_ELAUNCH, "%s: specialized launch failed", fn);
    jit_count_launch();
    return PDH_OK;
  };
  const int f32_mode = f32_contract_mode();
  if (ca.dtype != PDH_F32 && pro != nullptr) {  // 16-bit, computed operands: the one-plane split body
    if (g_cus == 0) g_cus = pdh_device_cus() > 0 ? pdh_device_cus() : 256;
    const bool small = batch * ((m + 127) / 128) * ((n + 127) / 128) < g_cus || m <= 64 || n <= 64 || ca.kp <= 2 * kBK;
    const int bm = small ? 64 : 128;
    ca.tiles_m = static_cast<int>((m + bm - 1) / bm);
    ca.tiles_n = static_cast<int>((n + bm - 1) / bm);
    const int64_t nblk = batch * ca.tiles_m * ca.tiles_n;
    if (spec) return launch_spec(fns[small ? 1 : 0], nblk);
    PDH_REQUIRE(nblk <= INT32_MAX, PDH_EINVAL, "%s: grid too large", fn);
    const dim3 grid(static_cast<unsigned>(nblk));
    PDH_REQUIRE(ca.dtype == PDH_BF16, PDH_EUNSUPPORTED, "%s: computed f16 operands", fn);
    if (small)
      contract_split16_pro_small<PDH_BF16><<<grid, 256, 0, st>>>(ca, *epi, ops, pro[0], pro[1]);
    else
      contract_split16_pro<PDH_BF16><<<grid, 256, 0, st>>>(ca, *epi, ops, pro[0], pro[1]);
    return check_launch(fn);
  }
  if (ca.dtype == PDH_F32 && f32_mode == 0) {
    ca.tiles_m = static_cast<int>((m + kFT - 1) / kFT);
    ca.tiles_n = static_cast<int>((n + kFT - 1) / kFT);
    const int64_t nblk = batch * ca.tiles_m * ca.tiles_n;
    if (spec) return launch_spec(fns[0], nblk);
    PDH_REQUIRE(nblk <= INT32_MAX, PDH_EINVAL, "%s: grid too large", fn);
    if (pro != nullptr)
      contract_f32_pro<<<dim3(static_cast<unsigned>(nblk)), 256, 0, st>>>(ca, *epi, ops, pro[0], pro[1]);
    else
      contract_f32<<<dim3(static_cast<unsigned>(nblk)), 256, 0, st>>>(ca, *epi, ops);
    return check_launch(fn);
  }
  if (g_cus == 0) g_cus = pdh_device_cus() > 0 ? pdh_device_cus() : 256;
  const int64_t big = batch * ((m + 127) / 128) * ((n + 127) / 128);
  // a side of 64 or under would leave big tiles half empty; a k of two tiles
  // or fewer leaves each workgroup too little work to hide its load latency,
  // which the small variant's higher occupancy does
  const bool small = big < g_cus || m <= 64 || n <= 64 || ca.kp <= 2 * kBK;
  const int bm = small ? 64 : 128;
  ca.tiles_m = static_cast<int>((m + bm - 1) / bm);
  ca.tiles_n = static_cast<int>((n + bm - 1) / bm);
  const int64_t nblk = batch * ca.tiles_m * ca.tiles_n;
  if (spec) return launch_spec(fns[small ? 1 : 0], nblk);
  PDH_REQUIRE(nblk <= INT32_MAX, PDH_EINVAL, "%s: grid too large", fn);
  const dim3 grid(static_cast<unsigned>(nblk));
  if (ca.dtype == PDH_F32) {  // on the bf16 matrix cores, split into planes
    if (f32_mode == 1)
      launch_split<1>(small, lay, grid, st, ca, *epi, ops, pro);
    else if (f32_mode == 3)
      launch_split<3>(small, lay, grid, st, ca, *epi, ops, pro);
    else
      launch_split<6>(small, lay, grid, st, ca, *epi, ops, pro);
  } else if (ca.dtype == PDH_BF16) {
    if (small)
      contract_mfma_small<PDH_BF16><<<grid, 256, 0, st>>>(ca, *epi, ops);
    else
      contract_mfma<PDH_BF16><<<grid, 256, 0, st>>>(ca, *epi, ops);
  } else {
    if (small)
      contract_mfma_small<PDH_F16><<<grid, 256, 0, st>>>(ca, *epi, ops);
    else
      contract_mfma<PDH_F16><<<grid, 256, 0, st>>>(ca, *epi, ops);
  }
  return check_launch(fn);
}

}  // namespace

int f32_contract_mode() { return g_f32_mode.load(); }

}  // namespace pdh

extern "C" int pdh_contract_set_f32_mode(int mode) {
  PDH_REQUIRE(mode == 0 || mode == 1 || mode == 3 || mode == 6, PDH_EINVAL,
              "pdh_contract_set_f32_mode: mode %d (0 VALU fma; 1, 3 or 6 bf16 products per term)", mode);
  return g_f32_mode.exchange(mode);
}

extern "C" int pdh_contract(const void* a, const void* bt, int64_t batch, int64_t m, int64_t n, int64_t k,
                            int64_t kp, const pdh_ew_program* epi, const void* const* operands, void* out, int dtype,
                            void* stream) {
  PDH_REQUIRE(dtype_ok(dtype), PDH_EUNSUPPORTED, "pdh_contract: dtype %d", dtype);
  PDH_REQUIRE(a && bt && out, PDH_EINVAL, "pdh_contract: null pointer");
  PDH_REQUIRE(batch >= 1 && m >= 1 && n >= 1 && k >= 1, PDH_EINVAL, "pdh_contract: bad shape");
  PDH_REQUIRE(kp >= k && kp % kBK == 0, PDH_EINVAL, "pdh_contract: kp = %lld must be >= k and a multiple of %d",
              (long long)kp, kBK);
  PDH_REQUIRE(batch * m * n <= INT32_MAX && m <= INT32_MAX / 2 && n <= INT32_MAX / 2, PDH_EINVAL,
              "pdh_contract: output too large for one call");
  PDH_REQUIRE(aligned16(a) && aligned16(bt), PDH_EINVAL, "pdh_contract: a / bt must be 16-byte aligned");
  const ContractArgs ca{a, bt, out, static_cast<int>(batch), static_cast<int>(m), static_cast<int>(n),
                        static_cast<int>(k), static_cast<int>(kp), 0, 0, dtype, m * kp, kp, n * kp, kp, 1, 1, 1, -1};
  return contract_launch(ca, epi, operands, dtype == PDH_F32 ? 4 : 2, as_stream(stream), "pdh_contract");
}

namespace {

// pdh_contract_strided and its k-split form: batch entry e's k columns in
// ksplit slices of k / ksplit, slice s of entry e as batch index e ksplit + s.
int contract_strided_impl(const void* a, int64_t sa_b, int64_t sa_r, const void* bt, int64_t sb_b, int64_t sb_r,
                          int64_t batch, int64_t m, int64_t n, int64_t k, int64_t ksplit,
                          const pdh_ew_program* epi, const void* const* operands, void* out, int dtype,
                          void* stream, const char* fn) {
  PDH_REQUIRE(dtype_ok(dtype), PDH_EUNSUPPORTED, "%s: dtype %d", fn, dtype);
  PDH_REQUIRE(a && bt && out, PDH_EINVAL, "%s: null pointer", fn);
  PDH_REQUIRE(batch >= 1 && m >= 1 && n >= 1 && k >= 1 && k % kBK == 0, PDH_EINVAL,
              "%s: need batch, m, n >= 1 and k a positive multiple of %d", fn, kBK);
  PDH_REQUIRE(ksplit >= 1 && ksplit <= 64 && k % (kBK * ksplit) == 0, PDH_EINVAL,
              "%s: ksplit = %lld must be in [1, 64] with k a multiple of %d * ksplit", fn, (long long)ksplit, kBK);
  PDH_REQUIRE(batch * ksplit * m * n <= INT32_MAX && m <= INT32_MAX / 2 && n <= INT32_MAX / 2, PDH_EINVAL,
              "%s: output too large for one call", fn);
  const int64_t align = dtype == PDH_F32 ? 4 : 8;  // 16-byte rows and batch slices
  PDH_REQUIRE(sa_r >= k && sb_r >= k && sa_b >= 0 && sb_b >= 0 && sa_r % align == 0 && sb_r % align == 0 &&
                  sa_b % align == 0 && sb_b % align == 0,
              PDH_EINVAL, "%s: row strides must be >= k and all strides multiples of %lld", fn, (long long)align);
  PDH_REQUIRE(aligned16(a) && aligned16(bt), PDH_EINVAL, "%s: a / bt must be 16-byte aligned", fn);
  const int64_t kc = k / ksplit;
  const ContractArgs ca{a, bt, out, static_cast<int>(batch * ksplit), static_cast<int>(m), static_cast<int>(n),
                        static_cast<int>(k), static_cast<int>(kc), 0, 0, dtype, sa_b, sa_r, sb_b, sb_r,
                        static_cast<int>(ksplit), 1, 1, -1};
  return contract_launch(ca, epi, operands, dtype == PDH_F32 ? 4 : 2, as_stream(stream), fn);
}

}  // namespace

extern "C" int pdh_contract_strided(const void* a, int64_t sa_b, int64_t sa_r, const void* bt, int64_t sb_b,
                                    int64_t sb_r, int64_t batch, int64_t m, int64_t n, int64_t k,
                                    const pdh_ew_program* epi, const void* const* operands, void* out, int dtype,
                                    void* stream) {
  return contract_strided_impl(a, sa_b, sa_r, bt, sb_b, sb_r, batch, m, n, k, 1, epi, operands, out, dtype, stream,
                               "pdh_contract_strided");
}

extern "C" int pdh_contract_strided_ksplit(const void* a, int64_t sa_b, int64_t sa_r, const void* bt, int64_t sb_b,
                                           int64_t sb_r, int64_t batch, int64_t m, int64_t n, int64_t k,
                                           int64_t ksplit, const pdh_ew_program* epi, const void* const* operands,
                                           void* out, int dtype, void* stream) {
  return contract_strided_impl(a, sa_b, sa_r, bt, sb_b, sb_r, batch, m, n, k, ksplit, epi, operands, out, dtype,
                               stream, "pdh_contract_strided_ksplit");
}

extern "C" int pdh_contract_views(const void* a, int64_t sa_b, int64_t sa_r, int64_t sa_k, const void* bt,
                                  int64_t sb_b, int64_t sb_r, int64_t sb_k, int64_t batch, int64_t m, int64_t n,
                                  int64_t k, int64_t ksplit, const pdh_ew_program* epi, const void* const* operands,
                                  void* out, int dtype, void* stream) {
  const char* fn = "pdh_contract_views";
  PDH_REQUIRE(dtype == PDH_F32, PDH_EUNSUPPORTED, "%s: fp32 operands only (16-bit ones: pdh_contract_strided)", fn);
  PDH_REQUIRE(a && bt && out, PDH_EINVAL, "%s: null pointer", fn);
  PDH_REQUIRE(batch >= 1 && m >= 1 && n >= 1 && k >= 1, PDH_EINVAL, "%s: need batch, m, n, k >= 1", fn);
  PDH_REQUIRE(ksplit >= 1 && ksplit <= 64, PDH_EINVAL, "%s: ksplit = %lld must be in [1, 64]", fn,
              (long long)ksplit);
  // slices of whole 64-column tiles; the last one may be ragged, none is empty
  const int64_t kc = ((k + kBK - 1) / kBK + ksplit - 1) / ksplit * kBK;
  PDH_REQUIRE((ksplit - 1) * kc < k, PDH_EINVAL, "%s: ksplit = %lld leaves a k slice empty (k = %lld)", fn,
              (long long)ksplit, (long long)k);
  PDH_REQUIRE(batch * ksplit * m * n <= INT32_MAX && m <= INT32_MAX / 2 && n <= INT32_MAX / 2 && k <= INT32_MAX / 2,
              PDH_EINVAL, "%s: output too large for one call", fn);
  PDH_REQUIRE(sa_b >= 0 && sa_r >= 0 && sa_k >= 0 && sb_b >= 0 && sb_r >= 0 && sb_k >= 0, PDH_EINVAL,
              "%s: negative stride", fn);
  PDH_REQUIRE((sa_k == 1 || sa_r == 1) && (sb_k == 1 || sb_r == 1), PDH_EINVAL,
              "%s: each operand needs k or its rows contiguous (a stride of 1)", fn);
  PDH_REQUIRE((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(bt)) % 4 == 0, PDH_EINVAL,
              "%s: a / bt must be 4-byte aligned", fn);
  const ContractArgs ca{a, bt, out, static_cast<int>(batch * ksplit), static_cast<int>(m), static_cast<int>(n),
                        static_cast<int>(k), static_cast<int>(kc), 0, 0, dtype, sa_b, sa_r, sb_b, sb_r,
                        static_cast<int>(ksplit), sa_k, sb_k, -1};
  return contract_launch(ca, epi, operands, 4, as_stream(stream), fn);
}

namespace {

// An operand prologue checked against its lattice (batch, rows, k) and its
// pointer table copied.
int check_pro(const pdh_ew_program* pr, const void* const* operands, int64_t batch, int64_t rows, int64_t k,
              ContractPro* out, const char* fn, const char* which) {
  int rc = check_program(pr, 3, false, fn);
  if (rc) return rc;
  PDH_REQUIRE(pr->shape[0] == batch && pr->shape[1] == rows && pr->shape[2] == k, PDH_EINVAL,
              "%s: the %s prologue's lattice must be {batch, %s, k}", fn, which, which[0] == 'a' ? "m" : "n");
  PDH_REQUIRE(pr->n_operands == 0 || operands != nullptr, PDH_EINVAL, "%s: null %s prologue operand table", fn, which);
  out->p = *pr;
  out->ops = EwOperands{};
  for (int i = 0; i < pr->n_operands; ++i) {
    PDH_REQUIRE(operands[i] != nullptr, PDH_EINVAL, "%s: %s prologue operand %d is null", fn, which, i);
    if ((rc = check_view(pr, pr->in_stride[i], fn, "prologue operand"))) return rc;
    out->ops.p[i] = operands[i];
  }
  return PDH_OK;
}

}  // namespace

extern "C" int pdh_contract_views_pro(const void* a, int64_t sa_b, int64_t sa_r, int64_t sa_k,
                                      const pdh_ew_program* pro_a, const void* const* pro_a_operands, const void* bt,
                                      int64_t sb_b, int64_t sb_r, int64_t sb_k, const pdh_ew_program* pro_b,
                                      const void* const* pro_b_operands, int64_t batch, int64_t m, int64_t n,
                                      int64_t k, int64_t ksplit, const pdh_ew_program* epi,
                                      const void* const* operands, void* out, int dtype, void* stream) {
  const char* fn = "pdh_contract_views_pro";
  PDH_REQUIRE(dtype == PDH_F32 || dtype == PDH_BF16, PDH_EUNSUPPORTED,
              "%s: dtype %d (fp32 or bf16; f16 operands would lose bits in bf16 planes)", fn, dtype);
  PDH_REQUIRE(pro_a != nullptr || pro_b != nullptr, PDH_EINVAL, "%s: no prologue (pdh_contract_views reads both)", fn);
  PDH_REQUIRE(dtype == PDH_F32 || (pro_a != nullptr && pro_b != nullptr), PDH_EUNSUPPORTED,
              "%s: with 16-bit storage both operands are computed (a stored one as a one-LOAD program)", fn);
  PDH_REQUIRE((pro_a || a) && (pro_b || bt) && out, PDH_EINVAL, "%s: null pointer", fn);
  PDH_REQUIRE(batch >= 1 && m >= 1 && n >= 1 && k >= 1, PDH_EINVAL, "%s: need batch, m, n, k >= 1", fn);
  PDH_REQUIRE(ksplit >= 1 && ksplit <= 64, PDH_EINVAL, "%s: ksplit = %lld must be in [1, 64]", fn,
              (long long)ksplit);
  const int64_t kc = ((k + kBK - 1) / kBK + ksplit - 1) / ksplit * kBK;
  PDH_REQUIRE((ksplit - 1) * kc < k, PDH_EINVAL, "%s: ksplit = %lld leaves a k slice empty (k = %lld)", fn,
              (long long)ksplit, (long long)k);
  PDH_REQUIRE(batch * ksplit * m * n <= INT32_MAX && m <= INT32_MAX / 2 && n <= INT32_MAX / 2 && k <= INT32_MAX / 2,
              PDH_EINVAL, "%s: output too large for one call", fn);
  ContractPro pro[2];
  int rc;
  if (pro_a) {
    if ((rc = check_pro(pro_a, pro_a_operands, batch, m, k, &pro[0], fn, "a"))) return rc;
    a = nullptr;
    sa_b = sa_r = 0;
    sa_k = 1;
  } else {
    PDH_REQUIRE(sa_b >= 0 && sa_r >= 0 && sa_k >= 0 && (sa_k == 1 || sa_r == 1), PDH_EINVAL,
                "%s: a needs k or its rows contiguous (a stride of 1), no negative stride", fn);
    PDH_REQUIRE(reinterpret_cast<uintptr_t>(a) % 4 == 0, PDH_EINVAL, "%s: a must be 4-byte aligned", fn);
  }
  if (pro_b) {
    if ((rc = check_pro(pro_b, pro_b_operands, batch, n, k, &pro[1], fn, "bt"))) return rc;
    bt = nullptr;
    sb_b = sb_r = 0;
    sb_k = 1;
  } else {
    PDH_REQUIRE(sb_b >= 0 && sb_r >= 0 && sb_k >= 0 && (sb_k == 1 || sb_r == 1), PDH_EINVAL,
                "%s: bt needs k or its rows contiguous (a stride of 1), no negative stride", fn);
    PDH_REQUIRE(reinterpret_cast<uintptr_t>(bt) % 4 == 0, PDH_EINVAL, "%s: bt must be 4-byte aligned", fn);
  }
  ContractArgs ca{a, bt, out, static_cast<int>(batch * ksplit), static_cast<int>(m), static_cast<int>(n),
                  static_cast<int>(k), static_cast<int>(kc), 0, 0, dtype, sa_b, sa_r, sb_b, sb_r,
                  static_cast<int>(ksplit), sa_k, sb_k, -1};
  ca.pro_a = pro_a != nullptr;
  ca.pro_b = pro_b != nullptr;
  return contract_launch(ca, epi, operands, 4, as_stream(stream), fn, pro);
}

extern "C" int pdh_contract_views_rowred(const void* a, int64_t sa_b, int64_t sa_r, int64_t sa_k, const void* bt,
                                         int64_t sb_b, int64_t sb_r, int64_t sb_k, int64_t batch, int64_t m, int64_t n,
                                         int64_t k, const pdh_ew_program* epi, const void* const* operands,
                                         int reducer, float* partials, int dtype, void* stream) {
  const char* fn = "pdh_contract_views_rowred";
  PDH_REQUIRE(dtype == PDH_F32, PDH_EUNSUPPORTED, "%s: fp32 operands only", fn);
  PDH_REQUIRE(reducer >= 0 && reducer <= 2, PDH_EINVAL, "%s: reducer %d (0 sum, 1 max, 2 min)", fn, reducer);
  PDH_REQUIRE(a && bt && partials, PDH_EINVAL, "%s: null pointer", fn);
  PDH_REQUIRE(batch >= 1 && m >= 1 && n >= 1 && k >= 1, PDH_EINVAL, "%s: need batch, m, n, k >= 1", fn);
  PDH_REQUIRE(batch * m * ((n + 31) / 32) <= INT32_MAX && batch * m * n <= (int64_t{1} << 40) && m <= INT32_MAX / 2 &&
                  n <= INT32_MAX / 2 && k <= INT32_MAX / 2,
              PDH_EINVAL, "%s: too large for one call", fn);
  PDH_REQUIRE(sa_b >= 0 && sa_r >= 0 && sa_k >= 0 && sb_b >= 0 && sb_r >= 0 && sb_k >= 0, PDH_EINVAL,
              "%s: negative stride", fn);
  PDH_REQUIRE((sa_k == 1 || sa_r == 1) && (sb_k == 1 || sb_r == 1), PDH_EINVAL,
              "%s: each operand needs k or its rows contiguous (a stride of 1)", fn);
  PDH_REQUIRE((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(bt)) % 4 == 0, PDH_EINVAL,
              "%s: a / bt must be 4-byte aligned", fn);
  const int64_t kc = (k + kBK - 1) / kBK * kBK;
  const ContractArgs ca{a, bt, partials, static_cast<int>(batch), static_cast<int>(m), static_cast<int>(n),
                        static_cast<int>(k), static_cast<int>(kc), 0, 0, dtype, sa_b, sa_r, sb_b, sb_r,
                        1, sa_k, sb_k, reducer};
  return contract_launch(ca, epi, operands, 4, as_stream(stream), fn);
}

extern "C" int pdh_reduce_rows(const pdh_ew_program* summand, int nk, const pdh_ew_program* epi,
                               const void* const* operands, int n_operands, void* out, int dtype, void* stream) {
  return pdh_reduce_rows_ex(summand, nk, epi, operands, n_operands, out, dtype, 0, stream);
}

extern "C" int pdh_reduce_rows_ex(const pdh_ew_program* summand, int nk, const pdh_ew_program* epi,
                                  const void* const* operands, int n_operands, void* out, int dtype, int reducer,
                                  void* stream) {
  PDH_REQUIRE(reducer >= 0 && reducer <= 2, PDH_EINVAL, "pdh_reduce_rows: reducer %d (0 sum, 1 max, 2 min)", reducer);
  int rc = check_program(summand, -1, false, "pdh_reduce_rows (summand)");
  if (rc) return rc;
  if ((rc = check_program(epi, -1, true, "pdh_reduce_rows (epilogue)"))) return rc;
  PDH_REQUIRE(dtype_ok(dtype), PDH_EUNSUPPORTED, "pdh_reduce_rows: dtype %d", dtype);
  PDH_REQUIRE(out != nullptr, PDH_EINVAL, "pdh_reduce_rows: null output");
  PDH_REQUIRE(nk >= 1 && epi->ndim + nk == summand->ndim, PDH_EINVAL,
              "pdh_reduce_rows: the summand's lattice must be the epilogue's plus nk = %d reduced dims", nk);
  for (int d = 0; d < epi->ndim; ++d)
    PDH_REQUIRE(summand->shape[d] == epi->shape[d] && summand->start[d] == epi->start[d], PDH_EINVAL,
                "pdh_reduce_rows: summand dim %d differs from the epilogue's", d);
  PDH_REQUIRE(n_operands >= 0 && n_operands <= PDH_EW_MAX_OPERANDS && summand->n_operands <= n_operands &&
                  epi->n_operands <= n_operands,
              PDH_EINVAL, "pdh_reduce_rows: %d operands for programs reading %d and %d", n_operands,
              summand->n_operands, epi->n_operands);
  PDH_REQUIRE(n_operands == 0 || operands != nullptr, PDH_EINVAL, "pdh_reduce_rows: null operand table");
  int64_t rows = 1, ktot = 1;
  for (int d = 0; d < epi->ndim; ++d) rows *= epi->shape[d];
  for (int d = epi->ndim; d < summand->ndim; ++d) ktot *= summand->shape[d];
  PDH_REQUIRE(rows <= INT32_MAX && ktot <= INT32_MAX, PDH_EINVAL, "pdh_reduce_rows: more than 2^31 rows or terms");
  if ((rc = check_view(epi, epi->out_stride, "pdh_reduce_rows", "output"))) return rc;
  EwOperands ops{};
  for (int i = 0; i < n_operands; ++i) {
    PDH_REQUIRE(operands[i] != nullptr, PDH_EINVAL, "pdh_reduce_rows: operand %d is null", i);
    ops.p[i] = operands[i];
  }
  for (int i = 0; i < summand->n_operands; ++i)
    if ((rc = check_view(summand, summand->in_stride[i], "pdh_reduce_rows", "summand operand"))) return rc;
  for (int i = 0; i < epi->n_operands; ++i)
    if ((rc = check_view(epi, epi->in_stride[i], "pdh_reduce_rows", "epilogue operand"))) return rc;
  hipStream_t st = as_stream(stream);
  const bool cols = reduce_by_columns(*summand, nk, epi->ndim, rows);
  const dim3 grid(static_cast<unsigned>(cols ? (rows + kColOut - 1) / kColOut : (rows + 3) / 4));
  const unsigned threads = cols ? kColOut * kColK : 256;
  int r32 = static_cast<int>(rows);
  hipFunction_t fns[2];
  if (jit_get_reduce(*summand, *epi, dtype, fns)) {
    pdh_ew_program a = *summand, b = *epi;
    void* args[] = {&a, &b, &ops, &out, &nk, &r32, &reducer};
    PDH_REQUIRE(hipModuleLaunchKernel(fns[cols ? 1 : 0], grid.x, 1, 1, threads, 1, 1, 0, st, args, nullptr) == hipSuccess,
                PDH_ELAUNCH, "pdh_reduce_rows: specialized launch failed");
    jit_count_launch();
    return PDH_OK;
  }
  auto go = [&](auto dt) {
    constexpr int DT = decltype(dt)::value;
    if (cols)
      reduce_cols_kernel<DT><<<grid, threads, 0, st>>>(*summand, *epi, ops, out, nk, r32, reducer);
    else
      reduce_rows_kernel<DT><<<grid, 256, 0, st>>>(*summand, *epi, ops, out, nk, r32, reducer);
  };
  if (dtype == PDH_F32)
    go(std::integral_constant<int, PDH_F32>{});
  else if (dtype == PDH_BF16)
    go(std::integral_constant<int, PDH_BF16>{});
  else
    go(std::integral_constant<int, PDH_F16>{});
  return check_launch("pdh_reduce_rows");
}
