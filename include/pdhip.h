/*
 * pdhip.h — the C ABI of libpdhip.so, the gfx950 (MI355X) execution backend
 * for the kernels pdum.dsl's fusion templates produce.
 *
 * The reference has no C ABI of its own: its one device seat is the Python
 * runner returned by
 *     compile_tile(region, launch=(), prune=()) -> run(values)
 * (conformance/triton_tile.py:662-698), which uploads f32 arrays, launches
 * one generated Triton program per fusion group and downloads the result.
 * Each entry point below replaces the device half of that runner for one
 * template row of the fusion registry (packages/tensorlib/src/pdum/tl/fusion.py):
 *
 *   pdh_row_softmax    <- template "row-normalization"  (fusion.py:818-825, 371-400)
 *   pdh_layernorm      <- template "row-statistics"     (fusion.py:826-843, 403-443)
 *   pdh_flash_fwd      <- template "flash" (+ artifacts m, den) (fusion.py:480-615)
 *   pdh_flash_bwd      <- the backward carves of the flash joint
 *                         (autodiff.py:102-122 + partition.py:586-607: dQ, dK, dV, D)
 *   pdh_attn_decode    <- the flash row at one query row per head, split over
 *                         the key axis and merged with the associative
 *                         online-softmax combine (zoo/attention.py:40-62)
 *   pdh_map_chain      <- template "map-chain" (fusion.py:844-854): a pointwise
 *                         program over one output lattice
 *   pdh_contract       <- template "contraction-epilogue" (fusion.py:159-324),
 *                         GEMM shape: sum over k of a broadcast product, the
 *                         epilogue program fused onto the accumulator
 *
 * Conventions
 *   - Every function returns 0 on success and a nonzero PDH_E* status on
 *     failure; nothing is launched when a shape, stride or dtype check fails.
 *     pdh_last_error() copies the calling thread's last message.
 *   - Pointers are caller-owned device pointers (non-owning). The library never
 *     allocates or frees caller memory; workspaces are passed in.
 *   - `stream` is a hipStream_t (NULL = the default stream). Calls are
 *     stream-ordered and asynchronous; calls on distinct streams are re-entrant.
 *   - Strides are in ELEMENTS. The innermost (feature / column) stride is 1.
 */
#ifndef PDHIP_H
#define PDHIP_H

#if !defined(__HIPCC_RTC__) /* hipRTC's builtins provide size_t */
#include <stddef.h>
#endif
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define PDH_OK 0
#define PDH_EINVAL 1       /* bad shape / stride / pointer / dtype combination */
#define PDH_EUNSUPPORTED 2 /* a legal request this build has no kernel for     */
#define PDH_ELAUNCH 3      /* the HIP runtime refused the launch               */

/* element types */
#define PDH_F32 0
#define PDH_BF16 1
#define PDH_F16 2

/* score masks: key s is live for query row t iff
 *   PDH_MASK_NONE : always
 *   PDH_MASK_BAND : band_lo <= s - t <= band_hi
 * Causal (le(iota_s, iota_t)) is BAND with band_lo = INT64_MIN, band_hi = 0;
 * strict causal (lt) is band_hi = -1; a sliding window of width W is
 * band_lo = 1 - W, band_hi = 0. Masked scores take the value `fill`
 * (the reference fills with -1e9, fusion.py:508-512, zoo/tiles.py:220). */
#define PDH_MASK_NONE 0
#define PDH_MASK_BAND 1

/* Attention geometry. Instances are (batch, head); query head h reads key/value
 * head h / (heads_q / heads_kv) (grouped-query attention when heads_kv < heads_q).
 * Row statistics (m, den, lse, delta) are dense fp32 [batch, heads_q, t]. */
typedef struct pdh_attn_geom {
  int64_t batch, heads_q, heads_kv;
  int64_t t;  /* query rows                  (reference dim "t") */
  int64_t s;  /* key / value rows            (reference dim "s") */
  int64_t e;  /* q/k feature, contracted     (reference dim "e") */
  int64_t od; /* v feature                   (reference dim "o") */
  int64_t q_sb, q_sh, q_st; /* element strides: batch, head, row */
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int64_t o_sb, o_sh, o_st;
} pdh_attn_geom;

/* Library version (major*10000 + minor*100 + patch). */
int pdh_version(void);

/* Copy the calling thread's last error text (NUL-terminated, truncated to n).
 * Returns the full length of the message. */
size_t pdh_last_error(char* buf, size_t n);

/* Number of compute units of the current device (0 on failure). */
int pdh_device_cus(void);

/* Row softmax over the last axis, fp32:
 *   y[r, :] = exp(x[r, :] - max x[r, :]) / sum exp(x[r, :] - max x[r, :])
 * Replaces the "row-normalization" group's runner (fusion.py:371-400 match,
 * :339-350 stage generator; conformance/triton_tile.py:442-469 lowering).
 * Rows are strided by ldx / ldy elements; columns are contiguous. */
int pdh_row_softmax(const float* x, float* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy,
                    void* stream);

/* Two-pass layernorm over the last axis, fp32 (zoo/zoo_common.py:56-60, 69-72):
 *   mu = mean x; xc = x - mu; y = xc / sqrt(mean(xc*xc) + eps) [* gamma] [+ beta]
 * gamma / beta may be NULL (the bare "row-statistics" core, fusion.py:403-443). */
int pdh_layernorm(const float* x, const float* gamma, const float* beta, float* y, int64_t rows,
                  int64_t cols, int64_t ldx, int64_t ldy, float eps, void* stream);

/* The same two row kernels over PDH_F32 / PDH_BF16 / PDH_F16 storage (x, y,
 * gamma and beta all of `dtype`), computing in fp32. These serve the carved
 * plan executor, whose boundary tensors carry the model's element type (the
 * reference runs its row groups at f32 only, triton_tile.py:442-469). */
int pdh_row_softmax_dt(const void* x, void* y, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int dtype,
                       void* stream);
int pdh_layernorm_dt(const void* x, const void* gamma, const void* beta, void* y, int64_t rows, int64_t cols,
                     int64_t ldx, int64_t ldy, float eps, int dtype, void* stream);

/* Row gather: out[i, :] = table[idx[i], :] for i < n_idx, rows of row_elems
 * elements (strides ld_table / ld_out), the device form of tl.take along the
 * table's leading dim (indexing.py:192-230). The reference plans a take as a
 * red group and runs it on the CPU (partition.py:586-607 with its executor,
 * tests/test_partition.py:15-37); the carved-plan executor runs it here. An
 * index outside [0, n_rows) writes a zero row and adds 1 to *bad (device int,
 * may be NULL), which the caller clears before and reads after. */
int pdh_take_rows(const void* table, const int64_t* idx, void* out, int64_t n_idx, int64_t row_elems,
                  int64_t n_rows, int64_t ld_table, int64_t ld_out, int dtype, int* bad, void* stream);

/* Row scatter-add: out[v, :] = sum of values[i, :] over the i < n_idx with
 * idx[i] == v, for every v < n_rows (rows no index names are zero), rows of
 * row_elems elements (strides ld_values / ld_out): tl.scatter_add, the
 * adjoint of the gather above along the output's leading dim
 * (indexing.py:153-190, 223-259; autodiff.py:846-856), which the reference
 * plans red and runs on the CPU; the carved-plan executor runs a model's
 * embedding gradient here. Deterministic: each row sums its value rows in
 * increasing i in fp32 and rounds once. An index outside [0, n_rows) is
 * dropped and adds 1 to *bad (device int, may be NULL). out must not overlap
 * values. n_idx <= 2^16 (the owner scan grows as n_idx^2 index compares);
 * larger batches return PDH_EUNSUPPORTED. */
int pdh_scatter_add_rows(const void* values, const int64_t* idx, void* out, int64_t n_idx, int64_t row_elems,
                         int64_t n_rows, int64_t ld_values, int64_t ld_out, int dtype, int* bad, void* stream);

/* Flash-attention forward: the online-softmax fold of _generate_flash
 * (fusion.py:542-615) over every (batch, head) instance:
 *   sc[t, s]  = scale * sum_e q[t, e] k[s, e]         (masked entries -> fill)
 *   m[t]      = max_s sc[t, s]
 *   den[t]    = sum_s exp(sc[t, s] - m[t])
 *   o[t, :]   = sum_s exp(sc[t, s] - m[t]) v[s, :] / den[t]
 *   lse[t]    = m[t] + log(den[t])
 * dtype PDH_BF16 / PDH_F16: q, k, v, o in that type, MFMA with fp32 accumulation
 *   (e == od in {64, 128}). PDH_F32: q, k, v, o fp32, any e / od.
 * m_out, den_out, lse_out are optional (NULL = not stored): (m, den) are the
 * reference's artifact outputs, yield order (out, m, den) (fusion.py:611-613).
 * prune != 0 lets kernels skip key tiles that the mask makes entirely inert;
 * it is ignored (everything is swept) when some query row has no live key,
 * the fully-masked-row law of fusion.py:659-690. */
int pdh_flash_fwd(const void* q, const void* k, const void* v, void* o, float* m_out, float* den_out,
                  float* lse_out, const pdh_attn_geom* geom, int dtype, float scale, float fill,
                  int mask_kind, int64_t band_lo, int64_t band_hi, int prune, void* stream);

/* The same forward split over the key axis, for grids too small to fill the
 * chip (few instances x query blocks, long rows: a batch-1 prefill). Each
 * query block's key-tile range is cut into `nsplit` runs swept by separate
 * workgroups, which store partial (o, running max, denominator) to `ws`; a
 * second kernel merges them with the associative online-softmax combine
 * (zoo/attention.py:40-46) and stores o and the optional m / den / lse as
 * pdh_flash_fwd does. The result equals pdh_flash_fwd's up to fp32 rounding
 * order (bf16 / f16 only; PDH_F32 runs unsplit). nsplit in [1, 64]; ws must
 * be 16-byte aligned and hold pdh_flash_fwd_workspace(geom, nsplit) bytes
 * (0 for nsplit <= 1). No counterpart in the reference: a launch shape of
 * the flash template's run (fusion.py:542-615). */
size_t pdh_flash_fwd_workspace(const pdh_attn_geom* geom, int nsplit);
int pdh_flash_fwd_split(const void* q, const void* k, const void* v, void* o, float* m_out, float* den_out,
                        float* lse_out, const pdh_attn_geom* geom, int dtype, float scale, float fill,
                        int mask_kind, int64_t band_lo, int64_t band_hi, int prune, int nsplit, void* ws,
                        size_t ws_bytes, void* stream);

/* Flash-attention backward (the closed form of the flash joint's gradients,
 * autodiff.py:102-122 over zoo/tiles.py:238-252's naive twin):
 *   P = exp(scale*q k^T - lse), dV = P^T dO, dP = dO v^T, delta = rowsum(dO * o),
 *   dS = P * (dP - delta), dQ = scale * dS k, dK = scale * dS^T q.
 * Row statistics come from the forward: lse (required), and optionally the
 * (m, den) artifacts. Masked scores take `fill` (as in the forward) and carry
 * no gradient. A row whose keys are ALL masked has uniform probabilities
 * 1/den (the reference's fully-masked-row semantics); fp32 cannot hold that
 * row's lse = fill + log(den) exactly, so with (m, den) given the kernels
 * use exp(fill - m) / den, and without them a row whose lse lies within
 * 2^6 of the fill (in log2 units) is taken as fully masked (P = 1/s).
 * dout / dq share o / q's strides; dk / dv share k / v's strides.
 * ws: fp32 workspace of 3*batch*heads_q*t elements (-delta, log2-domain
 * statistic, masked-entry probability per row; written).
 * dtype PDH_BF16 / PDH_F16: MFMA kernels, e == od in {64, 128}, 16-byte
 * aligned tensors, strides multiples of 8 elements. PDH_F32: the fp32 column
 * (VALU), any 1 <= e, od <= 512. Grouped-query heads (heads_q a multiple of
 * heads_kv; query head h reads K / V head h / (heads_q / heads_kv)): dk / dv
 * of a K / V head sum over the query heads of its group, each written by
 * one workgroup (no atomics). */
int pdh_flash_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout,
                  const float* lse, const float* m_in, const float* den_in, void* dq, void* dk, void* dv,
                  float* ws, const pdh_attn_geom* geom, int dtype, float scale, float fill,
                  int mask_kind, int64_t band_lo, int64_t band_hi, void* stream);

/* Decode attention (t query rows per head, small t), split over the key axis:
 * each of `nsplit` chunks writes partial (m, den, o) to `ws`, and a merge pass
 * applies the associative online-softmax combine (zoo/attention.py:40-46).
 * Grouped-query: heads_q / heads_kv query heads share one key/value head and
 * are packed into one workgroup so each key/value byte is read once.
 * No mask (every cache row is live). lse_out optional.
 * ws must hold pdh_attn_decode_workspace(geom, nsplit) bytes. */
size_t pdh_attn_decode_workspace(const pdh_attn_geom* geom, int nsplit);
int pdh_attn_decode(const void* q, const void* k, const void* v, void* o, float* lse_out,
                    const pdh_attn_geom* geom, int dtype, float scale, int nsplit, void* ws,
                    size_t ws_bytes, void* stream);

/* Inclusive prefix reduce along one dim (tl.scan; the reference's
 * compute.py:318-350, run by its evaluator as a red group: the
 * first-occurrence max / min adjoint, autodiff.py:635-665, carries one).
 * x, y: dense [outer][n][inner] of `dtype` (fp32 arithmetic); the scan runs
 * along n: y[o][t][i] folds x[o][0..t][i] (reverse != 0: x[o][t..n-1][i]).
 * A mean divides prefix t by its count. Max / min propagate NaN. y may be x. */
#define PDH_SCAN_SUM 0
#define PDH_SCAN_MAX 1
#define PDH_SCAN_MIN 2
#define PDH_SCAN_PROD 3
#define PDH_SCAN_MEAN 4
int pdh_scan(const void* x, void* y, int64_t outer, int64_t n, int64_t inner, int dtype, int reducer, int reverse,
             void* stream);

/* pdh_attn_decode without a workspace argument and without allocating: the
 * split partials go to a device array the library holds, one per GPU, of
 * PDH_DECODE_SCRATCH_BYTES, from the first call on that GPU until the process
 * ends. No counterpart in the reference; it is for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc). The caller still passes inputs and outputs. A request
 * whose pdh_attn_decode_workspace(geom, nsplit) exceeds the array is refused
 * (PDH_EINVAL) before anything runs. Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams or threads) race.
 * Results equal pdh_attn_decode's bit for bit (the same kernels). */
#define PDH_DECODE_SCRATCH_BYTES (16u << 20)
int pdh_attn_decode_noalloc(const void* q, const void* k, const void* v, void* o, float* lse_out,
                            const pdh_attn_geom* geom, int dtype, float scale, int nsplit, void* stream);

/* ------------------------------------------------------------------------
 * Elementwise programs. The pointwise chains of the map-chain template and
 * of a contraction's epilogue are lowered to a small register program, run
 * per output element by an interpreter whose instruction stream is uniform
 * across the wave (scalar decode, VGPR-indexed register file): no runtime
 * compilation. Registers hold fp32.
 *
 *   LOAD   r[dst] = operand a at the element (its strides over the output
 *                   dims; stride 0 broadcasts)
 *   ACC    r[dst] = the contraction accumulator (pdh_contract epilogues only)
 *   CONST  r[dst] = imm
 *   IOTA   r[dst] = coordinate along output dim a, plus that dim's start
 *   unary  r[dst] = f(r[a])            NEG EXP LOG SQRT TANH SIN COS ABS FLOOR
 *   binary r[dst] = f(r[a], r[b])      ADD SUB MUL DIV MAX MIN, and the
 *                                      comparisons EQ NE LT LE GT GE (1 or 0)
 *   WHERE  r[dst] = r[a] != 0 ? r[b] : r[c]
 * The result is r[out_reg]. Marker semantics follow the reference's numpy
 * markers (dsl/markers.py): maximum / minimum, where on a 0/1 mask. */
#define PDH_EW_MAX_INSNS 64
#define PDH_EW_MAX_REGS 16
#define PDH_EW_MAX_OPERANDS 8
#define PDH_EW_MAX_DIMS 4

enum pdh_ew_op {
  PDH_EW_LOAD = 0, PDH_EW_ACC, PDH_EW_CONST, PDH_EW_IOTA,
  PDH_EW_NEG, PDH_EW_EXP, PDH_EW_LOG, PDH_EW_SQRT, PDH_EW_TANH, PDH_EW_SIN, PDH_EW_COS, PDH_EW_ABS, PDH_EW_FLOOR,
  PDH_EW_ADD, PDH_EW_SUB, PDH_EW_MUL, PDH_EW_DIV, PDH_EW_MAX, PDH_EW_MIN,
  PDH_EW_EQ, PDH_EW_NE, PDH_EW_LT, PDH_EW_LE, PDH_EW_GT, PDH_EW_GE,
  PDH_EW_WHERE,
  PDH_EW_RBF16, PDH_EW_RF16, /* round to the nearest bf16 / f16 value (ties to even) and back: tl.round_to */
  PDH_EW_NOPS
};

typedef struct pdh_ew_insn {
  uint8_t op, dst, a, b, c, pad0, pad1, pad2;
  float imm;
} pdh_ew_insn;

typedef struct pdh_ew_program {
  int32_t n_insns, n_operands, ndim, out_reg;
  int64_t shape[PDH_EW_MAX_DIMS];  /* output extents, outermost first (the last dim is fastest) */
  int64_t start[PDH_EW_MAX_DIMS];  /* each output dim's domain start (IOTA adds it) */
  int64_t out_stride[PDH_EW_MAX_DIMS];
  int64_t in_stride[PDH_EW_MAX_OPERANDS][PDH_EW_MAX_DIMS];
  pdh_ew_insn insns[PDH_EW_MAX_INSNS];
} pdh_ew_program;

/* The map-chain template: out[c] = program(operands at c) for every
 * coordinate c of the output lattice (prog->shape, at most 2^31 - 1 elements).
 * operands[i] / out: device pointers of `dtype` (PDH_F32, PDH_BF16, PDH_F16);
 * the program computes in fp32 and rounds once on the store. */
int pdh_map_chain(const pdh_ew_program* prog, const void* const* operands, void* out, int dtype, void* stream);

/* The contraction-epilogue template, GEMM shape, batched:
 *   acc[b, m, n] = sum_k a[b, m, k] * bt[b, n, k]
 *   out[b, m, n] = epi(acc[b, m, n], operands at (b, m, n))
 * a: [batch][m][kp], bt: [batch][n][kp], row-major with kp (the row stride)
 * a multiple of 64 and columns k..kp-1 zero (the caller pads). The epilogue
 * program's output dims are (b, m, n) (ndim 3, shape {batch, m, n}); it reads
 * the accumulator with PDH_EW_ACC and may not LOAD more than n_operands.
 * dtype PDH_BF16 / PDH_F16: v_mfma_f32_32x32x16, fp32 accumulate, 128x128
 * workgroup tiles (64x64 when 128x128 tiles would not give every compute
 * unit one); PDH_F32: the same tiles on the bf16 matrix cores, each fp32
 * operand split into bf16 planes and the cross products summed with fp32
 * accumulation (pdh_contract_set_f32_mode). The sum over k is re-bracketed
 * by k tiles (license gemm.k-reassoc). */
int pdh_contract(const void* a, const void* bt, int64_t batch, int64_t m, int64_t n, int64_t k, int64_t kp,
                 const pdh_ew_program* epi, const void* const* operands, void* out, int dtype, void* stream);

/* The same batched contraction with a and bt read through element strides:
 * a[b, r, :] starts at a + b*sa_b + r*sa_r, bt[b, r, :] at bt + b*sb_b + r*sb_r,
 * and k (a positive multiple of 64) is contiguous, so a value stored in any
 * dim order with its contracted dims innermost feeds the product without a
 * copy (the carved-plan executor's boundary tensors: a head-major view of a
 * (t, heads, head_dim) tensor is sa_b = head_dim, sa_r = heads*head_dim).
 * Strides are multiples of 16 bytes; row strides are >= k. */
int pdh_contract_strided(const void* a, int64_t sa_b, int64_t sa_r, const void* bt, int64_t sb_b, int64_t sb_r,
                         int64_t batch, int64_t m, int64_t n, int64_t k, const pdh_ew_program* epi,
                         const void* const* operands, void* out, int dtype, void* stream);

/* pdh_contract_strided with each batch entry's k split into ksplit slices of
 * k / ksplit (k a multiple of 64 * ksplit) that run as separate workgroups:
 * batch index e * ksplit + s holds entry e's products over k columns
 * [s k / ksplit, (s + 1) k / ksplit), and the epilogue's lattice is
 * (batch * ksplit, m, n). With an identity epilogue into an fp32 buffer these
 * are partial sums a second pass adds (the executor does so, in slice order,
 * through the real epilogue): for grids whose output tiles cannot fill the
 * chip. No counterpart in the reference, whose contraction kernels do not
 * split k. */
int pdh_contract_strided_ksplit(const void* a, int64_t sa_b, int64_t sa_r, const void* bt, int64_t sb_b, int64_t sb_r,
                                int64_t batch, int64_t m, int64_t n, int64_t k, int64_t ksplit,
                                const pdh_ew_program* epi, const void* const* operands, void* out, int dtype,
                                void* stream);

/* The fp32 contraction over operands read in place as views: a[b, r, k] at
 * a + b sa_b + r sa_r + k sa_k, bt likewise. Each operand has k contiguous
 * (sa_k == 1) or its rows contiguous (sa_r == 1, any sa_k: a transposed
 * tensor such as P in P^T dO); k is any size, its columns in ksplit slices of
 * whole 64-column tiles (the last one ragged, none empty), and the epilogue's
 * lattice is (batch * ksplit, m, n) as in pdh_contract_strided_ksplit. Only
 * 4-byte alignment is needed. This replaces the operand layouts the
 * reference's contraction template lowers to strided loads
 * (fusion.py:159-324: its operands are any views of the lattice), which the
 * other entry points take only as zero-padded k-contiguous copies. PDH_F32
 * only: PDH_EUNSUPPORTED otherwise. */
int pdh_contract_views(const void* a, int64_t sa_b, int64_t sa_r, int64_t sa_k, const void* bt, int64_t sb_b,
                       int64_t sb_r, int64_t sb_k, int64_t batch, int64_t m, int64_t n, int64_t k, int64_t ksplit,
                       const pdh_ew_program* epi, const void* const* operands, void* out, int dtype, void* stream);

/* pdh_contract_views with either operand (or both) computed in the k loop
 * instead of read: pro_a, when not NULL, is an elementwise program over the
 * lattice (batch, m, k) whose value at (b, r, kk) is a[b, r, kk], its LOADs
 * indexing pro_a_operands (a and sa_* are then ignored); pro_b likewise over
 * (batch, n, k) for bt. k counts from the batch entry's first column across k
 * slices. The operand is evaluated once per element as the k tiles are
 * loaded (the hipRTC-specialized straight-line evaluator by default, the
 * interpreter otherwise) and never stored. Replaces the reference's operand
 * re-derivation inside the contraction's k loop (conformance/triton_tile.py:
 * 228-371, _dot_at / _reduce_at), where this library's other entry points take
 * a computed operand only as a buffer a map chain has filled first. No row
 * partials. PDH_BF16 storage: both operands are computed (a stored
 * operand as a one-LOAD program over its strides), their LOADs read 16-bit
 * values, each operand value is rounded to bf16 (as a 16-bit operand a map
 * chain materializes is) and the products accumulate in fp32; the output is
 * rounded once to bf16. Other element types: PDH_EUNSUPPORTED. */
int pdh_contract_views_pro(const void* a, int64_t sa_b, int64_t sa_r, int64_t sa_k, const pdh_ew_program* pro_a,
                           const void* const* pro_a_operands, const void* bt, int64_t sb_b, int64_t sb_r,
                           int64_t sb_k, const pdh_ew_program* pro_b, const void* const* pro_b_operands,
                           int64_t batch, int64_t m, int64_t n, int64_t k, int64_t ksplit,
                           const pdh_ew_program* epi, const void* const* operands, void* out, int dtype,
                           void* stream);

/* pdh_contract_views (no k split) whose epilogue values are not stored but
 * reduced along each output row in runs of 32 columns: partials[b, r, j] =
 * R over columns 32 j .. 32 j + 31 (those under n) of epi(acc)[b, r, col],
 * R = sum / max / min (reducer 0 / 1 / 2; max and min propagate NaN), fp32
 * [batch][m][ceil(n / 32)] dense. The caller finishes the rows with
 * pdh_reduce_rows_ex over the partials. This is the device form of a
 * contraction-epilogue group whose result feeds a row reduction (the
 * softmax's max and denominator over the scores a @ bt^T): the reference
 * runs that chain as two templates with the scores in between
 * (fusion.py:159-324, then :371-443); here the scores never reach HBM.
 * PDH_F32 only. */
int pdh_contract_views_rowred(const void* a, int64_t sa_b, int64_t sa_r, int64_t sa_k, const void* bt, int64_t sb_b,
                              int64_t sb_r, int64_t sb_k, int64_t batch, int64_t m, int64_t n, int64_t k,
                              const pdh_ew_program* epi, const void* const* operands, int reducer, float* partials,
                              int dtype, void* stream);

/* How PDH_F32 contractions run (pdh_contract, pdh_contract_strided): 6 (the
 * default) splits each operand into three bf16 terms and sums the six cross
 * products above 2^-24 of each product: fp32 grade; 3 keeps two terms and
 * three products (about 2^-16 of each product, twice the rate); 1 rounds the
 * operands to bf16 (fp32 accumulation and storage: the numerics of a bf16
 * autocast); 0 runs fp32 VALU fma. In the split modes a workgroup that loads
 * an inf, a NaN or a value beyond the bf16 range recomputes its tile by fp32
 * fma, so those behave as in fp32. Returns the previous mode; other values
 * are refused. The mode is
 * process-wide: contractions launched while it changes race. Replaces the
 * fp32 columns of the reference's contraction runners, which compute fp32
 * products directly (conformance/triton_tile.py:662-698, f32 dtype). */
int pdh_contract_set_f32_mode(int mode);

/* The ROWSUM and PLAIN shapes of the contraction-epilogue group (fusion.py:
 * 158-252: same-space operands multiplied and summed, or one operand summed,
 * e.g. the backward's D = rowsum(dO * O) and a bias gradient):
 *   out[r] = epi(sum_k summand(r, k))
 * `summand` runs over the lattice (row dims..., k dims...) whose last nk dims
 * are reduced; `epi` runs over the row dims (its ACC reads the fp32 sum).
 * Both programs index one table of n_operands pointers. One wave per output
 * element; when the one reduced dim is strided in every summand operand and
 * one operand is contiguous along the last output dim (a bias gradient), 16
 * consecutive outputs per workgroup of 1024 lanes instead, 64 lanes each
 * splitting k, so the loads stay coalesced. */
int pdh_reduce_rows(const pdh_ew_program* summand, int nk, const pdh_ew_program* epi, const void* const* operands,
                    int n_operands, void* out, int dtype, void* stream);
/* The same with the reducer chosen: 0 sum (pdh_reduce_rows), 1 max, 2 min.
 * A bare max / min over dims is a group the reference leaves red and serves on
 * its evaluator (partition.py:586-607); the carved-plan executor runs it here
 * (a softmax's row max that a backward joint materializes). */
int pdh_reduce_rows_ex(const pdh_ew_program* summand, int nk, const pdh_ew_program* epi,
                       const void* const* operands, int n_operands, void* out, int dtype, int reducer, void* stream);

/* Runtime specialization of elementwise programs. pdh_map_chain and
 * pdh_contract first compile the program into straight-line code with hipRTC
 * (once per distinct program and element type, cached for the process) and
 * fall back to the interpreter kernels when that is disabled or fails.
 * pdh_ew_set_jit(0) disables it (1 enables; the default is on unless the
 * environment sets PDH_JIT=0) and returns the previous setting;
 * pdh_ew_jit_stats fills {programs compiled, launches through specialized
 * kernels, compile failures}. */
int pdh_ew_set_jit(int enable);
void pdh_ew_jit_stats(int64_t* stats3);
/* The generated source of a program's specialized kernels (kind 0: map
 * chain, 1: contraction epilogue; 2, 3, 4: the fp32 contraction with a, bt or
 * both read rows-contiguous, as pdh_contract_views; 5, 6, 7: its row
 * partials by sum, max, min, as pdh_contract_views_rowred) for `dtype`, NUL-terminated into buf
 * (truncated to n); returns its full length (0 for a malformed program).
 * The readable counterpart of the reference runner's run.source. */
size_t pdh_ew_jit_source(const pdh_ew_program* prog, int kind, int dtype, char* buf, size_t n);
/* Compile that source with hipRTC without loading it (no GPU needed):
 * PDH_OK, or PDH_ELAUNCH with the compiler log in pdh_last_error(). */
int pdh_ew_jit_compile(const pdh_ew_program* prog, int kind, int dtype);

/* MFMA lane-layout probe (test support): multiplies one 32x16 by 16x32 bf16
 * tile with v_mfma_f32_32x32x16_bf16 and one 16x32 by 32x16 tile with
 * v_mfma_f32_16x16x32_bf16, each lane loading operands by the layout the
 * attention kernels assume; c32 (32x32) and c16 (16x16) are row-major fp32. */
int pdh_probe_mfma(const uint16_t* a32, const uint16_t* b32, float* c32, const uint16_t* a16,
                   const uint16_t* b16, float* c16, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PDHIP_H */
