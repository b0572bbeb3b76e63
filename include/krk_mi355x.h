/*
 * krk_mi355x.h -- C ABI of the MI355X (gfx950) quantized weight-math backend.
 *
 * This is the drop-in boundary for Kraken's `Backend` hot-path operators
 * (include/krk/backend.hpp:337-1876 in the reference).  The reference boundary
 * is a C++ virtual interface; here every operator is an `extern "C"` function
 * on an opaque handle, with plain pointers and sizes and an int status
 * instead of the reference's abort-on-error (backend_hip.hip:78-82).
 *
 * Conventions (same meaning as the reference, backend.hpp:859-860):
 *   - W is raw GGUF block bytes, row-major: n_out rows of
 *     krk_dtype_row_bytes(wt, n_in) bytes each.
 *   - x is [rows, n_in] and out is [rows, n_out], both in the handle's
 *     activation type (KRK_ACT_F32: float, KRK_ACT_F16: IEEE half).
 *   - Every data pointer is caller-owned DEVICE memory (as in the reference:
 *     x, w, out, ids, wts and the MoE table are device pointers).
 *   - Launches are asynchronous on the handle's stream (the null stream until
 *     krk_set_stream); krk_sync waits for them.
 *   - A handle is not thread-safe: one host thread drives one handle, as in
 *     the reference.  Several threads may each drive their own handle at the
 *     same time (the library's launch-shape caches are per thread).
 */
#ifndef KRK_MI355X_H
#define KRK_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids; these block formats (plus F16/F32 activations) are on
 * this path.  include/krk/quant.hpp:16-47.  Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q5_K, IQ4_NL, IQ4_XS,
 * MXFP4 and unquantized F16 / BF16 weights (16-byte aligned) are served by
 * the dequant, GEMV (rows 1..8, exact prefill) and MFMA GEMM paths, and by
 * moe_dispatch as expert banks (any served type per expert and matrix);
 * the int8 rung takes Q8_0, Q4_K, Q5_K and Q6_K.  The ids after MXFP4 below
 * take the same operators through a generic 32-value chunk path. */
enum krk_dtype {
    KRK_DT_F32 = 0,
    KRK_DT_F16 = 1,
    KRK_DT_Q4_0 = 2,
    KRK_DT_Q4_1 = 3,
    KRK_DT_Q5_0 = 6,
    KRK_DT_Q5_1 = 7,
    KRK_DT_Q8_0 = 8,
    KRK_DT_Q2_K = 10,
    KRK_DT_Q3_K = 11,
    KRK_DT_Q4_K = 12,
    KRK_DT_Q5_K = 13,
    KRK_DT_Q6_K = 14,
    KRK_DT_IQ4_NL = 20,
    KRK_DT_IQ4_XS = 23,
    KRK_DT_BF16 = 30,
    KRK_DT_MXFP4 = 39,
    /* served through the generic 32-value chunk path (include/krk/quant.hpp:
     * 25-31, 67-68, 105, 128-129, 166-168): dequant, GEMV rows 1..8, the MFMA
     * GEMM and MoE expert banks, at any byte alignment */
    KRK_DT_Q8_1 = 9,
    KRK_DT_Q8_K = 15,
    KRK_DT_TQ1_0 = 34,
    KRK_DT_TQ2_0 = 35,
    KRK_DT_NVFP4 = 40,
    KRK_DT_ROCMFP4 = 100,
    KRK_DT_ROCMFP4_FAST = 101,
    KRK_DT_Q6_0_ROCMFPX = 102,
    KRK_DT_Q3_0_ROCMFPX = 104,
    KRK_DT_Q2_0_ROCMFPX = 107,
    KRK_DT_Q1_0 = 41,      /* include/krk/quant.hpp:120-135 */
    KRK_DT_Q2_0 = 42,      /* the 128-value / 34-byte layout */
    KRK_DT_Q2_0_64 = 48,
    KRK_DT_PQ2_0 = 142,
    KRK_DT_PTQ1_0 = 143
};

/* Activation type of a handle: backend.hpp `act_type()` (F16 on the
 * reference GPU backend, F32 on its CPU oracle, backend_cpu.cpp:584). */
enum krk_act { KRK_ACT_F32 = 0, KRK_ACT_F16 = 1 };

/* Kernel family for rows > 8 (backend_hip.hip:2712-2893 `gemm_rung` and the
 * KRK_GEMM_EXACT / KRK_GEMM_PATH / KRK_GEMM_INT8 switches). */
enum krk_gemm_path {
    KRK_PATH_AUTO = 0,  /* MFMA f16 GEMM for rows > 8                       */
    KRK_PATH_EXACT = 1, /* multi-row GEMV, f32 products (gemv_grid analogue) */
    KRK_PATH_MFMA = 2,  /* W dequantized to f16 LDS tiles, f16 MFMA, f32 acc */
    KRK_PATH_INT8 = 3   /* Q8_0/Q4_K/Q5_K/Q6_K x Q8 activations (lossy rung) */
};

enum krk_status {
    KRK_OK = 0,
    KRK_ERR_ARG = -1,         /* null pointer, non-positive size            */
    KRK_ERR_DTYPE = -2,       /* weight type not on this path               */
    KRK_ERR_SHAPE = -3,       /* n_in not a whole number of blocks, etc.    */
    KRK_ERR_HIP = -4,         /* a HIP runtime call failed                  */
    KRK_ERR_NOMEM = -5,       /* scratch could not be allocated             */
    KRK_ERR_UNSUPPORTED = -6  /* valid request this backend does not serve  */
};

typedef struct krk_backend krk_backend;

/* One (layer, expert) bank, laid out exactly as the reference's POD table
 * (include/krk/moe_table.hpp:42-50): indexed table[layer * n_expert + e]. */
enum { KRK_MOE_GATE = 0, KRK_MOE_UP = 1, KRK_MOE_DOWN = 2 };
typedef struct krk_moe_entry {
    void *p[3];           /* device weight pointers               */
    int64_t n_out[3];     /* rows of each matrix                  */
    int64_t n_in[3];      /* columns                              */
    int64_t row_bytes[3]; /* bytes per quantized row              */
    int32_t type[3];      /* krk_dtype                            */
    int32_t present[3];   /* 0 => matrix absent                   */
    int32_t _pad;
} krk_moe_entry;

/* ---------------------------------------------------------------- handle -- */

/* make_hip_backend(device_index, err) -- backend.hpp:1886,
 * backend_hip.hip:5036.  act is a krk_act.  The handle allocates 16 KB of
 * device memory here (zeroed tile counters through which a two-way split-K
 * GEMM sums its splits inside the kernel; every call leaves them zero), so
 * calls on one handle must not overlap: the handle has one stream. */
int krk_backend_create(int device, int act, krk_backend **out);
int krk_backend_destroy(krk_backend *b);
/* Launch stream (a hipStream_t); NULL selects the null stream. */
int krk_set_stream(krk_backend *b, void *stream);
/* Rows > 8 policy (krk_gemm_path). */
int krk_set_gemm_path(krk_backend *b, int path);
int krk_act_type(const krk_backend *b);
/* sync() = hipDeviceSynchronize in the reference (backend_hip.hip:2325);
 * here a wait on the handle's stream. */
int krk_sync(krk_backend *b);
/* Text of the last error on this handle ("" when none). */
const char *krk_last_error(const krk_backend *b);
const char *krk_status_string(int status);

/* ------------------------------------------------------------- geometry -- */
/* dtype_block_size / dtype_block_bytes / dtype_row_bytes / dtype_row_aligned:
 * include/krk/quant.hpp:186-196, src/quant.cpp:1805-1900. */
int krk_dtype_block_size(int wt);
int krk_dtype_block_bytes(int wt);
int64_t krk_dtype_row_bytes(int wt, int64_t n);
int krk_dtype_row_aligned(int wt, int64_t n);

/* --------------------------------------------------------- hot operators -- */

/* Backend::gemm -- backend.hpp:859-860; HipBackend::gemm backend_hip.hip:3175.
 * out[rows, n_out] = x[rows, n_in] . W[n_out, n_in]^T.
 * rows == 1..8: fused dequant+dot GEMV with exact products and f32
 *               accumulation; Q4_K at rows == 1 forms the products on the
 *               int8 matrix cores from exact digit planes of x (rounded at
 *               2^-23 of each 32-value sub-block's maximum), and Q4_K at
 *               rows == 2..8 the same, the rows' digit tables built once per
 *               call in the handle's workspace (grown on the first such call).
 * rows  > 8   : per krk_set_gemm_path. */
int krk_gemm(krk_backend *b, void *out, const void *x, const void *w, int wt,
             int64_t n_out, int64_t n_in, int64_t rows);

/* krk_gemm without allocation.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory -- code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  Same
 * arguments, kernels and results as krk_gemm (bit-identical), but the
 * split-K partials, int8 activation codes and several-row digit tables that
 * krk_gemm keeps in the handle's growing workspace live in a fixed device array of
 * krk_gemm_noalloc_scratch_bytes() (64 MiB) instead: one per device, held
 * until the process ends, shared by every handle on that device.  The array
 * is part of the library's code object, so loading the library reserves
 * those 64 MiB on every device it runs on, whether or not this entry point
 * is ever called.  A call
 * whose scratch would exceed it returns KRK_ERR_NOMEM before any launch.
 * Calls that overlap on one device (several streams or threads) race on
 * that array; serialise them.  Nothing in the array needs to start at zero:
 * every call writes the scratch it reads. */
int krk_gemm_noalloc(krk_backend *b, void *out, const void *x, const void *w, int wt,
                     int64_t n_out, int64_t n_in, int64_t rows);
size_t krk_gemm_noalloc_scratch_bytes(void);

/* Backend::gemm_k_ok -- backend.hpp:869.  1 when a contraction of k columns
 * can be addressed (k > 0 and a multiple of 32; the weight type adds its own
 * block rule, see krk_dtype_row_aligned). */
int krk_gemm_k_ok(const krk_backend *b, int64_t k);

/* Backend::gemm_accumulate -- backend.hpp:894-901; backend_hip.hip:3121.
 * dst[rows, n_out] += x . W^T, the residual add folded into the projection.
 * rexp (nullable, device int32) is the decode row's storage exponent: the
 * contribution is multiplied by 2^-rexp[0] before the add.  *fused receives
 * 1 when the fused form ran (always for rows == 1; rows > 1 declines with
 * *fused = 0 and KRK_OK, and the caller falls back to gemm + add, as the
 * reference's engine does, engine.cpp:5197-5200). */
int krk_gemm_accumulate(krk_backend *b, void *dst, const void *x,
                        const void *w, int wt, int64_t n_out, int64_t n_in,
                        int64_t rows, const int32_t *rexp, int *fused);

/* Backend::gemm_group -- backend.hpp:1040-1054; backend_hip.hip:3491-3580.
 * n_mat projections sharing x (or each its own xs[m]) in ONE launch when
 * rows == 1.  silu != 0 asks for out[0] = silu(out[0]) * out[1] folded into
 * the epilogue (fused_gate_silu_kernel, fused.hpp:142-169); *silu_fused
 * reports whether it happened.  wts (nullable, host array) gives each
 * matrix its own type.  *fused receives 1 when the grouped launch ran.
 * out[], w[], n_out[], wts[], xs[] are HOST arrays of device pointers /
 * values. */
int krk_gemm_group(krk_backend *b, void *const out[], const void *x,
                   const void *const w[], int wt, const int64_t n_out[],
                   int64_t n_in, int n_mat, int64_t rows, int silu,
                   int *silu_fused, int row_parallel_only, const int wts[],
                   const void *const xs[], int *fused);

/* Backend::router_softmax -- backend.hpp:933-934.  probs f32 [n_rows,
 * n_expert] from logits in the activation type. */
int krk_router_softmax_supported(const krk_backend *b);
int krk_router_softmax(krk_backend *b, void *probs, const void *logits,
                       int64_t n_rows, int n_expert);

/* Backend::router_topk -- backend.hpp:949-950.  ids int32 / wts f32
 * [n_rows, k]; highest probability first, a tie keeps the lower id; weights
 * sum-normalized when normalize != 0, then multiplied by scale unless it is
 * 0 or 1 (engine.cpp:11853-11918). */
int krk_router_topk_supported(const krk_backend *b);
int krk_router_topk(krk_backend *b, const void *probs, int64_t n_rows,
                    int n_expert, int k, void *ids, void *wts, int normalize,
                    float scale);

/* Backend::scan_accum -- backend.hpp:955-972; backend_hip.hip:2455-2471.
 * Folds one layer's routing into cumulative device histograms (never
 * cleared here): hits u32 and mass f32, both [n_layer * n_expert];
 * hits[layer * n_expert + id] += 1 for every routed pair (ids int32
 * [n_rows, k], ids outside [0, n_expert) skipped) and
 * mass[layer * n_expert + e] += sum over rows of probs[row, e] (probs f32
 * [n_rows, n_expert]), one add per expert and call.  n_expert <= 1024. */
int krk_scan_accum_supported(const krk_backend *b);
int krk_scan_accum(krk_backend *b, const void *probs, const void *ids,
                   int64_t n_rows, int n_expert, int k, int layer, void *hits,
                   void *mass);

/* Backend::moe_plan_build -- backend.hpp:976-980; backend_hip.hip:2473-2485.
 * The layer's expert plan from device ids int32 [n_rows, k]: off int32
 * [n_expert + 1] prefix offsets; rows int32 and wt f32 [n_rows * k] in
 * expert-major order, each expert's pairs in (row, slot) order: rows[at] =
 * the pair's row, wt[at] = wts[pair] (0 when wts is null).  Entries past
 * off[n_expert] (dropped pairs) are not written.  n_expert <= 1024 (the
 * reference fills experts below 256 only). */
int krk_moe_plan_build(krk_backend *b, const void *ids, int64_t n_rows, int k,
                       int n_expert, void *off, void *rows, void *wt,
                       const void *wts);

/* Backend::moe_dispatch -- backend.hpp:1001-1009; backend_hip.hip:2494-2660.
 * The whole routed-expert FFN of one layer from device ids/wts through the
 * device table (table[layer * n_expert + e]):
 *   out[t] = sum over slots s (in ascending expert id) of
 *            wts[t,s] * down_e( silu(gate_e(xn[t])) * up_e(xn[t]) )
 * xn and out are [n_tok, n_embd] in the activation type; ids int32 and wts
 * f32 [n_tok, k] device arrays.  With f32 activations, batches of 32 tokens
 * or more whose banks are uniform Q4_K/Q5_K/Q6_K/Q8_0/Q4_0/MXFP4 (gate and
 * up of one type) form their products from f16 operands on the matrix
 * cores, as a gemm of more than 8 rows does, unless krk_set_gemm_path
 * selected KRK_PATH_EXACT.
 * The first call for a (table, layer, n_expert, n_embd, n_ff) reads that
 * layer's entries back once and validates every one: all three matrices
 * present, of a served type (types may vary from expert to expert and
 * between matrices), n_out / n_in equal to the layer's geometry, row_bytes equal to
 * krk_dtype_row_bytes(type, n_in), rows aligned for the type's loads.  Later
 * calls with the same key launch without a host round trip (and can be
 * graph-captured), so a table's layer must not change while the handle
 * remembers it.  The handle remembers up to 256 keys; past that the oldest
 * is dropped and is read and validated again on its next call (that call
 * blocks on the read-back and cannot be captured). */
int krk_moe_dispatch_supported(const krk_backend *b);
int krk_moe_dispatch(krk_backend *b, const void *table, int layer,
                     int n_expert, const void *ids, const void *wts,
                     const void *xn, void *out, int64_t n_tok, int64_t n_embd,
                     int64_t n_ff, int k);

/* Forget the validations remembered for every layer of `table` (call it
 * before a dispatched table is rewritten or freed, so that a new table at
 * the same address is read and checked again).  No counterpart in the
 * reference, whose dispatch keeps no host-side record of the table. */
int krk_moe_table_forget(krk_backend *b, const void *table);

/* ------------------------------------------------ dequant / quantize ops -- */

/* dequant_row (quant.hpp:203) on the device: out f32 [n_rows, n_in],
 * bit-identical to the reference's host decoders. */
int krk_dequant_rows_f32(krk_backend *b, float *out, const void *w, int wt,
                         int64_t n_rows, int64_t n_in);
/* The same values rounded to f16 (round to nearest even). */
int krk_dequant_rows_f16(krk_backend *b, void *out, const void *w, int wt,
                         int64_t n_rows, int64_t n_in);
/* quantize_q8_row (quant.hpp:398; quant.cpp:2167-2197) on the device for
 * rows of f32 activations: xq int8 [rows, n], dx f32 [rows, n/32]. */
int krk_quantize_q8_rows(krk_backend *b, const float *x, int64_t rows,
                         int64_t n, int8_t *xq, float *dx);

/* ------------------------------------------- synthetic inputs (host side) -- */
/* Seeded generators for the benchmark configurations.  All host memory.
 * normal: v[i] = mean + std * N(0,1) from a counter-based splitmix64 stream
 * and Box-Muller in f64, so value i depends on (seed, i) only. */
void krk_synth_normal(float *v, int64_t n, uint64_t seed, float mean,
                      float std, int nthreads);
/* Row quantizers, n a multiple of the block size.  Q8_0 / Q4_0 follow the
 * reference's fixture generator (tools/make_bench_gguf.py:191-218); the
 * reference has no Q4_K / Q6_K quantizer, these are this library's own. */
int krk_quantize_weights(int wt, const float *v, int64_t n_rows, int64_t n_in,
                         void *dst, int nthreads);

#ifdef __cplusplus
}
#endif
#endif /* KRK_MI355X_H */
