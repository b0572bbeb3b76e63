// krk_kernels.hpp -- internal interface between the C-ABI layer (backend.cpp)
// and the kernel translation units.  Host-side launchers only; no HIP types
// beyond hipStream_t / hipError_t cross this line.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace krk {

// One projection inside a grouped GEMV launch (the reference's FusedLayer,
// src/hip/kernels/fused.hpp:48-65).
enum : int { SEG_PLAIN = 0, SEG_ACC = 1, SEG_SILU = 2 };

struct Seg {
    const void *w;        // weight rows (gate rows for SEG_SILU)
    const void *w2;       // up rows for SEG_SILU, else null
    const void *x;        // activation rows
    void *out;            // output rows
    int64_t n_out;
    int64_t blk_begin;    // first workgroup of this segment (set by the launcher)
    int kind;
    int _pad;
};

constexpr int kMaxSegs = 8;

// One active expert of a routed layer: its gate, up and down banks and its
// plan positions [pb, pe) (written by the MoE plan on the device)
struct EmRun {
    const void *w[3];
    int32_t pb, pe;
};

struct SegTable {
    Seg seg[kMaxSegs];
    int n;               // segments in use
    int n_in;            // shared K
    int64_t row_bytes;   // shared (one dtype per launch)
    int64_t rows;        // activation rows
    int64_t x_stride;    // elements between activation rows
    int64_t out_stride;  // elements between output rows
    const int32_t *rexp; // SEG_ACC exponent (nullable)
    // Routed experts (moe_tab nullable).  Gate/up mode (moe_down == 0):
    // segment i's gate / up pointers are read on the device from
    // moe_tab[moe_ids[i]] (krk_moe_entry) instead of seg[i].w / w2, and
    // seg[i].out is seg[0].out + i * seg[0].n_out.  Down mode (moe_down == 1):
    // one segment whose K is moe_k slots of moe_kslot values; slot s's part of
    // every row lies in the down bank of expert moe_ids[s] (row stride
    // row_bytes) and its activations are scaled by moe_wts[s]; a dropped slot
    // (id outside [0, moe_ne)) contributes zero.
    const void *moe_tab;
    const int32_t *moe_ids;
    const float *moe_wts;
    int moe_ne;
    int moe_down;
    int moe_k;
    int64_t moe_kslot;
    // Several tokens (moe_tokens > 1): the grid is moe_tokens groups of
    // moe_wpt workgroups; group tk handles token tk: its ids and weights at
    // moe_ids / moe_wts + tk * k, its activations at seg[0].x + tk * moe_xtok
    // elements and its outputs at seg[0].out + tk * moe_otok elements.
    int moe_tokens;
    int moe_wpt;
    int64_t moe_xtok, moe_otok;
    // Expert-major rows (with em_runs below): activation rows seg[0].x row
    // em_tok[p] (row p when em_tok is null) of em_xrow elements, outputs
    // seg[0].out row p of em_orow elements; em_max_items bounds the runs.
    const int32_t *em_tok;
    int em_max_items;
    int64_t em_xrow, em_orow;
    // Expert-major runs (em_runs nullable; the register-streaming kernel,
    // with moe_tab and one segment): grid row a serves run em_runs[a] while
    // a < *em_n_act (em_max_items bounds the rows).  Its weights are the
    // run's gate/up pair (SEG_SILU) or down bank (SEG_PLAIN), loaded once for
    // all of its rows: plan positions p = pb .. pe - 1, activations seg[0].x
    // row em_tok[p] (row p when em_tok is null), outputs seg[0].out row p.
    const EmRun *em_runs;
    const int32_t *em_n_act;
    // Dense launches of 2..8 activation rows on the streaming kernel: device
    // scratch of gemv_stream_xtab_bytes(rows, n_in) for the rows' digit
    // tables, built once per call (nullable: then those launches take the
    // other kernels)
    uint8_t *xtab;
};

hipError_t gemv_segments(int dt, bool act_f16, const SegTable &t, hipStream_t st);
// Q4_K, Q6_K, Q4_0 and Q8_0, one activation row (or the rows of expert-major
// runs): every weight byte of a tile loaded into registers up front, digit
// planes per wave (gemv_stream.hip)
bool gemv_stream_ok(int dt, const SegTable &t);
// scratch bytes of the several-row streaming launches' digit tables
size_t gemv_stream_xtab_bytes(int64_t rows, int64_t n_in);
hipError_t gemv_stream(int dt, bool act_f16, const SegTable &t, hipStream_t st);
// Q4_K / Q6_K rows 1..8 on the int8 MFMA (activations as exact int8 digit planes)
bool gemv_digits_ok(int dt, const SegTable &t);
hipError_t gemv_digits(int dt, bool act_f16, const SegTable &t, hipStream_t st);

// Bit-exact dequantization (the chunk contract) to f32 / f16 (RNE).
hipError_t dequant_rows(int dt, const void *w, int64_t row_bytes, int64_t n_rows,
                        int64_t n_in, void *out, bool to_f16, hipStream_t st);

// Activation quantizer, quant.cpp:2167-2197 semantics.  x in f32 or f16.
hipError_t quantize_q8_rows(const void *x, bool x_f16, int64_t rows, int64_t n,
                            int8_t *xq, float *dx, hipStream_t st);
hipError_t quantize_q8_rows_f16codes(const void *x, bool x_f16, int64_t rows, int64_t n,
                                     _Float16 *xq, float *dx, float *sx16, hipStream_t st);

// Prefill GEMM (f16 MFMA, f32 accumulate) and the Q8_0 x Q8 int8 MFMA rung.
// out[M, N] = X[M, K] . deq(W)[N, K]^T.  `ws` is device scratch of ws_bytes.
// scratch of gemm_mfma: what its fastest form needs, or (minimal) the
// least it runs with
size_t gemm_mfma_workspace(int dt, int64_t M, int64_t N, int64_t K, bool minimal);
// compute units of the current device (cached on first use)
int device_cus();
// cnt: kTileCounters zeroed counters owned by the caller (left zero after
// every call), which let a two-way split-K launch sum its splits inside the
// GEMM; null keeps the separate reduce kernel.  Calls sharing counters must
// not overlap.
constexpr int kTileCounters = 4096;
hipError_t gemm_mfma(int dt, const void *w, int64_t row_bytes, const void *x, bool act_f16,
                     void *out, int64_t M, int64_t N, int64_t K, void *ws, size_t ws_bytes,
                     unsigned *cnt, hipStream_t st);
// Grouped expert GEMM on the f16 MFMA: one launch per projection over the
// MoE plan's items {expert, first plan position, rows <= 32 mi, 0}; X holds
// f16 activation rows in plan order [P, K].  Gate/up: out = f16 rows
// silu(gate) * up per plan position [P, n_ff]; down: out = f32 part rows
// per plan position [P, n_embd].  moe_gather_f16 writes f16 rows: with
// plan_tok, xg[pos] = f16(x[plan_tok[pos]]) for pos < *n_live; without,
// xg[pos] = f16(x[pos]).
struct MoeGemmArgs {
    const void *tab;           // krk_moe_entry[n_expert] of the layer
    const int32_t *items;      // 4 per item
    const int32_t *n_items;    // [1]
    const void *x;
    void *out;
    int64_t row_bytes;         // gate = up row size (gate/up), down row size
    int K, N;                  // K = n_embd, N = n_ff (gate/up); K = n_ff, N = n_embd (down)
    int max_items;             // items the grid covers (an upper bound)
    int mi;                    // item rows = 32 mi, mi in {1, 2}
    bool gate_up;
    // dense mode (w non-null, items unused, not gate/up): one weight matrix,
    // items of 32 mi of the M rows of X, out [M, N] in f32 or f16
    const void *w;
    int M;
    bool out_f16;
    int ksplit;                // dense: K in ksplit whole-block ranges, f32 partials [ksplit][M][N] at out
    const int32_t *xtok;       // non-null: plan position p's activation row is x row xtok[p] (gate/up on
                               // the tokens' rows); null: x rows in plan order
};
bool moe_gemm_ok(int dt);
hipError_t moe_gemm(int dt, const MoeGemmArgs &a, hipStream_t st);
hipError_t moe_gather_f16(const float *x, int64_t n, const int32_t *plan_tok, const int32_t *n_live,
                          int64_t max_rows, _Float16 *xg, hipStream_t st);
size_t gemm_int8_workspace(int64_t M, int64_t K);
bool gemm_int8_serves(int wt);
hipError_t gemm_int8(int wt, const void *w, int64_t row_bytes, const void *x, bool act_f16, void *out,
                     int64_t rows, int64_t n_out, int64_t n_in, void *ws, size_t ws_bytes, hipStream_t st);

// Router and MoE dispatch.
hipError_t router_softmax(const void *logits, bool act_f16, float *probs, int64_t n_rows,
                          int n_expert, hipStream_t st);
hipError_t router_topk(const float *probs, int64_t n_rows, int n_expert, int k, int32_t *ids,
                       float *wts, int normalize, float scale, hipStream_t st);
hipError_t moe_plan_build(const int32_t *ids, int64_t n_rows, int k, int n_expert, int32_t *off,
                          int32_t *rows, float *wt, const float *wts, hipStream_t st);
hipError_t scan_accum(const float *probs, const int32_t *ids, int64_t n_rows, int n_expert, int k, int layer,
                      unsigned *hits, float *mass, hipStream_t st);

struct MoeArgs {
    const void *table;   // krk_moe_entry[n_layer * n_expert]
    int layer, n_expert, k;
    const int32_t *ids;
    const float *wts;
    const void *xn;
    void *out;
    int64_t n_tok, n_embd, n_ff;
    bool act_f16;
    int wt;              // the experts' gate / up weight type
    int wt_down;         // the experts' down weight type
    int64_t rb_gate, rb_up, rb_down;
    bool aligned16;      // every bank's rows start 16-byte aligned
    bool mfma;           // the gemm path allows f16 MFMA products (not KRK_PATH_EXACT)
};
size_t moe_workspace(int64_t n_tok, int k, int n_expert, int64_t n_embd, int64_t n_ff);
hipError_t moe_dispatch(const MoeArgs &a, void *ws, size_t ws_bytes, hipStream_t st);

}  // namespace krk
