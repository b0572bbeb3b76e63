/*
 * krk_oracle.h -- CPU restatement of Kraken's scalar f32 reference for the
 * quantized weight-math path.  TEST INFRASTRUCTURE ONLY: the product library
 * (kraken_amd/) never links, loads or calls anything declared here.  Tests,
 * the smoke check and the bench's cpu_baseline leg use it as the checker.
 *
 * Every function cites the reference file:line it restates.  Built with
 * -O3 -ffp-contract=off so that the only fused multiply-adds are the explicit
 * fmaf() calls, which stand where the reference build (g++ -O3 -mfma, GNU
 * default -ffp-contract=fast) contracts.
 */
#ifndef KRK_ORACLE_H
#define KRK_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids (include/krk/quant.hpp:16-34). */
enum {
    ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_0 = 2, ORC_Q8_0 = 8,
    ORC_Q2_K = 10, ORC_Q3_K = 11, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14, ORC_IQ4_NL = 20, ORC_IQ4_XS = 23, ORC_MXFP4 = 39,
    ORC_Q4_1 = 3, ORC_Q5_0 = 6, ORC_Q5_1 = 7, ORC_BF16 = 30,
    /* include/krk/quant.hpp:25-31, 67-68, 105, 128-129, 166-168 */
    ORC_Q8_1 = 9, ORC_Q8_K = 15, ORC_TQ1_0 = 34, ORC_TQ2_0 = 35, ORC_NVFP4 = 40,
    ORC_ROCMFP4 = 100, ORC_ROCMFP4_FAST = 101, ORC_Q6_0_ROCMFPX = 102, ORC_Q3_0_ROCMFPX = 104,
    ORC_Q2_0_ROCMFPX = 107, ORC_Q1_0 = 41, ORC_Q2_0 = 42, ORC_Q2_0_64 = 48, ORC_PQ2_0 = 142, ORC_PTQ1_0 = 143
};

float    orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16(float f);

int      orc_block_size(int dt);
int      orc_block_bytes(int dt);
int64_t  orc_row_bytes(int dt, int64_t n);

void     orc_dequant_row(int dt, const void *src, float *out, int64_t n);
void     orc_dequant_row_f16(int dt, const void *src, uint16_t *out, int64_t n);
float    orc_vec_dot(int dt, const void *src, const float *x, int64_t n);

/* out[r*n_out + o] = vec_dot(W[o], x[r]) for o in [0,n_out), r in [0,rows). */
void     orc_gemm(float *out, const float *x, const void *w, int dt,
                  int64_t n_out, int64_t n_in, int64_t rows, int nthreads);

void     orc_quantize_q8_row(const float *x, int64_t n, int8_t *xq, float *dx);
float    orc_dot_q8_0_q8(const void *w, const int8_t *xq, const float *dx,
                         int64_t n);
float    orc_dot_kq_q8(int dt, const void *w, const int8_t *xq, const float *dx, int64_t n);
void     orc_gemm_int8(int dt, float *out, const float *x, const void *w,
                       int64_t n_out, int64_t n_in, int64_t rows, int nthreads);
void     orc_gemm_q8_0_q8(float *out, const float *x, const void *w,
                          int64_t n_out, int64_t n_in, int64_t rows,
                          int nthreads);

void     orc_silu_mul(float *out, const float *g, const float *u, int64_t n);
void     orc_router_softmax(float *probs, const float *logits, int64_t n_rows,
                            int n_expert);
void     orc_router_topk(const float *probs, int64_t n_rows, int n_expert,
                         int k, int32_t *ids, float *wts, int normalize,
                         float scale);

/* Routed-expert FFN on the host: experts visited in ascending id, each one's
 * rows gathered in token-then-slot order.  gate/up/down are arrays of
 * n_expert host pointers (raw GGUF bytes) of types wt_gate/wt_up/wt_down. */
void     orc_moe_ffn(float *out, const float *x, const void *const *gate,
                     const void *const *up, const void *const *down,
                     int wt_gate, int wt_up, int wt_down,
                     const int32_t *ids, const float *wts, int64_t n_tok,
                     int64_t n_embd, int64_t n_ff, int n_expert, int k,
                     int nthreads);

/* The reference GPU backend's f16 expert FFN (moe_table.hpp:230-305,
 * 418-441, 536-551): row-scaled f16 activations into down, f16 partials
 * added in slot order with an f16 rounding after every add.  x holds f16
 * values; out receives f16 bits. */
void     orc_moe_ffn_f16(uint16_t *out, const float *x, const void *const *gate,
                         const void *const *up, const void *const *down,
                         int wt_gate, int wt_up, int wt_down,
                         const int32_t *ids, const float *wts, int64_t n_tok,
                         int64_t n_embd, int64_t n_ff, int n_expert, int k,
                         int nthreads);

/* Fixture generator restated from tools/make_bench_gguf.py:191-202 (q8_0). */
void     orc_quantize_q8_0_weights(const float *v, int64_t n, uint8_t *dst);

#ifdef __cplusplus
}
#endif
#endif
