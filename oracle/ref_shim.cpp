// ref_shim.cpp -- extern "C" entry points over the REFERENCE's own host quant
// code (src/quant.cpp + src/common.cpp, compiled from /root/reference by
// oracle/Makefile into oracle/_ref/libkrk_ref.so).  Test infrastructure: it
// exists so the C restatement in krk_oracle.c can be compared bit for bit
// with the reference where the reference builds.  The strict scalar tier is
// selected the way the reference's own switches select it
// (include/krk/quant.hpp:245-273): fast, avx2 and int8 tiers off.
#include "krk/quant.hpp"

using namespace krk;

static void strict_tier() {
    set_vec_dot_fast(false);
    set_vec_dot_avx2(false);
    set_vec_dot_int8(false);
    set_vec_dot_wide(false);
}

extern "C" {
int64_t ref_row_bytes(int dt, int64_t n) {
    return static_cast<int64_t>(dtype_row_bytes(static_cast<DType>(dt), n));
}
int ref_block_size(int dt) { return dtype_block_size(static_cast<DType>(dt)); }
int ref_block_bytes(int dt) { return dtype_block_bytes(static_cast<DType>(dt)); }
void ref_dequant_row(int dt, const void *src, float *out, int64_t n) {
    dequant_row(static_cast<DType>(dt), src, out, n);
}
void ref_dequant_row_f16(int dt, const void *src, uint16_t *out, int64_t n) {
    dequant_row_f16(static_cast<DType>(dt), src, out, n);
}
float ref_vec_dot(int dt, const void *src, const float *x, int64_t n) {
    strict_tier();
    return vec_dot(static_cast<DType>(dt), src, x, n);
}
void ref_quantize_q8_row(const float *x, int64_t n, int8_t *xq, float *dx) {
    quantize_q8_row(x, n, xq, dx);
}
float ref_dot_q8_0_q8_scalar(const void *w, const int8_t *xq, const float *dx,
                             int64_t n) {
    return dot_q8_0_q8_scalar(static_cast<const u8 *>(w), xq, dx, n);
}
float ref_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }
uint16_t ref_fp32_to_fp16(float f) { return fp32_to_fp16(f); }
}
