/*
 * krk_oracle.c -- CPU restatement of Kraken's scalar f32 reference for the
 * quantized weight-math path (Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K / IQ4_NL / IQ4_XS dequant, the strict
 * single-chain GEMV dot, the Q8 activation quantizer and integer dot, the
 * host MoE routing and the routed-expert FFN).
 *
 * TEST INFRASTRUCTURE: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this library, and only as the checker.
 *
 * Compiled with -ffp-contract=off.  The reference is built with g++ -O3 -mfma
 * (CMakeLists.txt:35-37), where GCC MAY contract a*b+c into one FMA; each place
 * where it does (checked against the reference built from its own sources:
 * Q4_K's d1*q-m1, where it is exact either way, and scatter_axpy_rows'
 * dst += a*src) is written here as an
 * explicit fmaf(), and nothing else is fused.
 *
 * Pinning (see tests/test_oracle.py): the reference's own known-answer tests
 * (tests/test_kraken.cpp:396-1042, 2087, 8143), closed forms and brute force
 * in f64, committed golden vectors (tests/golden/), and, where
 * oracle/_ref/libkrk_ref.so was built from the reference sources, a bitwise
 * comparison against the reference itself.
 */
#include "krk_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* src/common.cpp:161-187 */
float orc_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            uint32_t mm = m;
            int ee = -1;
            do { mm <<= 1; ee++; } while (!(mm & 0x400u));
            mm &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - ee) << 23) | (mm << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* src/common.cpp:189-208.  Restated as written, including its tie rule: the
 * second rounding clause can never hold (it needs bit 13 both clear and set),
 * so an exact halfway case in the normal range is truncated rather than
 * rounded to even.  Only dequant_row_f16 uses this; the device f16 path is
 * compared against an RNE conversion instead. */
uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    int32_t e = (int32_t)((x >> 23) & 0xFFu) - 127 + 15;
    uint32_t m = x & 0x7FFFFFu;
    if (((x >> 23) & 0xFFu) == 0xFFu)
        return (uint16_t)(sign | 0x7C00u | (m ? 0x200u : 0));
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        int sh = 14 - e;
        uint32_t mm = m | 0x800000u;
        uint32_t half = mm >> sh;
        uint32_t rem = mm & ((1u << sh) - 1);
        uint32_t thresh = 1u << (sh - 1);
        if (rem > thresh || (rem == thresh && (half & 1))) half++;
        return (uint16_t)(sign | (half & 0x7FFu));
    }
    uint32_t half = ((uint32_t)e << 10) | (m >> 13);
    if ((m & 0x1FFFu) > 0x1000u || ((m & 0x3FFFu) == 0x1000u && (half & 1))) half++;
    return (uint16_t)(sign | (half & 0x7FFFu));
}

static inline float ld_f16(const uint8_t *p) {
    return orc_fp16_to_fp32((uint16_t)(p[0] | (p[1] << 8)));
}

/* Geometry: src/quant.cpp:1805-1900 (block size / bytes), 1891-1895 (row). */
int orc_block_size(int dt) {
    switch (dt) {
        case ORC_F32: case ORC_F16: case ORC_BF16: return 1;
        case ORC_Q4_0: case ORC_Q8_0: case ORC_IQ4_NL: case ORC_MXFP4:
        case ORC_Q4_1: case ORC_Q5_0: case ORC_Q5_1: return 32;
        case ORC_Q8_1: case ORC_ROCMFP4: case ORC_ROCMFP4_FAST: case ORC_Q6_0_ROCMFPX:
        case ORC_Q3_0_ROCMFPX: case ORC_Q2_0_ROCMFPX: return 32;
        case ORC_NVFP4: case ORC_Q2_0_64: return 64;
        case ORC_Q1_0: case ORC_Q2_0: case ORC_PQ2_0: case ORC_PTQ1_0: return 128;
        case ORC_Q2_K: case ORC_Q3_K: case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_IQ4_XS: return 256;
        case ORC_Q8_K: case ORC_TQ1_0: case ORC_TQ2_0: return 256;
        default: return 0;
    }
}
int orc_block_bytes(int dt) {
    switch (dt) {
        case ORC_F32: return 4;
        case ORC_F16: case ORC_BF16: return 2;
        case ORC_Q4_0: case ORC_IQ4_NL: return 18;
        case ORC_Q8_0: return 34;
        case ORC_MXFP4: return 17;
        case ORC_Q4_1: return 20;
        case ORC_Q5_0: return 22;
        case ORC_Q5_1: return 24;
        case ORC_Q2_K: return 84;
        case ORC_Q3_K: return 110;
        case ORC_Q4_K: return 144;
        case ORC_Q5_K: return 176;
        case ORC_IQ4_XS: return 136;
        case ORC_Q6_K: return 210;
        case ORC_Q8_1: return 36;
        case ORC_Q8_K: return 292;
        case ORC_TQ1_0: return 54;
        case ORC_TQ2_0: return 66;
        case ORC_NVFP4: return 36;
        case ORC_ROCMFP4: return 18;
        case ORC_ROCMFP4_FAST: return 17;
        case ORC_Q6_0_ROCMFPX: return 26;
        case ORC_Q3_0_ROCMFPX: return 14;
        case ORC_Q2_0_ROCMFPX: return 10;
        case ORC_Q1_0: case ORC_Q2_0_64: return 18;
        case ORC_Q2_0: case ORC_PQ2_0: return 34;
        case ORC_PTQ1_0: return 28;
        default: return 0;
    }
}
int64_t orc_row_bytes(int dt, int64_t n) {
    int bs = orc_block_size(dt);
    if (bs <= 0) return 0;
    return ((n + bs - 1) / bs) * (int64_t)orc_block_bytes(dt);
}

/* src/quant.cpp:331-339 */
static void deq_q4_0(const uint8_t *b, float *y) {
    float d = ld_f16(b);
    for (int k = 0; k < 16; k++) {
        y[k] = d * (float)((int)(b[2 + k] & 0xF) - 8);
        y[k + 16] = d * (float)((int)(b[2 + k] >> 4) - 8);
    }
}

/* IQ4_NL's non-linear grid: ggml's kvalues_iq4nl, a constant of the format
 * (src/quant.cpp:88-91). */
static const int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                  1, 13, 25, 38, 53, 69, 89, 113};

/* src/quant.cpp:566-574: Q4_0's layout, each nibble an index into the grid,
 * value d * grid[q] (one product). */
static void deq_iq4_nl(const uint8_t *b, float *y) {
    float d = ld_f16(b);
    for (int k = 0; k < 16; k++) {
        y[k] = d * (float)kIq4nl[b[2 + k] & 0xF];
        y[k + 16] = d * (float)kIq4nl[b[2 + k] >> 4];
    }
}

/* src/quant.cpp:641-659: 256 values in eight sub-blocks of 32, each with a
 * 6-bit scale ls (low 4 bits in scales_l, high 2 in scales_h) and IQ4_NL
 * grid indices; value (d * (ls - 32)) * grid[q]: the first product is exact
 * (11 + 6 bits), the second rounds. */
static void deq_iq4_xs(const uint8_t *b, float *y) {
    float d = ld_f16(b);
    uint16_t sh = (uint16_t)(b[2] | (b[3] << 8));
    const uint8_t *sl = b + 4, *qs = b + 8;
    for (int ib = 0; ib < 8; ib++, y += 32, qs += 16) {
        int ls = ((sl[ib / 2] >> (4 * (ib % 2))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4);
        float dl = d * (float)(ls - 32);
        for (int j = 0; j < 16; j++) {
            y[j] = dl * (float)kIq4nl[qs[j] & 0xF];
            y[j + 16] = dl * (float)kIq4nl[qs[j] >> 4];
        }
    }
}

/* src/quant.cpp:398-423.  84 B / 256: 16 scale bytes (low nibble scale,
 * high nibble min), 64 bytes of 2-bit codes, f16 d at 80 and dmin at 82.
 * Value index 128g + 32j + 16s + l takes bits 2j of qs[32g + 16s + l] and
 * scale byte 8g + 2j + s; value (d*sc)*q - dmin*m, where d*sc (<= 15 bits)
 * and its product with q (<= 17) are exact, so only the subtraction rounds
 * and an FMA gives the same bits. */
static void deq_q2_k(const uint8_t *b, float *y) {
    float d = ld_f16(b + 80), dmin = ld_f16(b + 82);
    for (int g = 0; g < 2; g++)
        for (int j = 0; j < 4; j++)
            for (int s = 0; s < 2; s++) {
                uint8_t sc = b[8 * g + 2 * j + s];
                float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
                const uint8_t *q = b + 16 + 32 * g + 16 * s;
                float *yy = y + 128 * g + 32 * j + 16 * s;
                for (int l = 0; l < 16; l++) yy[l] = fmaf(dl, (float)((q[l] >> (2 * j)) & 3), -ml);
            }
}

/* Q3_K 6-bit scale i (0..15) from the 12 packed bytes (quant.cpp:520-528):
 * low 4 bits from byte i (i < 8) or the high nibble of byte i - 8, high 2
 * bits from byte 8 + i % 4 at bit 2 (i / 4). */
static int q3k_scale(const uint8_t *r, int i) {
    int lo = i < 8 ? (r[i] & 0xF) : (r[i - 8] >> 4);
    int hi = (r[8 + (i & 3)] >> (2 * (i >> 2))) & 3;
    return lo | (hi << 4);
}

/* src/quant.cpp:514-554.  110 B / 256: hmask[32], 2-bit qs[64], 12 bytes of
 * 6-bit scales, f16 d at 108.  Value index 128n + 32j + 16s + l: code
 * (qs[32n + 16s + l] >> 2j) & 3, minus 4 unless bit 4n + j of
 * hmask[16s + l] is set; scale 8n + 2j + s; value (d*(sc - 32))*code, the
 * first product exact (11 + 6 bits), the second rounding once. */
static void deq_q3_k(const uint8_t *b, float *y) {
    float d = ld_f16(b + 108);
    const uint8_t *hm = b, *qs = b + 32, *sr = b + 96;
    for (int n = 0; n < 2; n++)
        for (int j = 0; j < 4; j++)
            for (int s = 0; s < 2; s++) {
                float dl = d * (float)(q3k_scale(sr, 8 * n + 2 * j + s) - 32);
                const uint8_t *q = qs + 32 * n + 16 * s;
                float *yy = y + 128 * n + 32 * j + 16 * s;
                for (int l = 0; l < 16; l++) {
                    int c = ((q[l] >> (2 * j)) & 3) - ((hm[16 * s + l] >> (4 * n + j)) & 1 ? 0 : 4);
                    yy[l] = dl * (float)c;
                }
            }
}

/* src/quant.cpp:83-86, 319-330, 674-686.  17 B / 32: an E8M0 exponent byte
 * e, then 16 bytes of E2M1 codes (value j the low nibble of byte j, j + 16
 * the high).  The FP4 grid is doubled (0, 1, 2, 3, 4, 6, 8, 12 and their
 * negatives), so the exponent decodes at half scale: d = 2^(e - 128)
 * exactly, e = 0 and 1 being the f32 denormals 2^-128 and 2^-127.  Value
 * grid[q] * d, one rounding (overflow to inf for the largest e). */
static const int8_t kFp4[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
static float e8m0_half(uint8_t e) {
    uint32_t bits = e < 2 ? (0x00200000u << e) : ((uint32_t)(e - 1) << 23);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
static void deq_mxfp4(const uint8_t *b, float *y) {
    float d = e8m0_half(b[0]);
    for (int j = 0; j < 16; j++) {
        y[j] = (float)kFp4[b[1 + j] & 0xF] * d;
        y[j + 16] = (float)kFp4[b[1 + j] >> 4] * d;
    }
}

/* src/quant.cpp:341-378: the legacy 32-value formats.  Q4_1 (20 B): f16 d,
 * f16 m, 16 code bytes, value d*q + m.  Q5_0 (22 B): f16 d, a 32-bit plane
 * qh (bit k is bit 4 of value k's code), 16 code bytes, value d*(q - 16).
 * Q5_1 (24 B): d, m, qh, codes, value d*q + m.  Value k is the low nibble
 * of code byte k, value k + 16 the high nibble.  d*q is exact (<= 16
 * significant bits), so the one rounding is the add's and an FMA agrees. */
static void deq_l32(const uint8_t *b, float *y, int has_m, int qh_off, int qs_off, int bias) {
    float d = ld_f16(b), m = has_m ? ld_f16(b + 2) : 0.0f;
    uint32_t qh = 0;
    if (qh_off >= 0) qh = (uint32_t)b[qh_off] | ((uint32_t)b[qh_off + 1] << 8) |
                          ((uint32_t)b[qh_off + 2] << 16) | ((uint32_t)b[qh_off + 3] << 24);
    for (int k = 0; k < 16; k++) {
        int lo = (b[qs_off + k] & 0xF) | (int)(((qh >> k) & 1u) << 4);
        int hi = (b[qs_off + k] >> 4) | (int)(((qh >> (k + 16)) & 1u) << 4);
        if (has_m) {
            y[k] = fmaf(d, (float)lo, m);
            y[k + 16] = fmaf(d, (float)hi, m);
        } else {
            y[k] = d * (float)(lo - bias);
            y[k + 16] = d * (float)(hi - bias);
        }
    }
}

/* src/quant.cpp:381-387 */
static void deq_q8_0(const uint8_t *b, float *y) {
    float d = ld_f16(b);
    for (int k = 0; k < 32; k++) y[k] = d * (float)(int8_t)b[2 + k];
}

/* src/quant.cpp:427-435 */
static void scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = (uint8_t)(q[j] & 63);
        *m = (uint8_t)(q[j + 4] & 63);
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* src/quant.cpp:437-460.  `d1 * q - m1` is contracted to one FMA by the
 * reference build (vfmsub in dequant_block), hence fmaf(d1, q, -m1).  The
 * contraction is immaterial here: d1 = d*sc carries at most 17 significant
 * bits and d1*q at most 21, so the product is exact and both forms round
 * only the subtraction (tests/test_oracle.py checks this). */
static void deq_q4_k(const uint8_t *b, float *y) {
    float d = ld_f16(b), dmin = ld_f16(b + 2);
    const uint8_t *sc = b + 4, *q = b + 16;
    for (int j = 0, is = 0; j < 256; j += 64, is += 2, q += 32) {
        uint8_t si, mi;
        scale_min_k4(is, sc, &si, &mi);
        float d1 = d * (float)si, m1 = dmin * (float)mi;
        scale_min_k4(is + 1, sc, &si, &mi);
        float d2 = d * (float)si, m2 = dmin * (float)mi;
        for (int l = 0; l < 32; l++) {
            y[j + l] = fmaf(d1, (float)(q[l] & 0xF), -m1);
            y[j + l + 32] = fmaf(d2, (float)(q[l] >> 4), -m2);
        }
    }
}

/* src/quant.cpp:462-489.  Q4_K's header and scales, then 32 high-bit bytes
 * qh and 128 code bytes: chunk pair j takes bit 2j of qh[l] as bit 4 of its
 * low-nibble code and bit 2j+1 for its high-nibble code.  As in Q4_K the
 * product d1*q is exact (at most 17 + 5 significant bits), so the FMA the
 * reference build forms and a separate multiply agree. */
static void deq_q5_k(const uint8_t *b, float *y) {
    float d = ld_f16(b), dmin = ld_f16(b + 2);
    const uint8_t *sc = b + 4, *qh = b + 16, *q = b + 48;
    for (int j = 0, is = 0; j < 256; j += 64, is += 2, q += 32) {
        uint8_t si, mi;
        scale_min_k4(is, sc, &si, &mi);
        float d1 = d * (float)si, m1 = dmin * (float)mi;
        scale_min_k4(is + 1, sc, &si, &mi);
        float d2 = d * (float)si, m2 = dmin * (float)mi;
        for (int l = 0; l < 32; l++) {
            int lo = (q[l] & 0xF) | (((qh[l] >> is) & 1) << 4);
            int hi = (q[l] >> 4) | (((qh[l] >> (is + 1)) & 1) << 4);
            y[j + l] = fmaf(d1, (float)lo, -m1);
            y[j + l + 32] = fmaf(d2, (float)hi, -m2);
        }
    }
}

/* src/quant.cpp:491-512.  `d * sc * (q - 32)` is (d*sc)*(q-32): two products,
 * nothing to contract. */
static void deq_q6_k(const uint8_t *b, float *y) {
    float d = ld_f16(b + 208);
    for (int n = 0; n < 256; n += 128) {
        const uint8_t *ql = b + n / 2, *qh = b + 128 + n / 4;
        const int8_t *sc = (const int8_t *)(b + 192) + n / 16;
        float *yy = y + n;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4);
            int q2 = (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4);
            int q3 = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
            int q4 = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4);
            yy[l] = d * (float)sc[is + 0] * (float)(q1 - 32);
            yy[l + 32] = d * (float)sc[is + 2] * (float)(q2 - 32);
            yy[l + 64] = d * (float)sc[is + 4] * (float)(q3 - 32);
            yy[l + 96] = d * (float)sc[is + 6] * (float)(q4 - 32);
        }
    }
}

/* ---- formats served through the generic 32-value chunk path ---------- */

/* src/quant.cpp:389-396: Q8_1 (36 B): f16 d, f16 s, 32 int8 codes; value
 * d*q + s, the product rounded before the add (unfused in the reference
 * build, and here: this file is built with -ffp-contract=off). */
static void deq_q8_1(const uint8_t *b, float *y) {
    float d = ld_f16(b), s = ld_f16(b + 2);
    for (int k = 0; k < 32; k++) y[k] = d * (float)(int8_t)b[4 + k] + s;
}

/* src/quant.cpp:557-564: Q8_K (292 B): f32 d, 256 int8 codes, then 16 int16
 * block sums the decoder does not read; value d*q. */
static void deq_q8_k(const uint8_t *b, float *y) {
    float d;
    memcpy(&d, b, 4);
    for (int k = 0; k < 256; k++) y[k] = d * (float)(int8_t)b[4 + k];
}

/* src/quant.cpp:576-585: a UE4M3 scale byte; 0x00 and 0x7F are 0, bit 7 is
 * not read; exponent field 0 is man * 2^-9, else (1 + man/8) * 2^(exp-7);
 * both halved. */
static float ue4m3(uint8_t x) {
    if (x == 0 || x == 0x7F) return 0.0f;
    int e = (x >> 3) & 0xF, m = x & 7;
    float raw = e == 0 ? ldexpf((float)m, -9) : ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return raw * 0.5f;
}

/* src/quant.cpp:661-672: NVFP4 (36 B / 64 values): four UE4M3 scales, then
 * four 8-byte runs; run s holds values 16s + j (low nibble of byte j) and
 * 16s + 8 + j (high nibble), on the doubled E2M1 grid. */
static void deq_nvfp4(const uint8_t *b, float *y) {
    for (int s = 0; s < 4; s++) {
        float d = ue4m3(b[s]);
        const uint8_t *qs = b + 4 + 8 * s;
        for (int j = 0; j < 8; j++) {
            y[16 * s + j] = (float)kFp4[qs[j] & 0xF] * d;
            y[16 * s + j + 8] = (float)kFp4[qs[j] >> 4] * d;
        }
    }
}

/* src/quant.cpp:310-318: the ROCmFP4 code ladder, magnitudes 0, 1, 2, 3, 4,
 * 6, 8, 10 (the top level is 10, not E2M1's 12), bit 3 the sign. */
static int rocmfp4_code(int q) {
    int m = q & 7, mag = m <= 4 ? m : 2 * m - 4;
    return (q & 8) ? -mag : mag;
}

/* src/quant.cpp:692-713: ROCmFP4 (18 B): 16 nibble bytes (value j the low
 * nibble of byte j, j + 16 the high), then the two half scales (UE4M3);
 * ROCmFP4_FAST (17 B): one scale for all 32. */
static void deq_rocmfp4(const uint8_t *b, float *y, int two_scales) {
    float d0 = ue4m3(b[16]), d1 = two_scales ? ue4m3(b[17]) : d0;
    for (int j = 0; j < 16; j++) {
        y[j] = (float)rocmfp4_code(b[j] & 0xF) * d0;
        y[j + 16] = (float)rocmfp4_code(b[j] >> 4) * d1;
    }
}

/* src/quant.cpp:740-857: the ROCmFPX 32-value formats, each with two UE4M3
 * half scales after the codes.  FP2 (10 B): 2-bit codes, four to a byte
 * from the low bits, on the ladder {-4, -1, 1, 4}.  FP3 (14 B): eight 3-bit
 * codes per 3 bytes, LSB first; magnitude {0, 1, 2, 4}[c & 3], sign bit 2.
 * FP6 (26 B): four 6-bit codes per 3 bytes, LSB first; magnitude c & 31,
 * sign bit 5, and a negative zero is -32. */
static void deq_rocmfpx2(const uint8_t *b, float *y) {
    static const int lad[4] = {-4, -1, 1, 4};
    float d0 = ue4m3(b[8]), d1 = ue4m3(b[9]);
    for (int j = 0; j < 32; j++) {
        int c = (b[j / 4] >> (2 * (j % 4))) & 3;
        y[j] = (float)lad[c] * (j < 16 ? d0 : d1);
    }
}
static void deq_rocmfpx3(const uint8_t *b, float *y) {
    static const int mag[4] = {0, 1, 2, 4};
    float d0 = ue4m3(b[12]), d1 = ue4m3(b[13]);
    for (int j = 0; j < 32; j++) {
        const uint8_t *g = b + 3 * (j / 8);
        uint32_t w = (uint32_t)g[0] | ((uint32_t)g[1] << 8) | ((uint32_t)g[2] << 16);
        int c = (int)((w >> (3 * (j % 8))) & 7);
        int v = mag[c & 3];
        y[j] = (float)((c & 4) ? -v : v) * (j < 16 ? d0 : d1);
    }
}
static void deq_rocmfpx6(const uint8_t *b, float *y) {
    float d0 = ue4m3(b[24]), d1 = ue4m3(b[25]);
    for (int j = 0; j < 32; j++) {
        const uint8_t *g = b + 3 * (j / 4);
        uint32_t w = (uint32_t)g[0] | ((uint32_t)g[1] << 8) | ((uint32_t)g[2] << 16);
        int c = (int)((w >> (6 * (j % 4))) & 63), m = c & 31;
        int v = (c & 32) ? -(m == 0 ? 32 : m) : m;
        y[j] = (float)v * (j < 16 ? d0 : d1);
    }
}

/* src/quant.cpp:859-889: TQ1_0 (54 B): base-3 packed trits, five per byte
 * in qs[0..47] and four per byte in qh[48..51], f16 d at 52.  Trit n of a
 * byte q is ((uint8)(q * 3^n) * 3) >> 8, minus 1 (the product wraps to a
 * byte first).  Element v: v < 160 -> byte v % 32, trit v / 32; v < 240 ->
 * byte 32 + (v - 160) % 16, trit (v - 160) / 16; else byte 48 + (v - 240)
 * % 4, trit (v - 240) / 4.  Value d * trit. */
static int tq1_trit(int q, int n) {
    static const int p3[6] = {1, 3, 9, 27, 81, 243};
    uint8_t w = (uint8_t)(q * p3[n]);
    return (int)(((uint16_t)w * 3u) >> 8) - 1;
}
static void deq_tq1_0(const uint8_t *b, float *y) {
    float d = ld_f16(b + 52);
    for (int v = 0; v < 256; v++) {
        int t;
        if (v < 160) t = tq1_trit(b[v % 32], v / 32);
        else if (v < 240) t = tq1_trit(b[32 + (v - 160) % 16], (v - 160) / 16);
        else t = tq1_trit(b[48 + (v - 240) % 4], (v - 240) / 4);
        y[v] = d * (float)t;
    }
}

/* src/quant.cpp:907-918: TQ2_0 (66 B): 2-bit codes q in planes, f16 d at
 * 64; element 128 h + 32 l + m is bits 2l of byte 32 h + m; value d*(q-1). */
static void deq_tq2_0(const uint8_t *b, float *y) {
    float d = ld_f16(b + 64);
    for (int h = 0; h < 2; h++)
        for (int l = 0; l < 4; l++)
            for (int m = 0; m < 32; m++)
                y[128 * h + 32 * l + m] = d * (float)((int)((b[32 * h + m] >> (2 * l)) & 3) - 1);
}

/* src/quant_fmt_a.inc:71-83: Q1_0 (18 B / 128): f16 d, one bit per value
 * (low bit first): +d for a 1, -d for a 0 (no zero). */
static void deq_q1_0(const uint8_t *b, float *y) {
    float d = ld_f16(b);
    for (int j = 0; j < 128; j++) y[j] = ((b[2 + j / 8] >> (j % 8)) & 1) ? d : -d;
}

/* src/quant_fmt_a.inc:85-129: Q2_0 and PQ2_0 (34 B / 128) and Q2_0_64
 * (18 B / 64): f16 d, 2-bit codes four to a byte from the low pair, value
 * (q - 1) * d. */
static void deq_q2_0n(const uint8_t *b, float *y, int n) {
    float d = ld_f16(b);
    for (int j = 0; j < n; j++) y[j] = (float)((int)((b[2 + j / 4] >> (2 * (j % 4))) & 3) - 1) * d;
}

/* src/quant.cpp:933-950: PTQ1_0 (28 B / 128): TQ1_0's trits at group 128,
 * f16 d at 26.  Element v < 80: byte v % 16, trit v / 16; v < 120: byte
 * 16 + (v - 80) % 8, trit (v - 80) / 8; else byte 24 + (v - 120) % 2, trit
 * (v - 120) / 2. */
static void deq_ptq1_0(const uint8_t *b, float *y) {
    float d = ld_f16(b + 26);
    for (int v = 0; v < 128; v++) {
        int t;
        if (v < 80) t = tq1_trit(b[v % 16], v / 16);
        else if (v < 120) t = tq1_trit(b[16 + (v - 80) % 8], (v - 80) / 8);
        else t = tq1_trit(b[24 + (v - 120) % 2], (v - 120) / 2);
        y[v] = d * (float)t;
    }
}

/* src/quant.cpp:1553-1601 (the formats on this path plus F16). */
static void dequant_block(int dt, const uint8_t *p, float *buf) {
    switch (dt) {
        case ORC_F16: buf[0] = ld_f16(p); break;
        case ORC_BF16: { /* src/quant.cpp:1558-1559: the high half of an f32 */
            uint32_t bits = ((uint32_t)p[0] | ((uint32_t)p[1] << 8)) << 16;
            memcpy(buf, &bits, 4);
            break;
        }
        case ORC_F32: memcpy(buf, p, 4); break;
        case ORC_Q4_0: deq_q4_0(p, buf); break;
        case ORC_Q8_0: deq_q8_0(p, buf); break;
        case ORC_MXFP4: deq_mxfp4(p, buf); break;
        case ORC_Q4_1: deq_l32(p, buf, 1, -1, 4, 0); break;
        case ORC_Q5_0: deq_l32(p, buf, 0, 2, 6, 16); break;
        case ORC_Q5_1: deq_l32(p, buf, 1, 4, 8, 0); break;
        case ORC_IQ4_NL: deq_iq4_nl(p, buf); break;
        case ORC_IQ4_XS: deq_iq4_xs(p, buf); break;
        case ORC_Q2_K: deq_q2_k(p, buf); break;
        case ORC_Q3_K: deq_q3_k(p, buf); break;
        case ORC_Q4_K: deq_q4_k(p, buf); break;
        case ORC_Q5_K: deq_q5_k(p, buf); break;
        case ORC_Q6_K: deq_q6_k(p, buf); break;
        case ORC_Q8_1: deq_q8_1(p, buf); break;
        case ORC_Q8_K: deq_q8_k(p, buf); break;
        case ORC_NVFP4: deq_nvfp4(p, buf); break;
        case ORC_ROCMFP4: deq_rocmfp4(p, buf, 1); break;
        case ORC_ROCMFP4_FAST: deq_rocmfp4(p, buf, 0); break;
        case ORC_Q2_0_ROCMFPX: deq_rocmfpx2(p, buf); break;
        case ORC_Q3_0_ROCMFPX: deq_rocmfpx3(p, buf); break;
        case ORC_Q6_0_ROCMFPX: deq_rocmfpx6(p, buf); break;
        case ORC_TQ1_0: deq_tq1_0(p, buf); break;
        case ORC_TQ2_0: deq_tq2_0(p, buf); break;
        case ORC_Q1_0: deq_q1_0(p, buf); break;
        case ORC_Q2_0: case ORC_PQ2_0: deq_q2_0n(p, buf, 128); break;
        case ORC_Q2_0_64: deq_q2_0n(p, buf, 64); break;
        case ORC_PTQ1_0: deq_ptq1_0(p, buf); break;
        default: break;
    }
}

/* src/quant.cpp:1911-1960 (block formats branch). */
void orc_dequant_row(int dt, const void *src, float *out, int64_t n) {
    const uint8_t *p = (const uint8_t *)src;
    int bs = orc_block_size(dt), bb = orc_block_bytes(dt);
    float buf[256];
    for (int64_t i = 0; i < n;) {
        int cnt = (int)((n - i) < bs ? (n - i) : bs);
        dequant_block(dt, p, buf);
        memcpy(out + i, buf, (size_t)cnt * sizeof(float));
        i += cnt;
        p += bb;
    }
}

/* src/quant.cpp:1962-1979 */
void orc_dequant_row_f16(int dt, const void *src, uint16_t *out, int64_t n) {
    float *tmp = (float *)malloc((size_t)n * sizeof(float));
    orc_dequant_row(dt, src, tmp, n);
    for (int64_t i = 0; i < n; i++) out[i] = orc_fp32_to_fp16(tmp[i]);
    free(tmp);
}

/* src/quant.cpp:5576-5591: the strict scalar branch of vec_dot (fast, avx2
 * and int8 tiers off): ONE f32 chain over the dequantized blocks.
 * `sum += buf[k] * x[i + k]` is NOT contracted in the reference build: the
 * product is rounded, then added.  Measured, not assumed: against
 * oracle/_ref/libkrk_ref.so (the reference's quant.cpp built with its own
 * flags) the unfused chain matches bit for bit and the fused one does not. */
/* src/quant.cpp:5431-5510: the unquantized types are not block-dotted but
 * summed in four lanes (lane k takes elements i = k mod 4, each step a fused
 * multiply-add: _mm_fmadd_ps for F32 / F16, the 4-accumulator loop contracted
 * by the reference build for BF16), combined as (a0 + a1) + (a2 + a3), then a
 * scalar tail. */
static float float_dot(int dt, const uint8_t *p, const float *x, int64_t n) {
    float a[4] = {0, 0, 0, 0}, w[4];
    int64_t i = 0;
    for (; i + 4 <= n; i += 4)
        for (int k = 0; k < 4; k++) {
            dequant_block(dt, p + (i + k) * orc_block_bytes(dt), &w[k]);
            a[k] = fmaf(w[k], x[i + k], a[k]);
        }
    float s = (a[0] + a[1]) + (a[2] + a[3]);
    for (; i < n; i++) {
        dequant_block(dt, p + i * orc_block_bytes(dt), &w[0]);
        s = fmaf(w[0], x[i], s);
    }
    return s;
}

float orc_vec_dot(int dt, const void *src, const float *x, int64_t n) {
    if (dt == ORC_F32 || dt == ORC_F16 || dt == ORC_BF16) return float_dot(dt, (const uint8_t *)src, x, n);
    int bs = orc_block_size(dt), bb = orc_block_bytes(dt);
    const uint8_t *p = (const uint8_t *)src;
    float buf[256], sum = 0.0f;
    for (int64_t i = 0; i < n;) {
        int cnt = (int)((n - i) < bs ? (n - i) : bs);
        dequant_block(dt, p, buf);
        for (int k = 0; k < cnt; k++) sum += buf[k] * x[i + k];
        i += cnt;
        p += bb;
    }
    return sum;
}

/* ---- a fixed-size pool over independent outputs (src/backend_cpu.cpp:1-8:
 * parallel over outputs only, never a split reduction, so the answer does not
 * depend on the thread count). */
typedef struct {
    void (*fn)(void *ctx, int64_t b, int64_t e);
    void *ctx;
    int64_t b, e;
} orc_job;

static void *orc_job_run(void *a) {
    orc_job *j = (orc_job *)a;
    j->fn(j->ctx, j->b, j->e);
    return NULL;
}

static void par_for(int64_t n, int nthreads,
                    void (*fn)(void *ctx, int64_t b, int64_t e), void *ctx) {
    if (nthreads <= 1 || n < 2) { fn(ctx, 0, n); return; }
    if (nthreads > 256) nthreads = 256;
    if (nthreads > n) nthreads = (int)n;
    pthread_t th[256];
    orc_job jobs[256];
    int64_t per = (n + nthreads - 1) / nthreads;
    int started = 0;
    for (int t = 0; t < nthreads; t++) {
        int64_t b = per * t, e = b + per < n ? b + per : n;
        if (b >= e) break;
        jobs[t].fn = fn; jobs[t].ctx = ctx; jobs[t].b = b; jobs[t].e = e;
        if (pthread_create(&th[t], NULL, orc_job_run, &jobs[t]) != 0) {
            fn(ctx, b, e);
            jobs[t].fn = NULL;
        }
        started = t + 1;
    }
    for (int t = 0; t < started; t++)
        if (jobs[t].fn) pthread_join(th[t], NULL);
}

typedef struct {
    float *out; const float *x; const uint8_t *w; int dt;
    int64_t n_out, n_in, rows, rb;
} gemm_ctx;

static void gemm_body(void *c, int64_t b, int64_t e) {
    gemm_ctx *g = (gemm_ctx *)c;
    for (int64_t o = b; o < e; o++)
        for (int64_t r = 0; r < g->rows; r++)
            g->out[r * g->n_out + o] =
                orc_vec_dot(g->dt, g->w + o * g->rb, g->x + r * g->n_in, g->n_in);
}

/* src/backend_cpu.cpp:914-1320 with the int8/fast/avx2 tiers off: every
 * output element is vec_dot(row o, x row r) (src/quant.cpp:5420-5428). */
void orc_gemm(float *out, const float *x, const void *w, int dt,
              int64_t n_out, int64_t n_in, int64_t rows, int nthreads) {
    gemm_ctx g = {out, x, (const uint8_t *)w, dt, n_out, n_in, rows,
                  orc_row_bytes(dt, n_in)};
    par_for(n_out, nthreads, gemm_body, &g);
}

/* src/quant.cpp:2167-2197 (quantize_q8_32_d): per 32 values amax, d =
 * amax/127 (0 for an all-zero block), codes cvtps(x * (1/d)) -- round to
 * nearest even under the default MXCSR -- clamped to [-127, 127].  A NaN
 * product converts to INT_MIN there and clamps to -127. */
void orc_quantize_q8_row(const float *x, int64_t n, int8_t *xq, float *dx) {
    for (int64_t b = 0; b < n; b += 32) {
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            float a = fabsf(x[b + i]);
            amax = a > amax ? a : amax;
        }
        float d = amax > 0.0f ? amax / 127.0f : 0.0f;
        dx[b / 32] = d;
        if (d == 0.0f) { memset(xq + b, 0, 32); continue; }
        float inv = 1.0f / d;
        for (int i = 0; i < 32; i++) {
            float p = x[b + i] * inv;
            long q = isnan(p) ? -2147483647L - 1 : lrintf(p);
            if (q < -127) q = -127;
            if (q > 127) q = 127;
            xq[b + i] = (int8_t)q;
        }
    }
}

/* src/quant.cpp:3261-3279 (dot_q8_0_q8_scalar): exact integer block sum, then
 * acc = fma((f32)sum, d * dx[b], acc). */
float orc_dot_q8_0_q8(const void *w, const int8_t *xq, const float *dx,
                      int64_t n) {
    const uint8_t *p = (const uint8_t *)w;
    float acc = 0.0f;
    for (int64_t b = 0; b < n / 32; b++, p += 34) {
        float d = ld_f16(p);
        int64_t sum = 0;
        for (int i = 0; i < 32; i++)
            sum += (int64_t)(int8_t)p[2 + i] * (int64_t)xq[b * 32 + i];
        acc = fmaf((float)sum, d * dx[b], acc);
    }
    return acc;
}

/* The GPU int8 rung's fold for the affine K-quants (gemm_dp4a.hpp:379-570,
 * weight staging 197-375): per 32-value block b of the activation row, with
 * sa = dx[b], the integer dot I and code sum S (exact) of each half, and the
 * weight half's scale bsc and min bmin:
 *     acc = fma(sa * bsc, (f32) I, acc);  acc = fma(-(sa * S), bmin, acc)
 * Q4_K / Q5_K: one half of 32 values; bsc = d*s, bmin = dmin*m of the
 * sub-block (get_scale_min_k4), S the sum over the 32 codes (the sum of its
 * two 16-value halves, exact).  Codes are the unsigned Q4_K/Q5_K nibbles
 * (0..15 / 0..31).  Q6_K: two halves of 16 values with bsc = d*sc of the
 * 16-value group; the offset 32 is taken in the integer dot as the CPU
 * twin does (t = I - 32*S in int32, dot_q6_K_q8_d, quant.cpp:2755-2800):
 *     acc = fma(sa * bsc, (f32)(I - 32*S), acc)
 * which equals the GPU rung's two-term fold up to its one extra rounding. */
static void kq_half(int dt, const uint8_t *blk, int b32, int h, int *codes, float *bsc, float *bmin) {
    /* codes of values 32*b32 + 16*h .. +16 of the 256-value block */
    int base = 32 * b32 + 16 * h;
    if (dt == ORC_Q4_K || dt == ORC_Q5_K) {
        float d = ld_f16(blk), dmin = ld_f16(blk + 2);
        uint8_t si, mi;
        scale_min_k4(b32, blk + 4, &si, &mi);
        *bsc = d * (float)si;
        *bmin = dmin * (float)mi;
        const uint8_t *q = blk + (dt == ORC_Q4_K ? 16 : 48) + 32 * (b32 / 2);
        for (int l = 0; l < 16; l++) {
            int li = 16 * h + l;
            int c = (b32 & 1) ? (q[li] >> 4) : (q[li] & 0xF);
            if (dt == ORC_Q5_K) c |= ((blk[16 + li] >> b32) & 1) << 4;
            codes[l] = c;
        }
    } else { /* Q6_K: value v = 128n + 32qd + l */
        float d = ld_f16(blk + 208);
        for (int l = 0; l < 16; l++) {
            int v = base + l, n = v / 128, qd = (v % 128) / 32, ll = v % 32;
            const uint8_t *ql = blk + 64 * n, *qh = blk + 128 + 32 * n;
            int lo = (qd & 1) ? ql[ll + 32] : ql[ll];
            lo = (qd >> 1) ? (lo >> 4) : (lo & 0xF);
            codes[l] = lo | (((qh[ll] >> (2 * qd)) & 3) << 4);
        }
        int g = (base % 128) / 16 + 8 * (base / 128);
        *bsc = d * (float)(int8_t)blk[192 + g];
        *bmin = 32.0f * *bsc;
    }
}

float orc_dot_kq_q8(int dt, const void *w, const int8_t *xq, const float *dx, int64_t n) {
    const uint8_t *p = (const uint8_t *)w;
    int bb = orc_block_bytes(dt);
    float acc = 0.0f;
    for (int64_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = p + (b / 8) * bb;
        int b32 = (int)(b % 8);
        const int8_t *x = xq + 32 * b;
        float sa = dx[b];
        if (dt == ORC_Q6_K) {
            for (int h = 0; h < 2; h++) {
                int codes[16], I = 0, S = 0;
                float bsc, bmin;
                kq_half(dt, blk, b32, h, codes, &bsc, &bmin);
                for (int l = 0; l < 16; l++) { I += codes[l] * x[16 * h + l]; S += x[16 * h + l]; }
                (void)bmin;
                acc = fmaf(sa * bsc, (float)(I - 32 * S), acc);
            }
        } else {
            int I = 0, S0 = 0, S1 = 0;
            float bsc = 0, bmin = 0;
            for (int h = 0; h < 2; h++) {
                int codes[16];
                kq_half(dt, blk, b32, h, codes, &bsc, &bmin);
                for (int l = 0; l < 16; l++) {
                    I += codes[l] * x[16 * h + l];
                    if (h) S1 += x[16 * h + l]; else S0 += x[16 * h + l];
                }
            }
            acc = fmaf(sa * bsc, (float)I, acc);
            acc = fmaf(-(sa * ((float)S0 + (float)S1)), bmin, acc);
        }
    }
    return acc;
}

typedef struct {
    float *out; const int8_t *xq; const float *dx; const uint8_t *w;
    int64_t n_out, n_in, rows, rb;
    int dt;
} gq_ctx;

static void gq_body(void *c, int64_t b, int64_t e) {
    gq_ctx *g = (gq_ctx *)c;
    for (int64_t o = b; o < e; o++)
        for (int64_t r = 0; r < g->rows; r++)
            g->out[r * g->n_out + o] = g->dt == ORC_Q8_0
                ? orc_dot_q8_0_q8(g->w + o * g->rb, g->xq + r * g->n_in, g->dx + r * (g->n_in / 32), g->n_in)
                : orc_dot_kq_q8(g->dt, g->w + o * g->rb, g->xq + r * g->n_in,
                                g->dx + r * (g->n_in / 32), g->n_in);
}

/* The CPU backend's Q8_0 x int8 rung (src/backend_cpu.cpp:952-1000): each
 * activation row quantized once, then the scalar integer dot per output. */
void orc_gemm_int8(int dt, float *out, const float *x, const void *w,
                   int64_t n_out, int64_t n_in, int64_t rows, int nthreads) {
    int8_t *xq = (int8_t *)malloc((size_t)(rows * n_in));
    float *dx = (float *)malloc((size_t)(rows * (n_in / 32)) * sizeof(float));
    for (int64_t r = 0; r < rows; r++)
        orc_quantize_q8_row(x + r * n_in, n_in, xq + r * n_in, dx + r * (n_in / 32));
    gq_ctx g = {out, xq, dx, (const uint8_t *)w, n_out, n_in, rows,
                orc_row_bytes(dt, n_in), dt};
    par_for(n_out, nthreads, gq_body, &g);
    free(xq);
    free(dx);
}

void orc_gemm_q8_0_q8(float *out, const float *x, const void *w,
                      int64_t n_out, int64_t n_in, int64_t rows, int nthreads) {
    orc_gemm_int8(ORC_Q8_0, out, x, w, n_out, n_in, rows, nthreads);
}

/* src/backend_cpu.cpp:2401-2406: o = (g / (1 + exp(-g))) * u, std::exp on a
 * float argument (expf). */
void orc_silu_mul(float *out, const float *g, const float *u, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float x = g[i];
        out[i] = (x / (1.0f + expf(-x))) * u[i];
    }
}

/* src/engine.cpp:11704-11714 (softmax branch): running max, sequential sum of
 * exp(l - max), multiply by 1/sum. */
void orc_router_softmax(float *probs, const float *logits, int64_t n_rows,
                        int ne) {
    for (int64_t r = 0; r < n_rows; r++) {
        const float *l = logits + r * ne;
        float *p = probs + r * ne;
        float mx = l[0];
        for (int e = 1; e < ne; e++) mx = l[e] > mx ? l[e] : mx;
        float sum = 0.0f;
        for (int e = 0; e < ne; e++) {
            p[e] = expf(l[e] - mx);
            sum += p[e];
        }
        float inv = sum > 0 ? 1.0f / sum : 0.0f;
        for (int e = 0; e < ne; e++) p[e] *= inv;
    }
}

/* src/engine.cpp:11853-11918 with no residency preference and no bias: k
 * rounds of argmax over the not-yet-taken experts (strict >, ascending id, so
 * a tie keeps the lower id); the weight is the probability; then
 * sum-normalize when asked (wt *= 1/sum) and multiply by scale unless it is
 * 0 or 1. */
void orc_router_topk(const float *probs, int64_t n_rows, int ne, int k,
                     int32_t *ids, float *wts, int normalize, float scale) {
    for (int64_t r = 0; r < n_rows; r++) {
        const float *p = probs + r * ne;
        int32_t *sel = ids + r * k;
        float *wt = wts + r * k;
        for (int s = 0; s < k; s++) {
            int best = -1;
            float bestp = -1.0f;
            for (int e = 0; e < ne; e++) {
                int taken = 0;
                for (int q = 0; q < s; q++)
                    if (sel[q] == e) { taken = 1; break; }
                if (taken) continue;
                if (p[e] > bestp) { bestp = p[e]; best = e; }
            }
            sel[s] = best;
            wt[s] = best >= 0 ? p[best] : 0.0f;
        }
        if (normalize) {
            float ksum = 0;
            for (int s = 0; s < k; s++) ksum += wt[s];
            float kinv = ksum > 0 ? 1.0f / ksum : 0.0f;
            for (int s = 0; s < k; s++) wt[s] *= kinv;
        }
        if (scale != 0.0f && scale != 1.0f)
            for (int s = 0; s < k; s++) wt[s] *= scale;
    }
}

/* The host MoE loop (src/engine.cpp:12360-12700): for each expert in
 * ascending id, gather the rows that selected it (token-then-slot order),
 * gate and up gemm, silu_mul (src/backend_cpu.cpp:2369-2410), down gemm, then
 * scatter_axpy_rows (src/backend_cpu.cpp:3193-3217): dst += a * src, which the
 * reference build contracts to one FMA per element (a plain add when a==1,
 * the same value).  The destination starts at zero. */
void orc_moe_ffn(float *out, const float *x, const void *const *gate,
                 const void *const *up, const void *const *down, int wt_gate,
                 int wt_up, int wt_down, const int32_t *ids, const float *wts,
                 int64_t n_tok, int64_t n_embd, int64_t n_ff, int n_expert,
                 int k, int nthreads) {
    memset(out, 0, (size_t)(n_tok * n_embd) * sizeof(float));
    int64_t cap = n_tok * k;
    int32_t *rows = (int32_t *)malloc((size_t)cap * sizeof(int32_t));
    float *alpha = (float *)malloc((size_t)cap * sizeof(float));
    float *xg = (float *)malloc((size_t)(cap * n_embd) * sizeof(float));
    float *g = (float *)malloc((size_t)(cap * n_ff) * sizeof(float));
    float *u = (float *)malloc((size_t)(cap * n_ff) * sizeof(float));
    float *mid = (float *)malloc((size_t)(cap * n_ff) * sizeof(float));
    float *dn = (float *)malloc((size_t)(cap * n_embd) * sizeof(float));
    for (int e = 0; e < n_expert; e++) {
        int64_t m = 0;
        for (int64_t t = 0; t < n_tok; t++)
            for (int s = 0; s < k; s++)
                if (ids[t * k + s] == e) {
                    rows[m] = (int32_t)t;
                    alpha[m] = wts[t * k + s];
                    m++;
                }
        if (m == 0) continue;
        for (int64_t i = 0; i < m; i++)
            memcpy(xg + i * n_embd, x + (int64_t)rows[i] * n_embd,
                   (size_t)n_embd * sizeof(float));
        orc_gemm(g, xg, gate[e], wt_gate, n_ff, n_embd, m, nthreads);
        orc_gemm(u, xg, up[e], wt_up, n_ff, n_embd, m, nthreads);
        orc_silu_mul(mid, g, u, m * n_ff);
        orc_gemm(dn, mid, down[e], wt_down, n_embd, n_ff, m, nthreads);
        for (int64_t i = 0; i < m; i++) {
            float *dr = out + (int64_t)rows[i] * n_embd;
            const float *sr = dn + i * n_embd;
            float a = alpha[i];
            for (int64_t j = 0; j < n_embd; j++) dr[j] = fmaf(a, sr[j], dr[j]);
        }
    }
    free(rows); free(alpha); free(xg); free(g); free(u); free(mid); free(dn);
}

/* The reference GPU backend's f16 expert FFN (act_type F16), restated from
 * src/hip/kernels/moe_table.hpp: gate/up tiles (230-254), the row scale
 * (256-305), the down partial (418-441) and the slot-order reduce (536-551);
 * dispatched by backend_hip.hip:2525-2659.  Per token t and slot s in slot
 * order, expert e = ids[t k + s] (a dropped slot adds nothing):
 *   mid_j  = silu(f16(gate_e . x_t)_j) * f16(up_e . x_t)_j        (f32)
 *   scale  = the smallest power of two >= 1 (at most 2^24) with
 *            max_j |mid_j| <= 65504 * scale
 *   midf_j = f16(mid_j * (1 / scale))
 *   part_i = wts[t, s] * (f16(down_e . midf)_i * scale)          (two RN products)
 *   a_i    = f16(a_i + part_i)                                    (a starts at 0)
 * out is f16.  x holds f16 values (as f32); the row dots are the strict f32
 * chain of vec_dot, silu is x / (1 + exp(-x)) in f32.  Output: f16 bits. */
static float f16r(float v) { return orc_fp16_to_fp32(orc_fp32_to_fp16(v)); }

void orc_moe_ffn_f16(uint16_t *out, const float *x, const void *const *gate,
                     const void *const *up, const void *const *down, int wt_gate,
                     int wt_up, int wt_down, const int32_t *ids, const float *wts,
                     int64_t n_tok, int64_t n_embd, int64_t n_ff, int n_expert,
                     int k, int nthreads) {
    float *g = (float *)malloc((size_t)n_ff * sizeof(float));
    float *u = (float *)malloc((size_t)n_ff * sizeof(float));
    float *mid = (float *)malloc((size_t)n_ff * sizeof(float));
    float *v = (float *)malloc((size_t)n_embd * sizeof(float));
    float *a = (float *)malloc((size_t)n_embd * sizeof(float));
    for (int64_t t = 0; t < n_tok; t++) {
        const float *xt = x + t * n_embd;
        for (int64_t j = 0; j < n_embd; j++) a[j] = 0.0f;
        for (int s = 0; s < k; s++) {
            const int e = ids[t * k + s];
            if (e < 0 || e >= n_expert) continue;
            orc_gemm(g, xt, gate[e], wt_gate, n_ff, n_embd, 1, nthreads);
            orc_gemm(u, xt, up[e], wt_up, n_ff, n_embd, 1, nthreads);
            float mx = 0.0f;
            for (int64_t j = 0; j < n_ff; j++) {
                const float gf = f16r(g[j]), uf = f16r(u[j]);
                mid[j] = (gf / (1.0f + expf(-gf))) * uf;
                const float m = fabsf(mid[j]);
                if (m > mx) mx = m;
            }
            float mul = 1.0f;
            while (mx > 65504.0f * mul && mul < 16777216.0f) mul *= 2.0f;
            const float inv = 1.0f / mul;
            for (int64_t j = 0; j < n_ff; j++) mid[j] = f16r(mid[j] * inv);
            orc_gemm(v, mid, down[e], wt_down, n_embd, n_ff, 1, nthreads);
            const float w = wts[t * k + s];
            for (int64_t j = 0; j < n_embd; j++) {
                const float vs = f16r(v[j]) * mul;
                a[j] = f16r(a[j] + w * vs);
            }
        }
        for (int64_t j = 0; j < n_embd; j++) out[t * n_embd + j] = orc_fp32_to_fp16(a[j]);
    }
    free(g); free(u); free(mid); free(v); free(a);
}

/* ---- tools/make_bench_gguf.py:191-202 (quantize_q8_0), the repo's own q8_0
 * fixture generator.  Python floats are f64: amax = max|v| (1e-8 for an all-
 * zero block), d = amax / 127.0, q = clamp(round_half_even(v / d), +-127),
 * scale stored with struct.pack('<e', d) -- f64 rounded once to f16, RNE. */
static uint16_t f64_to_f16_rne(double v) {
    /* Exact for every finite double: scale into the f16 grid with ldexp and
     * let nearbyint (round-half-even) pick the neighbour. */
    uint16_t sign = signbit(v) ? 0x8000u : 0;
    double a = fabs(v);
    if (isnan(v)) return 0x7E00u;
    if (a >= 65520.0) return (uint16_t)(sign | 0x7C00u);
    int e;
    frexp(a, &e);           /* a = f * 2^e, f in [0.5, 1) */
    int ue = e - 1;         /* unbiased exponent */
    if (ue < -14) ue = -14; /* subnormal grid */
    double q = nearbyint(ldexp(a, 10 - ue));   /* units of 2^(ue-10) */
    if (q >= 2048.0) { q /= 2; ue++; }
    if (ue > 15) return (uint16_t)(sign | 0x7C00u);
    uint32_t qi = (uint32_t)q;
    if (qi < 1024) return (uint16_t)(sign | qi);          /* subnormal */
    return (uint16_t)(sign | ((uint32_t)(ue + 15) << 10) | (qi - 1024));
}

void orc_quantize_q8_0_weights(const float *v, int64_t n, uint8_t *dst) {
    for (int64_t b = 0; b < n; b += 32, dst += 34) {
        double amax = 0.0;
        for (int i = 0; i < 32; i++) {
            double a = fabs((double)v[b + i]);
            amax = a > amax ? a : amax;
        }
        if (amax == 0.0) amax = 1e-8;
        double d = amax / 127.0;
        uint16_t h = f64_to_f16_rne(d);
        dst[0] = (uint8_t)(h & 0xFF);
        dst[1] = (uint8_t)(h >> 8);
        for (int i = 0; i < 32; i++) {
            double q = nearbyint((double)v[b + i] / d);
            if (q < -127) q = -127;
            if (q > 127) q = 127;
            dst[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}
