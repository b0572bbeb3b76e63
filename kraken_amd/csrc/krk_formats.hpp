// krk_formats.hpp -- device decoders for the four GGUF block formats on this
// path, in two shapes:
//
//  * dequant_chunk<DT>(block, c, out[32]): the reference's 32-value chunk
//    contract (src/hip/kernels/dequant.hpp:423-427): chunk c of a block is
//    its 32 consecutive values, decoded with exactly the host oracle's
//    arithmetic (src/quant.cpp:331-512) so the f32 result is bit-identical.
//
//  * LaneFmt<DT>: the wave64 GEMV/GEMM view.  A lane owns a 32-value "piece"
//    of a block; the piece's bytes arrive through dword loads, are widened
//    byte-parallel, and the piece's dot product with x is formed as
//        sum_g  scale_g * (sum_{i in g} wq_i * x_i)  -  off_g * (sum_{i in g} x_i)
//    with wq the raw code (times a power of two), so the activation sums
//    sum x_i -- fixed across weight rows -- are computed once per lane.
#pragma once

#include "krk_dev.hpp"

namespace krk {

// ---------------------------------------------------------------- geometry --
// F16 and BF16 weights are handled as 32-value pseudo-blocks of 64 bytes (a
// row of n values is n / 32 of them), so they ride the same chunk contract.
// Formats served through the generic chunk path: every kernel reads them
// through dequant_chunk alone (byte loads, any alignment).  X(type) for each,
// for the launchers' switches.
#define KRK_CHUNK_FORMATS(X)                                                                       \
    X(DT_Q8_1) X(DT_Q8_K) X(DT_TQ1_0) X(DT_TQ2_0) X(DT_NVFP4) X(DT_ROCMFP4) X(DT_ROCMFP4_FAST)      \
    X(DT_Q6_0_ROCMFPX) X(DT_Q3_0_ROCMFPX) X(DT_Q2_0_ROCMFPX) X(DT_Q1_0) X(DT_Q2_0) X(DT_Q2_0_64)   \
    X(DT_PQ2_0) X(DT_PTQ1_0)
__host__ __device__ constexpr bool chunk_fmt(int dt) {
#define KRK_CHUNK_IS(D) dt == D ||
    return KRK_CHUNK_FORMATS(KRK_CHUNK_IS) false;
#undef KRK_CHUNK_IS
}
__host__ __device__ constexpr int blk_vals(int dt) {
    return dt == DT_Q4_K || dt == DT_Q5_K || dt == DT_Q6_K || dt == DT_IQ4_XS || dt == DT_Q2_K ||
                   dt == DT_Q3_K || dt == DT_Q8_K || dt == DT_TQ1_0 || dt == DT_TQ2_0
               ? 256
           : dt == DT_NVFP4 || dt == DT_Q2_0_64 ? 64
           : dt == DT_Q1_0 || dt == DT_Q2_0 || dt == DT_PQ2_0 || dt == DT_PTQ1_0 ? 128
           : (dt == DT_Q4_0 || dt == DT_Q8_0 || dt == DT_IQ4_NL || dt == DT_MXFP4 || dt == DT_Q4_1 ||
              dt == DT_Q5_0 || dt == DT_Q5_1 || dt == DT_F16 || dt == DT_BF16 || dt == DT_Q8_1 ||
              dt == DT_ROCMFP4 || dt == DT_ROCMFP4_FAST || dt == DT_Q6_0_ROCMFPX || dt == DT_Q3_0_ROCMFPX ||
              dt == DT_Q2_0_ROCMFPX)
               ? 32
                                                                  : 1;
}
__host__ __device__ constexpr int blk_bytes(int dt) {
    return dt == DT_Q4_K ? 144 : dt == DT_Q5_K ? 176 : dt == DT_Q6_K ? 210 : dt == DT_IQ4_XS ? 136
         : dt == DT_Q2_K ? 84 : dt == DT_Q3_K ? 110 : dt == DT_MXFP4 ? 17 : dt == DT_Q4_1 ? 20
         : dt == DT_Q5_0 ? 22 : dt == DT_Q5_1 ? 24
         : dt == DT_Q4_0 || dt == DT_IQ4_NL ? 18
         : dt == DT_Q8_0 ? 34 : dt == DT_F16 || dt == DT_BF16 ? 64
         : dt == DT_Q8_1 ? 36 : dt == DT_Q8_K ? 292 : dt == DT_TQ1_0 ? 54 : dt == DT_TQ2_0 ? 66
         : dt == DT_NVFP4 ? 36 : dt == DT_ROCMFP4 ? 18 : dt == DT_ROCMFP4_FAST ? 17
         : dt == DT_Q6_0_ROCMFPX ? 26 : dt == DT_Q3_0_ROCMFPX ? 14 : dt == DT_Q2_0_ROCMFPX ? 10
         : dt == DT_Q1_0 || dt == DT_Q2_0_64 ? 18 : dt == DT_Q2_0 || dt == DT_PQ2_0 ? 34 : dt == DT_PTQ1_0 ? 28
         : 4;
}

__device__ __forceinline__ float ldh(const uint8_t *p) {
    return h2f(static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8));
}

// ------------------------------------------------------- chunk contract ----
// Decode chunk c (32 values) of one block into f32, bit-identical to the host
// decoders.  Byte loads: this is the exactness surface, not the fast path.
template <int DT>
__device__ __forceinline__ void dequant_chunk(const uint8_t *b, int c, float *y);

// src/quant.cpp:331-339
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q4_0>(const uint8_t *b, int, float *y) {
    const float d = ldh(b);
    for (int k = 0; k < 16; k++) {
        y[k] = d * static_cast<float>(static_cast<int>(b[2 + k] & 0xF) - 8);
        y[k + 16] = d * static_cast<float>(static_cast<int>(b[2 + k] >> 4) - 8);
    }
}

// IQ4_NL's grid (ggml's kvalues_iq4nl, src/quant.cpp:88-91), a format constant
__device__ __constant__ const int8_t kIq4nlGrid[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                                       1,    13,   25,  38,  53,  69,  89,  113};

// src/quant.cpp:566-574: value d * grid[q], one product
template <>
__device__ __forceinline__ void dequant_chunk<DT_IQ4_NL>(const uint8_t *b, int, float *y) {
    const float d = ldh(b);
    for (int k = 0; k < 16; k++) {
        y[k] = d * static_cast<float>(kIq4nlGrid[b[2 + k] & 0xF]);
        y[k + 16] = d * static_cast<float>(kIq4nlGrid[b[2 + k] >> 4]);
    }
}

// src/quant.cpp:641-659: chunk c = sub-block c, value (d * (ls - 32)) * grid[q]
template <>
__device__ __forceinline__ void dequant_chunk<DT_IQ4_XS>(const uint8_t *b, int c, float *y) {
    const float d = ldh(b);
    const uint32_t sh = static_cast<uint32_t>(b[2]) | (static_cast<uint32_t>(b[3]) << 8);
    const int ls = ((b[4 + c / 2] >> (4 * (c % 2))) & 0xF) | (((sh >> (2 * c)) & 3) << 4);
    const float dl = d * static_cast<float>(ls - 32);
    const uint8_t *qs = b + 8 + 16 * c;
    for (int j = 0; j < 16; j++) {
        y[j] = dl * static_cast<float>(kIq4nlGrid[qs[j] & 0xF]);
        y[j + 16] = dl * static_cast<float>(kIq4nlGrid[qs[j] >> 4]);
    }
}

// src/quant.cpp:381-387
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q8_0>(const uint8_t *b, int, float *y) {
    const float d = ldh(b);
    for (int k = 0; k < 32; k++) y[k] = d * static_cast<float>(static_cast<int8_t>(b[2 + k]));
}

// src/quant.cpp:427-435
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *q, int &d, int &m) {
    if (j < 4) {
        d = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// src/quant.cpp:437-460: chunk c is sub-block c, 32 values; the host build
// contracts d1*q - m1 into one FMA.
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q4_K>(const uint8_t *b, int c, float *y) {
    const float d = ldh(b), dmin = ldh(b + 2);
    int si, mi;
    scale_min_k4(c, b + 4, si, mi);
    const float d1 = d * static_cast<float>(si), m1 = dmin * static_cast<float>(mi);
    const uint8_t *q = b + 16 + 32 * (c >> 1);
    const int sh = (c & 1) * 4;
    for (int l = 0; l < 32; l++)
        y[l] = __builtin_fmaf(d1, static_cast<float>((q[l] >> sh) & 0xF), -m1);
}

// src/quant.cpp:462-489: Q4_K's layout with 32 high-bit bytes at 16 and the
// codes at 48; chunk c takes bit c of qh[l] as bit 4 of its code.  d1*q is
// exact (17 + 5 significant bits), so the FMA matches either host form.
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q5_K>(const uint8_t *b, int c, float *y) {
    const float d = ldh(b), dmin = ldh(b + 2);
    int si, mi;
    scale_min_k4(c, b + 4, si, mi);
    const float d1 = d * static_cast<float>(si), m1 = dmin * static_cast<float>(mi);
    const uint8_t *qh = b + 16, *q = b + 48 + 32 * (c >> 1);
    const int sh = (c & 1) * 4;
    for (int l = 0; l < 32; l++) {
        const int code = ((q[l] >> sh) & 0xF) | (((qh[l] >> c) & 1) << 4);
        y[l] = __builtin_fmaf(d1, static_cast<float>(code), -m1);
    }
}

// src/quant.cpp:491-512: chunk c = quadrant (c & 3) of half (c >> 2).
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q6_K>(const uint8_t *b, int c, float *y) {
    const float d = ldh(b + 208);
    const int h = c >> 2, qd = c & 3;
    const uint8_t *ql = b + 64 * h + 32 * (qd & 1);
    const uint8_t *qh = b + 128 + 32 * h;
    const int8_t *sc = reinterpret_cast<const int8_t *>(b + 192) + 8 * h + 2 * qd;
    const int nsh = (qd >> 1) * 4, hsh = 2 * qd;
    for (int l = 0; l < 32; l++) {
        const int q = ((ql[l] >> nsh) & 0xF) | (((qh[l] >> hsh) & 3) << 4);
        // (d * sc) * (q - 32), left to right as the host writes it
        const float ds = d * static_cast<float>(sc[l / 16]);
        y[l] = ds * static_cast<float>(q - 32);
    }
}

// Q2_K and Q3_K share Q6_K's four planes: chunk c = 4h + j holds values
// 128h + 32j + l whose code is bit pair j of byte 32h + l of the 64 code
// bytes, with scale 8h + 2j + l / 16.
// src/quant.cpp:398-423: value (d * (sc & 15)) * q - dmin * (sc >> 4); both
// products are exact, so the FMA rounds as the host's multiply-subtract does.
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q2_K>(const uint8_t *b, int c, float *y) {
    const float d = ldh(b + 80), dmin = ldh(b + 82);
    const int h = c >> 2, j = c & 3;
    const uint8_t *q = b + 16 + 32 * h;
    for (int l = 0; l < 32; l++) {
        const int sc = b[8 * h + 2 * j + l / 16];
        y[l] = __builtin_fmaf(d * static_cast<float>(sc & 0xF), static_cast<float>((q[l] >> (2 * j)) & 3),
                              -(dmin * static_cast<float>(sc >> 4)));
    }
}

// Q3_K 6-bit scale i from the 12 packed bytes r (quant.cpp:520-528)
__device__ __forceinline__ int q3k_scale(const uint8_t *r, int i) {
    return ((r[i & 7] >> (4 * (i >> 3))) & 0xF) | (((r[8 + (i & 3)] >> (2 * (i >> 2))) & 3) << 4);
}

// src/quant.cpp:514-554: code (q >> 2j & 3) - (hmask[l] bit 4h + j ? 0 : 4),
// value (d * (sc - 32)) * code
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q3_K>(const uint8_t *b, int c, float *y) {
    const float d = ldh(b + 108);
    const int h = c >> 2, j = c & 3;
    const uint8_t *q = b + 32 + 32 * h;
    for (int l = 0; l < 32; l++) {
        const float dl = d * static_cast<float>(q3k_scale(b + 96, 8 * h + 2 * j + l / 16) - 32);
        const int code = ((q[l] >> (2 * j)) & 3) - (((b[l] >> (4 * h + j)) & 1) ? 0 : 4);
        y[l] = dl * static_cast<float>(code);
    }
}

// MXFP4 half-scale exponent: 2^(e - 128) as f32 bits (e < 2: the denormals
// 2^-128, 2^-127), quant.cpp:319-330
__device__ __forceinline__ float e8m0_half(uint32_t e) {
    const uint32_t bits = e < 2 ? (0x00200000u << e) : ((e - 1) << 23);
    return __builtin_bit_cast(float, bits);
}
__constant__ static const int8_t kFp4Grid[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

// src/quant.cpp:674-686: value grid[q] * d, low nibbles first
template <>
__device__ __forceinline__ void dequant_chunk<DT_MXFP4>(const uint8_t *b, int, float *y) {
    const float d = e8m0_half(b[0]);
    for (int j = 0; j < 16; j++) {
        y[j] = static_cast<float>(kFp4Grid[b[1 + j] & 0xF]) * d;
        y[j + 16] = static_cast<float>(kFp4Grid[b[1 + j] >> 4]) * d;
    }
}

// ---------------------------------------------- generic-chunk formats ----
// These blocks sit at any byte alignment (17-, 10-, 54-byte blocks ...).
// The part runs global memory with unaligned access allowed, so a block's
// bytes come in as whole 16/8/4/2-byte loads at any address; no load reaches
// past the block's last byte.  Bytes are then taken out of the words with
// compile-time indices.
__device__ __forceinline__ u32x4 ldu16(const uint8_t *p) { u32x4 v; __builtin_memcpy(&v, p, 16); return v; }
__device__ __forceinline__ u32x2 ldu8(const uint8_t *p) { u32x2 v; __builtin_memcpy(&v, p, 8); return v; }
__device__ __forceinline__ uint32_t ldu4(const uint8_t *p) { uint32_t v; __builtin_memcpy(&v, p, 4); return v; }
__device__ __forceinline__ uint32_t ldu2(const uint8_t *p) { uint16_t v; __builtin_memcpy(&v, p, 2); return v; }
// byte k (a constant after unrolling) of a little-endian word array
template <int NW> __device__ __forceinline__ uint32_t byte_k(const uint32_t (&w)[NW], int k) {
    return (w[k >> 2] >> (8 * (k & 3))) & 0xFFu;
}
__device__ __forceinline__ void put4(uint32_t (&w)[4], u32x4 v, int at = 0) {
    w[at] = v.x; w[at + 1] = v.y; w[at + 2] = v.z; w[at + 3] = v.w;
}
template <int NW> __device__ __forceinline__ void put16(uint32_t (&w)[NW], u32x4 v, int at) {
    w[at] = v.x; w[at + 1] = v.y; w[at + 2] = v.z; w[at + 3] = v.w;
}

// src/quant.cpp:389-396: Q8_1, value d*q + s with the product rounded before
// the add (the reference build does not contract it)
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q8_1>(const uint8_t *b, int, float *y) {
    const uint32_t ds = ldu4(b);
    const float d = h2f(ds & 0xFFFFu), s = h2f(ds >> 16);
    uint32_t q[8];
    put16(q, ldu16(b + 4), 0);
    put16(q, ldu16(b + 20), 4);
#pragma unroll
    for (int k = 0; k < 32; k++)
        y[k] = __fadd_rn(__fmul_rn(d, static_cast<float>(static_cast<int8_t>(byte_k(q, k)))), s);
}

// src/quant.cpp:557-564: Q8_K, f32 d then 256 int8 codes (the 16 block sums
// after them are not read)
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q8_K>(const uint8_t *b, int c, float *y) {
    const float d = __builtin_bit_cast(float, ldu4(b));
    uint32_t q[8];
    put16(q, ldu16(b + 4 + 32 * c), 0);
    put16(q, ldu16(b + 20 + 32 * c), 4);
#pragma unroll
    for (int k = 0; k < 32; k++) y[k] = d * static_cast<float>(static_cast<int8_t>(byte_k(q, k)));
}

// src/quant.cpp:576-585: UE4M3 scale byte.  0x00 and 0x7F are 0, bit 7 is
// not read; exponent 0 gives m * 2^-9, else (1 + m/8) * 2^(e-7), both halved
// -- i.e. m * 2^-10 or (8 + m) * 2^(e-11), each exact in f32.
__device__ __forceinline__ float ue4m3_f(uint32_t x) {
    x &= 0xFFu;
    if (x == 0 || x == 0x7F) return 0.0f;
    const uint32_t e = (x >> 3) & 0xFu, m = x & 7u;
    if (e == 0) return static_cast<float>(m) * 0x1p-10f;
    return static_cast<float>(8u + m) * __builtin_bit_cast(float, (e + 116u) << 23);   // 2^(e - 11)
}

// the doubled E2M1 grid (kFp4Grid) of one code from two registers (v_perm
// picks magnitude byte q & 7 of 0, 1, 2, 3, 4, 6, 8, 12), bit 3 the sign: no
// per-lane constant-memory lookup
__device__ __forceinline__ int e2m1_grid(uint32_t q) {
    const int m = static_cast<int>(__builtin_amdgcn_perm(0x0C080604u, 0x03020100u, q & 7u) & 0xFFu);
    return (q & 8u) ? -m : m;
}

// src/quant.cpp:661-672: NVFP4, 64-value blocks: four UE4M3 scales, four
// 8-byte runs; chunk c is runs 2c and 2c + 1 (run s: value 16 s + j the low
// nibble of byte j, 16 s + 8 + j the high)
template <>
__device__ __forceinline__ void dequant_chunk<DT_NVFP4>(const uint8_t *b, int c, float *y) {
    const uint32_t sc = ldu2(b + 2 * c);
    uint32_t q[4];
    put4(q, ldu16(b + 4 + 16 * c));
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const float d = ue4m3_f(sc >> (8 * h));
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t v = byte_k(q, 8 * h + j);
            y[16 * h + j] = static_cast<float>(e2m1_grid(v & 0xFu)) * d;
            y[16 * h + 8 + j] = static_cast<float>(e2m1_grid(v >> 4)) * d;
        }
    }
}

// src/quant.cpp:310-318: ROCmFP4 ladder 0, 1, 2, 3, 4, 6, 8, 10, sign bit 3
__device__ __forceinline__ int rocmfp4_code(uint32_t q) {
    const int m = static_cast<int>(q & 7u), mag = m <= 4 ? m : 2 * m - 4;
    return (q & 8u) ? -mag : mag;
}
// src/quant.cpp:692-713: ROCmFP4 (two half scales after 16 nibble bytes)
// and ROCmFP4_FAST (one scale); value j the low nibble of byte j, j + 16 the
// high
template <bool TWO>
__device__ __forceinline__ void dequant_rocmfp4(const uint8_t *b, float *y) {
    uint32_t q[4];
    put4(q, ldu16(b));
    const uint32_t sc = TWO ? ldu2(b + 16) : b[16];
    const float d0 = ue4m3_f(sc), d1 = TWO ? ue4m3_f(sc >> 8) : d0;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t v = byte_k(q, j);
        y[j] = static_cast<float>(rocmfp4_code(v & 0xFu)) * d0;
        y[j + 16] = static_cast<float>(rocmfp4_code(v >> 4)) * d1;
    }
}
template <>
__device__ __forceinline__ void dequant_chunk<DT_ROCMFP4>(const uint8_t *b, int, float *y) { dequant_rocmfp4<true>(b, y); }
template <>
__device__ __forceinline__ void dequant_chunk<DT_ROCMFP4_FAST>(const uint8_t *b, int, float *y) {
    dequant_rocmfp4<false>(b, y);
}

// src/quant.cpp:740-857: the ROCmFPX formats, two UE4M3 half scales after
// the codes.  FP2: four codes a byte from the low bits on {-4, -1, 1, 4};
// FP3: eight 3-bit codes per 3 bytes, magnitude {0, 1, 2, 4}[c & 3], sign
// bit 2; FP6: four 6-bit codes per 3 bytes, magnitude c & 31, sign bit 5,
// negative zero = -32.  Code j of a packing of W bits per code, LSB first,
// is bits [W j, W j + W) of the code bytes (a group never splits a code).
template <int NW> __device__ __forceinline__ uint32_t bits_at(const uint32_t (&w)[NW], int bit, int n) {
    const uint32_t lo = w[bit >> 5] >> (bit & 31);
    const uint32_t hi = (bit & 31) + n > 32 ? w[(bit >> 5) + 1] << (32 - (bit & 31)) : 0u;
    return (lo | hi) & ((1u << n) - 1u);
}
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q2_0_ROCMFPX>(const uint8_t *b, int, float *y) {
    const u32x2 qq = ldu8(b);
    const uint32_t q[2] = {qq.x, qq.y};
    const uint32_t sc = ldu2(b + 8);
    const float d0 = ue4m3_f(sc), d1 = ue4m3_f(sc >> 8);
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const uint32_t c = bits_at(q, 2 * j, 2);
        const int v = c == 0 ? -4 : c == 1 ? -1 : c == 2 ? 1 : 4;
        y[j] = static_cast<float>(v) * (j < 16 ? d0 : d1);
    }
}
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q3_0_ROCMFPX>(const uint8_t *b, int, float *y) {
    const u32x2 qq = ldu8(b);
    const uint32_t q[3] = {qq.x, qq.y, ldu4(b + 8)};
    const uint32_t sc = ldu2(b + 12);
    const float d0 = ue4m3_f(sc), d1 = ue4m3_f(sc >> 8);
#pragma unroll
    for (int j = 0; j < 32; j++) {
        // group g = j / 8 is bytes 3g..3g+2, i.e. bits 24 g + 3 (j % 8)
        const uint32_t c = bits_at(q, 24 * (j >> 3) + 3 * (j & 7), 3);
        const int m = (c & 3u) == 3u ? 4 : static_cast<int>(c & 3u);
        y[j] = static_cast<float>((c & 4u) ? -m : m) * (j < 16 ? d0 : d1);
    }
}
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q6_0_ROCMFPX>(const uint8_t *b, int, float *y) {
    uint32_t q[6];
    put16(q, ldu16(b), 0);
    const u32x2 t = ldu8(b + 16);
    q[4] = t.x;
    q[5] = t.y;
    const uint32_t sc = ldu2(b + 24);
    const float d0 = ue4m3_f(sc), d1 = ue4m3_f(sc >> 8);
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const uint32_t c = bits_at(q, 24 * (j >> 2) + 6 * (j & 3), 6);
        const int m = static_cast<int>(c & 31u);
        y[j] = static_cast<float>((c & 32u) ? -(m == 0 ? 32 : m) : m) * (j < 16 ? d0 : d1);
    }
}

// src/quant.cpp:859-889: TQ1_0 trit n of byte q: ((uint8)(q * 3^n) * 3) >> 8,
// less 1.  Element v < 160: byte v % 32, trit v / 32; v < 240: byte
// 32 + (v - 160) % 16, trit (v - 160) / 16; else byte 48 + (v - 240) % 4,
// trit (v - 240) / 4.  f16 d at byte 52.  In chunk c (v = 32 c + k) the byte
// index depends on k alone: k (c < 5), 32 + k % 16 (c = 5, 6 and c = 7,
// k < 16), 48 + (k - 16) % 4 (c = 7, k >= 16).
__device__ __forceinline__ int tq1_trit(uint32_t q, int n) {
    const uint32_t p3 = n == 0 ? 1u : n == 1 ? 3u : n == 2 ? 9u : n == 3 ? 27u : 81u;
    return static_cast<int>((((q * p3) & 0xFFu) * 3u) >> 8) - 1;
}
template <>
__device__ __forceinline__ void dequant_chunk<DT_TQ1_0>(const uint8_t *b, int c, float *y) {
    const float d = h2f(ldu2(b + 52));
    if (c < 5) {
        uint32_t q[8];
        put16(q, ldu16(b), 0);
        put16(q, ldu16(b + 16), 4);
#pragma unroll
        for (int k = 0; k < 32; k++) y[k] = d * static_cast<float>(tq1_trit(byte_k(q, k), c));
        return;
    }
    uint32_t q[5];
    put16(q, ldu16(b + 32), 0);
    q[4] = ldu4(b + 48);
#pragma unroll
    for (int k = 0; k < 32; k++) {
        int t;
        if (c < 7 || k < 16) t = tq1_trit(byte_k(q, k & 15), 2 * (c - 5) + (k >> 4));
        else t = tq1_trit(byte_k(q, 16 + ((k - 16) & 3)), (k - 16) >> 2);
        y[k] = d * static_cast<float>(t);
    }
}

// src/quant.cpp:907-918: TQ2_0, element 128 h + 32 l + m is bits 2l of byte
// 32 h + m, value d (q - 1); f16 d at byte 64.  Chunk c: h = c / 4, l = c % 4.
template <>
__device__ __forceinline__ void dequant_chunk<DT_TQ2_0>(const uint8_t *b, int c, float *y) {
    const float d = h2f(ldu2(b + 64));
    const int h = c >> 2, l = c & 3;
    uint32_t q[8];
    put16(q, ldu16(b + 32 * h), 0);
    put16(q, ldu16(b + 32 * h + 16), 4);
#pragma unroll
    for (int m = 0; m < 32; m++)
        y[m] = d * static_cast<float>(static_cast<int>((byte_k(q, m) >> (2 * l)) & 3u) - 1);
}

// src/quant_fmt_a.inc:71-83: Q1_0, one bit per value from the low bit, +d
// for a 1 and -d for a 0; chunk c is bytes 2 + 4c .. 2 + 4c + 3
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q1_0>(const uint8_t *b, int c, float *y) {
    const float d = h2f(ldu2(b));
    const uint32_t w = ldu4(b + 2 + 4 * c);
#pragma unroll
    for (int k = 0; k < 32; k++) y[k] = ((w >> k) & 1u) ? d : -d;
}
// src/quant_fmt_a.inc:85-129: Q2_0 / PQ2_0 (128 values) and Q2_0_64 (64):
// 2-bit codes four to a byte from the low pair, value (q - 1) * d; chunk c is
// bytes 2 + 8c .. 2 + 8c + 7
__device__ __forceinline__ void dequant_q2_0n(const uint8_t *b, int c, float *y) {
    const float d = h2f(ldu2(b));
    const u32x2 w = ldu8(b + 2 + 8 * c);
#pragma unroll
    for (int k = 0; k < 32; k++)
        y[k] = static_cast<float>(static_cast<int>(((k < 16 ? w.x : w.y) >> (2 * (k & 15))) & 3u) - 1) * d;
}
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q2_0>(const uint8_t *b, int c, float *y) { dequant_q2_0n(b, c, y); }
template <>
__device__ __forceinline__ void dequant_chunk<DT_PQ2_0>(const uint8_t *b, int c, float *y) { dequant_q2_0n(b, c, y); }
template <>
__device__ __forceinline__ void dequant_chunk<DT_Q2_0_64>(const uint8_t *b, int c, float *y) { dequant_q2_0n(b, c, y); }
// src/quant.cpp:933-950: PTQ1_0, TQ1_0's trits at group 128, f16 d at 26:
// v < 80 byte v % 16 trit v / 16; v < 120 byte 16 + (v - 80) % 8 trit
// (v - 80) / 8; else byte 24 + (v - 120) % 2 trit (v - 120) / 2.  The whole
// 26 code bytes are loaded; each (chunk, k) names its byte and trit.
template <>
__device__ __forceinline__ void dequant_chunk<DT_PTQ1_0>(const uint8_t *b, int c, float *y) {
    uint32_t q[7];
    put16(q, ldu16(b), 0);
    const u32x2 t8 = ldu8(b + 16);
    q[4] = t8.x;
    q[5] = t8.y;
    const uint32_t dq = ldu4(b + 24);
    q[6] = dq & 0xFFFFu;
    const float d = h2f(dq >> 16);
#pragma unroll
    for (int k = 0; k < 32; k++) {
        const int v = 32 * c + k;
        int t;
        if (v < 80) t = tq1_trit(byte_k(q, k & 15), v >> 4);
        else if (v < 120) t = tq1_trit(byte_k(q, 16 + (k & 7)), (v - 80) >> 3);
        else t = tq1_trit(byte_k(q, 24 + (k & 1)), (v - 120) >> 1);
        y[k] = d * static_cast<float>(t);
    }
}

// F16 / BF16 weights (dequant.hpp:428-440): widening, exact
template <>
__device__ __forceinline__ void dequant_chunk<DT_F16>(const uint8_t *b, int, float *y) {
    for (int j = 0; j < 32; j++) y[j] = ldh(b + 2 * j);
}
__device__ __forceinline__ float bf2f(uint32_t h) { return __builtin_bit_cast(float, h << 16); }
template <>
__device__ __forceinline__ void dequant_chunk<DT_BF16>(const uint8_t *b, int, float *y) {
    for (int j = 0; j < 32; j++)
        y[j] = bf2f(static_cast<uint32_t>(b[2 * j]) | (static_cast<uint32_t>(b[2 * j + 1]) << 8));
}

// ----------------------------------------------------- aligned raw loads ----
// NW dwords holding bytes [p, p + 4*NW) of a 2-byte aligned pointer.  Only
// dwords overlapping that range are read; a 4-aligned dword never crosses a
// page, so a block's bytes can be fetched without reading past the buffer.
template <int NW>
__device__ __forceinline__ void load_bytes2(const uint8_t *p, uint32_t (&o)[NW]);

// the byte at p, from the 4-aligned dword that holds it
__device__ __forceinline__ uint32_t byte_at(const uint8_t *p) {
    return ld32_at(p) & 0xFF;
}

// (any byte alignment works: the window shift is a & 3)
template <int NW>
__device__ __forceinline__ void load_bytes2(const uint8_t *p, uint32_t (&o)[NW]) {
    const uint32_t s = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3);
    const uint8_t *base = p - s;   // pointer arithmetic keeps p's address space
    uint32_t d[NW + 1];
#pragma unroll
    for (int k = 0; k < NW; k++) d[k] = ld32(base + 4 * k);
    d[NW] = s ? ld32(base + 4 * NW) : 0u;
#pragma unroll
    for (int k = 0; k < NW; k++) o[k] = align_bytes(d[k + 1], d[k], s);
}

// ------------------------------------------------ legacy 32-value formats --
// Q4_1, Q5_0, Q5_1 (src/quant.cpp:341-378): f16 d at 0, an f16 min m at 2
// (Q4_1, Q5_1), a 32-bit high-bit plane qh (Q5_0 at 2, Q5_1 at 4; bit k is
// bit 4 of value k's code), 16 code bytes (value k the low nibble of byte
// k, k + 16 the high).  Value d*q + m, or d*(q - 16) for Q5_0.
template <int DT> struct L32;
template <> struct L32<DT_Q4_1> { static constexpr int BB = 20, QH = -1, QS = 4, BIAS = 0; static constexpr bool M = true; };
template <> struct L32<DT_Q5_0> { static constexpr int BB = 22, QH = 2, QS = 6, BIAS = 16; static constexpr bool M = false; };
template <> struct L32<DT_Q5_1> { static constexpr int BB = 24, QH = 4, QS = 8, BIAS = 0; static constexpr bool M = true; };

template <int DT>
__device__ __forceinline__ void dequant_l32(const uint8_t *b, float *y) {
    using L = L32<DT>;
    const float d = ldh(b), m = L::M ? ldh(b + 2) : 0.0f;
    uint32_t qh = 0;
    if constexpr (L::QH >= 0)
        qh = static_cast<uint32_t>(b[L::QH]) | (static_cast<uint32_t>(b[L::QH + 1]) << 8) |
             (static_cast<uint32_t>(b[L::QH + 2]) << 16) | (static_cast<uint32_t>(b[L::QH + 3]) << 24);
    for (int k = 0; k < 16; k++) {
        const int lo = (b[L::QS + k] & 0xF) | static_cast<int>(((qh >> k) & 1u) << 4);
        const int hi = (b[L::QS + k] >> 4) | static_cast<int>(((qh >> (k + 16)) & 1u) << 4);
        if constexpr (L::M) {
            y[k] = __builtin_fmaf(d, static_cast<float>(lo), m);
            y[k + 16] = __builtin_fmaf(d, static_cast<float>(hi), m);
        } else {
            y[k] = d * static_cast<float>(lo - L::BIAS);
            y[k + 16] = d * static_cast<float>(hi - L::BIAS);
        }
    }
}
template <> __device__ __forceinline__ void dequant_chunk<DT_Q4_1>(const uint8_t *b, int, float *y) { dequant_l32<DT_Q4_1>(b, y); }
template <> __device__ __forceinline__ void dequant_chunk<DT_Q5_0>(const uint8_t *b, int, float *y) { dequant_l32<DT_Q5_0>(b, y); }
template <> __device__ __forceinline__ void dequant_chunk<DT_Q5_1>(const uint8_t *b, int, float *y) { dequant_l32<DT_Q5_1>(b, y); }

// one block's raw words: codes q[0..3], qh, and d (low half) | m (high half)
template <int DT>
__device__ __forceinline__ void load_l32(const uint8_t *blk, uint32_t *raw) {
    using L = L32<DT>;
    uint32_t q[4], h[1] = {0u}, dm[1];
    load_bytes2<4>(blk + L::QS, q);
    if constexpr (L::QH >= 0) load_bytes2<1>(blk + L::QH, h);
    if constexpr (L::M) {
        load_bytes2<1>(blk, dm);
    } else {
        dm[0] = ld32_at(blk);
    }
    raw[0] = q[0]; raw[1] = q[1]; raw[2] = q[2]; raw[3] = q[3];
    raw[4] = h[0]; raw[5] = dm[0];
}
// four bits b0..b3 of n as bit 4 of four bytes
__device__ __forceinline__ uint32_t spread4(uint32_t n) { return ((n * 0x00204081u) & 0x01010101u) << 4; }
// codes of values 4t..4t+3 (hi = 0) or 16+4t.. (hi = 1) as four bytes
template <int DT>
__device__ __forceinline__ uint32_t l32_codes(const uint32_t *raw, int t, int hi) {
    const uint32_t n = (raw[t] >> (4 * hi)) & 0x0F0F0F0Fu;
    if constexpr (L32<DT>::QH >= 0) return n | spread4((raw[4] >> (16 * hi + 4 * t)) & 0xFu);
    return n;
}
// --------------------------------------------------------------- LaneFmt ----
// The lane view: LPB lanes per block, each owning 32 values ("a piece").
// run_start(p, r) is where, inside the block, the r-th run of RUN consecutive
// values of piece p starts; the lane's activations arrive in that order as
// xv[0..31].  dot() returns the piece's contribution sum_i w_i * xv_i.
//
// Codes are never converted with v_cvt: a code c < 1024 placed in the low 10
// bits of a 16-bit lane IS the f16 subnormal c * 2^-24, which v_fma_mix_f32
// widens exactly inside the FMA.  So sum_i c_i * x_i costs one FMA per value
// plus ~0.6 ops of masking, and the 2^24 goes back into the block scale
// (a power of two: exact).  Per group g of values sharing a scale:
//     contribution = scale_g * 2^24 * sum(c_i * x_i) - off_g * sum(x_i)
// where off_g folds the format's zero point (Q4_K's min, Q6_K's 32, ...).
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }

// acc += c(v.lo) * x0 + c(v.hi) * x1 for a dword holding two codes
__device__ __forceinline__ float mix2(uint32_t v, float x0, float x1, float acc) {
    const half2v h = as_h2(v);
    acc = __builtin_fmaf(static_cast<float>(h.x), x0, acc);
    return __builtin_fmaf(static_cast<float>(h.y), x1, acc);
}

// Eight 4-bit codes of a dword: bytes k = 0..3 hold (lo nibble, hi nibble).
// Low nibbles go to xl[k], high nibbles (as 16*c) to xh[k].
__device__ __forceinline__ void nib8(uint32_t v, const float *xl, const float *xh, float &sl,
                                     float &sh) {
    const uint32_t s8 = v >> 8;
    sl = mix2(v & 0x000F000Fu, xl[0], xl[2], sl);
    sl = mix2(s8 & 0x000F000Fu, xl[1], xl[3], sl);
    sh = mix2(v & 0x00F000F0u, xh[0], xh[2], sh);
    sh = mix2(s8 & 0x00F000F0u, xh[1], xh[3], sh);
}

constexpr float kTwo24 = 16777216.0f, kTwo20 = 1048576.0f;

// The 6-bit (scale, min) bytes of sub-blocks 2j and 2j+1 from a K-quant
// header held as dwords raw[1..3] (get_scale_min_k4, quant.cpp:427-435).
__device__ __forceinline__ void q4k_pair_scale_bytes(const uint32_t *raw, int j, uint32_t &sa, uint32_t &sb,
                                                     uint32_t &ma, uint32_t &mb) {
    const uint32_t sh = 16u * static_cast<uint32_t>(j & 1);
    const uint32_t Y = raw[1] >> sh, Z = raw[2] >> sh, W = raw[3] >> sh;
    const bool hi = j >= 2;
    const uint32_t A = hi ? W : Y, Am = hi ? (W >> 4) : Z, s2 = hi ? 2u : 0u;
    sa = (A & 15u) | ((Y >> s2) & 0x30u);
    sb = ((A >> 8) & 15u) | ((Y >> (8u + s2)) & 0x30u);
    ma = (Am & 15u) | ((Z >> s2) & 0x30u);
    mb = ((Am >> 8) & 15u) | ((Z >> (8u + s2)) & 0x30u);
}

template <int DT> struct LaneFmt;

// Q4_K: piece p covers qs bytes [16p, 16p+16): sub-block 2j low nibbles
// (values 64j + 16(p&1) + i) and sub-block 2j+1 high nibbles, j = p/2.
template <> struct LaneFmt<DT_Q4_K> {
    static constexpr int LPB = 8, NG = 2, RUN = 16, NRUN = 2, NRAW = 8;
    __device__ static int run_start(int p, int r) { return 64 * (p >> 1) + 32 * r + 16 * (p & 1); }
    __device__ static int group_of(int i) { return i >> 4; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int p) {
        const u32x4 h = ld128(blk);
        const u32x4 q = ld128(blk + 16 + 16 * p);
        raw[0] = h.x; raw[1] = h.y; raw[2] = h.z; raw[3] = h.w;
        raw[4] = q.x; raw[5] = q.y; raw[6] = q.z; raw[7] = q.w;
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int p, const float (&xv)[32],
                                const float (&xs)[NG]) {
        const float d = h2f(raw[0] & 0xFFFF), dmin = h2f(raw[0] >> 16);
        // this lane's two sub-blocks 2j, 2j+1 (get_scale_min_k4, quant.cpp:427)
        const uint32_t sh = 16u * static_cast<uint32_t>((p >> 1) & 1);
        const uint32_t Y = raw[1] >> sh, Z = raw[2] >> sh, W = raw[3] >> sh;
        uint32_t sa, sb, ma, mb;
        if (p < 4) {
            sa = Y & 63; sb = (Y >> 8) & 63; ma = Z & 63; mb = (Z >> 8) & 63;
        } else {
            sa = (W & 0xF) | (((Y >> 6) & 3) << 4);
            sb = ((W >> 8) & 0xF) | (((Y >> 14) & 3) << 4);
            ma = ((W >> 4) & 0xF) | (((Z >> 6) & 3) << 4);
            mb = ((W >> 12) & 0xF) | (((Z >> 14) & 3) << 4);
        }
        float sl = 0.0f, shi = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) nib8(raw[4 + t], &xv[4 * t], &xv[16 + 4 * t], sl, shi);
        const float dl = d * static_cast<float>(sa), dh = d * static_cast<float>(sb);
        float a = (dl * kTwo24) * sl;
        a = __builtin_fmaf(dh * kTwo20, shi, a);
        a = __builtin_fmaf(-dmin * static_cast<float>(ma), xs[0], a);
        return __builtin_fmaf(-dmin * static_cast<float>(mb), xs[1], a);
    }
};

// Five-bit codes of a dword of code bytes A and high-bit bytes H: the nibble
// at bit NS of each byte of A, plus bit HB of each byte of H as bit 4,
// summed against x as f16 subnormals (c * 2^-24) like nib8.
__device__ __forceinline__ float q5x4(uint32_t A, uint32_t H, int ns, int hb, const float *x, float acc) {
    const uint32_t q = ((A >> ns) & 0x0F0F0F0Fu) | (((H >> hb) << 4) & 0x10101010u);
    acc = mix2(q & 0x001F001Fu, x[0], x[2], acc);
    return mix2((q >> 8) & 0x001F001Fu, x[1], x[3], acc);
}

// Q5_K: piece p covers qs bytes [16p, 16p+16) (at block offset 48) and the
// same 16 positions l of qh: sub-block 2j low nibbles + qh bit 2j (values
// 64j + 16(p&1) + i), sub-block 2j+1 high nibbles + qh bit 2j+1, j = p/2.
template <> struct LaneFmt<DT_Q5_K> {
    static constexpr int LPB = 8, NG = 2, RUN = 16, NRUN = 2, NRAW = 12;
    __device__ static int run_start(int p, int r) { return 64 * (p >> 1) + 32 * r + 16 * (p & 1); }
    __device__ static int group_of(int i) { return i >> 4; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int p) {
        const u32x4 h = ld128(blk);
        const u32x4 hb = ld128(blk + 16 + 16 * (p & 1));
        const u32x4 q = ld128(blk + 48 + 16 * p);
        raw[0] = h.x; raw[1] = h.y; raw[2] = h.z; raw[3] = h.w;
        raw[4] = q.x; raw[5] = q.y; raw[6] = q.z; raw[7] = q.w;
        raw[8] = hb.x; raw[9] = hb.y; raw[10] = hb.z; raw[11] = hb.w;
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int p, const float (&xv)[32],
                                const float (&xs)[NG]) {
        const float d = h2f(raw[0] & 0xFFFF), dmin = h2f(raw[0] >> 16);
        const int j = p >> 1;
        uint32_t sa, sb, ma, mb;
        q4k_pair_scale_bytes(raw, j, sa, sb, ma, mb);
        float sl = 0.0f, shi = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            sl = q5x4(raw[4 + t], raw[8 + t], 0, 2 * j, &xv[4 * t], sl);
            shi = q5x4(raw[4 + t], raw[8 + t], 4, 2 * j + 1, &xv[16 + 4 * t], shi);
        }
        float a = (d * static_cast<float>(sa) * kTwo24) * sl;
        a = __builtin_fmaf(d * static_cast<float>(sb) * kTwo24, shi, a);
        a = __builtin_fmaf(-dmin * static_cast<float>(ma), xs[0], a);
        return __builtin_fmaf(-dmin * static_cast<float>(mb), xs[1], a);
    }
};

// Q6_K: piece p = (half h = p/4, sub = p%4): values 128h + 32qd + 8sub + t for
// quadrant qd (0..3) and t (0..7).  Needs ql[64h+8sub..+8], ql[64h+32+8sub..+8],
// qh[32h+8sub..+8], scales sc[8h + sub/2 + 2qd] and d.
template <> struct LaneFmt<DT_Q6_K> {
    static constexpr int LPB = 8, NG = 4, RUN = 8, NRUN = 4, NRAW = 9;
    __device__ static int run_start(int p, int r) { return 128 * (p >> 2) + 32 * r + 8 * (p & 3); }
    __device__ static int group_of(int i) { return i >> 3; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int p) {
        const int h = p >> 2, o = 8 * (p & 3);
        uint32_t a[2], b[2], q[2], s[2];
        load_bytes2<2>(blk + 64 * h + o, a);
        load_bytes2<2>(blk + 64 * h + 32 + o, b);
        load_bytes2<2>(blk + 128 + 32 * h + o, q);
        load_bytes2<2>(blk + 192 + 8 * h, s);
        // d is the last two bytes of the block; read the dword that holds them
        // without touching anything past the block.
        raw[8] = ld32_at(blk + 208);
        raw[0] = a[0]; raw[1] = a[1]; raw[2] = b[0]; raw[3] = b[1];
        raw[4] = q[0]; raw[5] = q[1]; raw[6] = s[0]; raw[7] = s[1];
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int p, const float (&xv)[32],
                                const float (&xs)[NG]) {
        const float d = h2f(raw[8] & 0xFFFF);
        const int sub2 = (p & 3) >> 1;
        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint32_t A = raw[t], B = raw[2 + t], H = raw[4 + t];
            // byte-parallel 6-bit codes of the four quadrants
            const uint32_t q[4] = {(A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u),
                                   (B & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u),
                                   ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u),
                                   ((B >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u)};
#pragma unroll
            for (int qd = 0; qd < 4; qd++) {
                const float *x = &xv[8 * qd + 4 * t];
                s[qd] = mix2(q[qd] & 0x003F003Fu, x[0], x[2], s[qd]);
                s[qd] = mix2((q[qd] >> 8) & 0x003F003Fu, x[1], x[3], s[qd]);
            }
        }
        float a = 0.0f;
#pragma unroll
        for (int qd = 0; qd < 4; qd++) {
            const int idx = sub2 + 2 * qd;  // byte in the 8 scale bytes
            const uint32_t sw = idx < 4 ? raw[6] : raw[7];
            const int s8 = static_cast<int32_t>(sw << (24 - 8 * (idx & 3))) >> 24;
            const float ds = d * static_cast<float>(s8);
            a = __builtin_fmaf(ds * kTwo24, s[qd], a);
            a = __builtin_fmaf(-32.0f * ds, xs[qd], a);
        }
        return a;
    }
};

// Two-bit planes (Q2_K, Q3_K).  Plane j of four code bytes q as byte-parallel
// codes; Q3_K adds 4 where the hmask bit is set (non-negative codes 0..7,
// the -4 going into the x-sum term).
__device__ __forceinline__ uint32_t plane2(uint32_t q, int j) { return (q >> (2 * j)) & 0x03030303u; }
__device__ __forceinline__ uint32_t plane3(uint32_t q, uint32_t hm, int bit) {
    return ((q >> 0) & 0x03030303u) | (((hm >> bit) & 0x01010101u) << 2);
}
// Q2_K (scale, min) of scale byte idx (0..7) held in two dwords
__device__ __forceinline__ uint32_t byte_of(uint32_t w0, uint32_t w1, int idx) {
    return ((idx < 4 ? w0 : w1) >> (8 * (idx & 3))) & 0xFF;
}
// Q3_K scale 8h + b (b = 2j + s, 0..7) from the packed dwords R0, R1, R2 of
// bytes 96..107: low nibble of byte b at 4h, two high bits from byte 8 + b % 4
// at 4h + 2 (j / 2)
__device__ __forceinline__ int q3k_scale_w(uint32_t R0, uint32_t R1, uint32_t R2, int h, int b) {
    const uint32_t lo = (byte_of(R0, R1, b) >> (4 * h)) & 0xF;
    const uint32_t hi = (R2 >> (8 * (b & 3) + 4 * h + 2 * (b >> 2))) & 3;
    return static_cast<int>(lo | (hi << 4));
}

// Q3_K's d (bytes 108..109) in the low half of a dword, read from the
// 4-aligned dword that holds them, which never leaves the block's page
__device__ __forceinline__ uint32_t q3k_d_word(const uint8_t *blk) {
    return ld32_at(blk + 108);
}

// Q2_K lane view: piece p, half h = p / 4, bytes o = 8 (p % 4) .. +7 of the
// half's 32 code bytes; run r = plane j (values 128h + 32j + o + t).
template <> struct LaneFmt<DT_Q2_K> {
    static constexpr int LPB = 8, NG = 4, RUN = 8, NRUN = 4, NRAW = 5;
    __device__ static int run_start(int p, int r) { return 128 * (p >> 2) + 32 * r + 8 * (p & 3); }
    __device__ static int group_of(int i) { return i >> 3; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int p) {
        const int h = p >> 2, o = 8 * (p & 3);
        const u32x2 q = ld64(blk + 16 + 32 * h + o), sc = ld64(blk + 8 * h);
        raw[0] = q.x; raw[1] = q.y; raw[2] = sc.x; raw[3] = sc.y;
        raw[4] = ld32(blk + 80);
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int p, const float (&xv)[32],
                                const float (&xs)[NG]) {
        const float d = h2f(raw[4] & 0xFFFF), dmin = h2f(raw[4] >> 16);
        const int s = (p & 3) >> 1;
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float sj = 0.0f;
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint32_t q = plane2(raw[t], j);
                const float *x = &xv[8 * j + 4 * t];
                sj = mix2(q & 0x00030003u, x[0], x[2], sj);
                sj = mix2((q >> 8) & 0x00030003u, x[1], x[3], sj);
            }
            const uint32_t sc = byte_of(raw[2], raw[3], 2 * j + s);
            a = __builtin_fmaf(d * static_cast<float>(sc & 0xF) * kTwo24, sj, a);
            a = __builtin_fmaf(-(dmin * static_cast<float>(sc >> 4)), xs[j], a);
        }
        return a;
    }
};

// Q3_K lane view: as Q2_K's, with the hmask bytes o .. +7 (bit 4h + j)
template <> struct LaneFmt<DT_Q3_K> {
    static constexpr int LPB = 8, NG = 4, RUN = 8, NRUN = 4, NRAW = 8;
    __device__ static int run_start(int p, int r) { return 128 * (p >> 2) + 32 * r + 8 * (p & 3); }
    __device__ static int group_of(int i) { return i >> 3; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int p) {
        const int h = p >> 2, o = 8 * (p & 3);
        uint32_t q[2], m[2], sc[3];
        load_bytes2<2>(blk + 32 + 32 * h + o, q);
        load_bytes2<2>(blk + o, m);
        load_bytes2<3>(blk + 96, sc);
        raw[0] = q[0]; raw[1] = q[1]; raw[2] = m[0]; raw[3] = m[1];
        raw[4] = sc[0]; raw[5] = sc[1]; raw[6] = sc[2];
        raw[7] = q3k_d_word(blk);
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int p, const float (&xv)[32],
                                const float (&xs)[NG]) {
        const float d = h2f(raw[7] & 0xFFFF);
        const int h = p >> 2, s = (p & 3) >> 1;
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float sj = 0.0f;
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const uint32_t q = plane3(raw[t] >> (2 * j), raw[2 + t], 4 * h + j);
                const float *x = &xv[8 * j + 4 * t];
                sj = mix2(q & 0x00070007u, x[0], x[2], sj);
                sj = mix2((q >> 8) & 0x00070007u, x[1], x[3], sj);
            }
            const float dl = d * static_cast<float>(q3k_scale_w(raw[4], raw[5], raw[6], h, 2 * j + s) - 32);
            a = __builtin_fmaf(dl * kTwo24, sj, a);
            a = __builtin_fmaf(-4.0f * dl, xs[j], a);
        }
        return a;
    }
};

// Q4_0: one lane per 32-value block.  Low nibbles are values 0..15, high
// nibbles 16..31; value = d * (q - 8).
template <> struct LaneFmt<DT_Q4_0> {
    static constexpr int LPB = 1, NG = 2, RUN = 32, NRUN = 1, NRAW = 5;
    __device__ static int run_start(int, int) { return 0; }
    __device__ static int group_of(int i) { return i >> 4; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) {
        uint32_t q[4];
        load_bytes2<4>(blk + 2, q);
        raw[4] = ld32_at(blk);
        raw[0] = q[0]; raw[1] = q[1]; raw[2] = q[2]; raw[3] = q[3];
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int, const float (&xv)[32],
                                const float (&xs)[NG]) {
        const float d = h2f(raw[4] & 0xFFFF);
        float sl = 0.0f, shi = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) nib8(raw[t], &xv[4 * t], &xv[16 + 4 * t], sl, shi);
        float a = (d * kTwo24) * sl;
        a = __builtin_fmaf(d * kTwo20, shi, a);
        return __builtin_fmaf(-8.0f * d, xs[0] + xs[1], a);
    }
};

// IQ4_NL grid values biased by 128 (1..241), as bytes: grid lookups of four
// indices at a time with v_perm (a selector byte 0..7 picks a byte of the
// 8-byte table in its two dword operands), two halves joined on index bit 3
constexpr uint32_t kIq4B0 = 0x3F2D1801u, kIq4B1 = 0x766A5D4Fu, kIq4B2 = 0xA6998D81u, kIq4B3 = 0xF1D9C5B5u;
__device__ __forceinline__ uint32_t iq4_lookup(uint32_t idx) {   // idx: four indices 0..15 as bytes
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kIq4B1, kIq4B0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(kIq4B3, kIq4B2, sel);
    const uint32_t m = ((idx >> 3) & 0x01010101u) * 0xFFu;
    return (hi & m) | (lo & ~m);
}
// the same lookup over the MXFP4 grid biased by 12 (0..24): a small bias
// keeps the x-sum correction at the grid's own magnitude
constexpr uint32_t kFp4B0 = 0x0F0E0D0Cu, kFp4B1 = 0x18141210u, kFp4B2 = 0x090A0B0Cu, kFp4B3 = 0x00040608u;
__device__ __forceinline__ uint32_t fp4_lookup(uint32_t idx) {
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kFp4B1, kFp4B0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(kFp4B3, kFp4B2, sel);
    const uint32_t m = ((idx >> 3) & 0x01010101u) * 0xFFu;
    return (hi & m) | (lo & ~m);
}
// acc += sum over the 8 indices of a dword (low nibbles with xl[0..3], high
// nibbles with xh[0..3]) of (grid + bias) * 2^-24 * x, as f16 subnormals
template <bool FP4 = false>
__device__ __forceinline__ float iq4x8(uint32_t v, const float *xl, const float *xh, float acc) {
    const uint32_t a = FP4 ? fp4_lookup(v & 0x0F0F0F0Fu) : iq4_lookup(v & 0x0F0F0F0Fu);
    const uint32_t b = FP4 ? fp4_lookup((v >> 4) & 0x0F0F0F0Fu) : iq4_lookup((v >> 4) & 0x0F0F0F0Fu);
    acc = mix2(a & 0x00FF00FFu, xl[0], xl[2], acc);
    acc = mix2((a >> 8) & 0x00FF00FFu, xl[1], xl[3], acc);
    acc = mix2(b & 0x00FF00FFu, xh[0], xh[2], acc);
    return mix2((b >> 8) & 0x00FF00FFu, xh[1], xh[3], acc);
}

// IQ4_NL: Q4_0's block (one lane per block), value d * grid[q]; the 128 bias
// comes off through the x sums
template <> struct LaneFmt<DT_IQ4_NL> {
    static constexpr int LPB = 1, NG = 2, RUN = 32, NRUN = 1, NRAW = 5;
    __device__ static int run_start(int, int) { return 0; }
    __device__ static int group_of(int i) { return i >> 4; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int p) {
        LaneFmt<DT_Q4_0>::load(raw, blk, p);
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int, const float (&xv)[32],
                                const float (&xs)[NG]) {
        const float d = h2f(raw[4] & 0xFFFF);
        float s = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) s = iq4x8(raw[t], &xv[4 * t], &xv[16 + 4 * t], s);
        return __builtin_fmaf(-128.0f * d, xs[0] + xs[1], (d * kTwo24) * s);
    }
};

// MXFP4: one lane per 17-byte block (byte aligned): the 16 code bytes by an
// in-block window, the exponent byte by its aligned dword
template <> struct LaneFmt<DT_MXFP4> {
    static constexpr int LPB = 1, NG = 2, RUN = 32, NRUN = 1, NRAW = 5;
    __device__ static int run_start(int, int) { return 0; }
    __device__ static int group_of(int i) { return i >> 4; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) {
        uint32_t q[4];
        load_bytes2<4>(blk + 1, q);
        raw[0] = q[0]; raw[1] = q[1]; raw[2] = q[2]; raw[3] = q[3];
        raw[4] = byte_at(blk);
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int, const float (&xv)[32],
                                const float (&xs)[NG]) {
        const float d = e8m0_half(raw[4]);
        float s = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) s = iq4x8<true>(raw[t], &xv[4 * t], &xv[16 + 4 * t], s);
        return __builtin_fmaf(-12.0f * d, xs[0] + xs[1], (d * kTwo24) * s);
    }
};

// sum_i code_i * 2^-24 * x_i over the block's 32 values (xl: 0..15, xh: 16..31)
template <int DT>
__device__ __forceinline__ float l32_sum(const uint32_t *raw, const float *xl, const float *xh, float s) {
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int hi = 0; hi < 2; hi++) {
            const uint32_t c = l32_codes<DT>(raw, t, hi);
            const float *x = (hi ? xh : xl) + 4 * t;
            s = mix2(c & 0x001F001Fu, x[0], x[2], s);
            s = mix2((c >> 8) & 0x001F001Fu, x[1], x[3], s);
        }
    return s;
}
// the block's dot from the code sum s and the block's x sum
template <int DT>
__device__ __forceinline__ float l32_fold(const uint32_t *raw, float s, float xsum, float acc) {
    const float d = h2f(raw[5] & 0xFFFF);
    acc = __builtin_fmaf(d * 16777216.0f, s, acc);
    const float off = L32<DT>::M ? h2f(raw[5] >> 16) : -static_cast<float>(L32<DT>::BIAS) * d;
    return __builtin_fmaf(off, xsum, acc);
}

template <int DT> struct LaneFmtL32 {
    static constexpr int LPB = 1, NG = 2, RUN = 32, NRUN = 1, NRAW = 6;
    __device__ static int run_start(int, int) { return 0; }
    __device__ static int group_of(int i) { return i >> 4; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) { load_l32<DT>(blk, raw); }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int, const float (&xv)[32],
                                const float (&xs)[NG]) {
        return l32_fold<DT>(raw, l32_sum<DT>(raw, &xv[0], &xv[16], 0.0f), xs[0] + xs[1], 0.0f);
    }
};
template <> struct LaneFmt<DT_Q4_1> : LaneFmtL32<DT_Q4_1> {};
template <> struct LaneFmt<DT_Q5_0> : LaneFmtL32<DT_Q5_0> {};
template <> struct LaneFmt<DT_Q5_1> : LaneFmtL32<DT_Q5_1> {};

// F16 / BF16 weights: one lane per 32-value pseudo-block (64 bytes, rows
// 16-byte aligned); F16 values enter v_fma_mix as f16 operands, BF16 values
// widen by a shift
template <int DT> struct LaneFmtFloat {
    static constexpr int LPB = 1, NG = 1, RUN = 32, NRUN = 1, NRAW = 16;
    __device__ static int run_start(int, int) { return 0; }
    __device__ static int group_of(int) { return 0; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const u32x4 v = ld128(blk + 16 * k);
            raw[4 * k] = v.x; raw[4 * k + 1] = v.y; raw[4 * k + 2] = v.z; raw[4 * k + 3] = v.w;
        }
    }
    __device__ static float pair(uint32_t v, float x0, float x1, float acc) {
        if constexpr (DT == DT_F16) return mix2(v, x0, x1, acc);
        acc = __builtin_fmaf(__builtin_bit_cast(float, v << 16), x0, acc);
        return __builtin_fmaf(__builtin_bit_cast(float, v & 0xFFFF0000u), x1, acc);
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int, const float (&xv)[32], const float (&)[NG]) {
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; k += 2) {
            a = pair(raw[k], xv[2 * k], xv[2 * k + 1], a);
            b = pair(raw[k + 1], xv[2 * k + 2], xv[2 * k + 3], b);
        }
        return a + b;
    }
};
template <> struct LaneFmt<DT_F16> : LaneFmtFloat<DT_F16> {};
template <> struct LaneFmt<DT_BF16> : LaneFmtFloat<DT_BF16> {};

// IQ4_XS scale of sub-block ib from the header dwords h0 = d | scales_h << 16
// and h1 = scales_l[0..3]: d * (ls - 32) (quant.cpp:646-650)
__device__ __forceinline__ float iq4xs_scale(uint32_t h0, uint32_t h1, int ib) {
    const uint32_t ls = ((h1 >> (4 * ib)) & 0xFu) | (((h0 >> (16 + 2 * ib)) & 3u) << 4);
    return h2f(h0 & 0xFFFF) * static_cast<float>(static_cast<int>(ls) - 32);
}

// IQ4_XS: piece p = sub-block p (32 values: 16 index bytes at 8 + 16p, low
// nibbles first), eight lanes per 256-value block
template <> struct LaneFmt<DT_IQ4_XS> {
    static constexpr int LPB = 8, NG = 2, RUN = 32, NRUN = 1, NRAW = 6;
    __device__ static int run_start(int p, int) { return 32 * p; }
    __device__ static int group_of(int i) { return i >> 4; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int p) {
        const u32x2 h = ld64(blk);
        const u32x4 q = ld128(blk + 8 + 16 * p);
        raw[0] = q.x; raw[1] = q.y; raw[2] = q.z; raw[3] = q.w;
        raw[4] = h.x; raw[5] = h.y;
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int p, const float (&xv)[32],
                                const float (&xs)[NG]) {
        const float dl = iq4xs_scale(raw[4], raw[5], p);
        float s = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) s = iq4x8(raw[t], &xv[4 * t], &xv[16 + 4 * t], s);
        return __builtin_fmaf(-128.0f * dl, xs[0] + xs[1], (dl * kTwo24) * s);
    }
};

// Q8_0: one lane per 32-value block; value = d * (int8)q.  Codes are biased
// to q + 128 (xor 0x80) so they are non-negative subnormals.
template <> struct LaneFmt<DT_Q8_0> {
    static constexpr int LPB = 1, NG = 1, RUN = 32, NRUN = 1, NRAW = 9;
    __device__ static int run_start(int, int) { return 0; }
    __device__ static int group_of(int) { return 0; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) {
        uint32_t q[8];
        load_bytes2<8>(blk + 2, q);
        raw[8] = ld32_at(blk);
#pragma unroll
        for (int k = 0; k < 8; k++) raw[k] = q[k];
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int, const float (&xv)[32],
                                const float (&xs)[NG]) {
        const float d = h2f(raw[8] & 0xFFFF);
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const uint32_t u = raw[t] ^ 0x80808080u;
            const float *x = &xv[4 * t];
            s0 = mix2(u & 0x00FF00FFu, x[0], x[2], s0);
            s1 = mix2((u >> 8) & 0x00FF00FFu, x[1], x[3], s1);
        }
        const float a = (d * kTwo24) * (s0 + s1);
        return __builtin_fmaf(-128.0f * d, xs[0], a);
    }
};


// --------------------------------------------------------------- WaveFmt ----
// The independent-wave view used by the decode GEMV: one lane owns 64
// consecutive-in-block weights of a row (two LaneFmt pieces that share their
// scales), so a wave covers a whole "step" of 4096 values (Q4_K / Q6_K: 16
// blocks; Q4_0 / Q8_0: 128 blocks) and a row of K <= 4096 needs no other
// wave.  xv[0..63] are the lane's activations in run order.
template <int DT> struct WaveFmt;

template <> struct WaveFmt<DT_Q4_K> {
    // lane slot jp = lane % 4 of block lane / 4: qs bytes [32jp, 32jp+32) =
    // sub-block 2jp (low nibbles, values 64jp + 0..31) and 2jp+1 (high
    // nibbles, values 64jp + 32..63)
    static constexpr int LPB = 4, BPS = 16, NG = 2, RUN = 64, NRUN = 1, NRAW = 12;
    __device__ static int blk_of(int lane) { return lane >> 2; }
    __device__ static int slot_of(int lane) { return lane & 3; }
    __device__ static int run_start(int jp, int) { return 64 * jp; }
    __device__ static int group_of(int i) { return i >> 5; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int jp) {
        const u32x4 h = ld128(blk);
        const u32x4 a = ld128(blk + 16 + 32 * jp);
        const u32x4 b = ld128(blk + 32 + 32 * jp);
        raw[0] = h.x; raw[1] = h.y; raw[2] = h.z; raw[3] = h.w;
        raw[4] = a.x; raw[5] = a.y; raw[6] = a.z; raw[7] = a.w;
        raw[8] = b.x; raw[9] = b.y; raw[10] = b.z; raw[11] = b.w;
    }
    // Partial sums: acc[0..1] low nibbles (even / odd dwords), acc[2..3]
    // high nibbles -- four independent chains per row.
    static constexpr int NACC = 4;
    __device__ static void accum(const uint32_t (&raw)[NRAW], int t, const float (&xv)[64],
                                 float (&acc)[NACC]) {
        const int e = t & 1;
        nib8(raw[4 + t], &xv[4 * t], &xv[32 + 4 * t], acc[e], acc[2 + e]);
    }
    static constexpr int NDW = 8;  // dwords of codes per lane
    __device__ static float finish(const uint32_t (&raw)[NRAW], int jp, const float (&acc)[NACC],
                                   const float (&xs)[NG]) {
        const float d = h2f(raw[0] & 0xFFFF), dmin = h2f(raw[0] >> 16);
        // sub-blocks 2jp, 2jp+1 (get_scale_min_k4, quant.cpp:427-435), no branches
        const uint32_t sh = 16u * static_cast<uint32_t>(jp & 1);
        const uint32_t Y = raw[1] >> sh, Z = raw[2] >> sh, W = raw[3] >> sh;
        const bool hi = jp >= 2;
        const uint32_t A = hi ? W : Y, Am = hi ? (W >> 4) : Z, s2 = hi ? 2u : 0u;
        const uint32_t sa = (A & 15u) | ((Y >> s2) & 0x30u);
        const uint32_t sb = ((A >> 8) & 15u) | ((Y >> (8u + s2)) & 0x30u);
        const uint32_t ma = (Am & 15u) | ((Z >> s2) & 0x30u);
        const uint32_t mb = ((Am >> 8) & 15u) | ((Z >> (8u + s2)) & 0x30u);
        float a = (d * static_cast<float>(sa) * kTwo24) * (acc[0] + acc[1]);
        a = __builtin_fmaf(d * static_cast<float>(sb) * kTwo20, acc[2] + acc[3], a);
        a = __builtin_fmaf(-dmin * static_cast<float>(ma), xs[0], a);
        return __builtin_fmaf(-dmin * static_cast<float>(mb), xs[1], a);
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int jp, const float (&xv)[64],
                                const float (&xs)[NG]) {
        float acc[NACC] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < NDW; t++) accum(raw, t, xv, acc);
        return finish(raw, jp, acc, xs);
    }
};

template <> struct WaveFmt<DT_Q5_K> {
    // lane slot jp = lane % 4 of block lane / 4: qs bytes [32jp, 32jp+32)
    // (block offset 48) and all 32 qh bytes, bits 2jp (low nibbles,
    // sub-block 2jp, values 64jp + 0..31) and 2jp+1 (high nibbles, values
    // 64jp + 32..63)
    static constexpr int LPB = 4, BPS = 16, NG = 2, RUN = 64, NRUN = 1, NRAW = 20;
    __device__ static int blk_of(int lane) { return lane >> 2; }
    __device__ static int slot_of(int lane) { return lane & 3; }
    __device__ static int run_start(int jp, int) { return 64 * jp; }
    __device__ static int group_of(int i) { return i >> 5; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int jp) {
        const u32x4 h = ld128(blk);
        const u32x4 h0 = ld128(blk + 16), h1 = ld128(blk + 32);
        const u32x4 a = ld128(blk + 48 + 32 * jp);
        const u32x4 b = ld128(blk + 64 + 32 * jp);
        raw[0] = h.x; raw[1] = h.y; raw[2] = h.z; raw[3] = h.w;
        raw[4] = a.x; raw[5] = a.y; raw[6] = a.z; raw[7] = a.w;
        raw[8] = b.x; raw[9] = b.y; raw[10] = b.z; raw[11] = b.w;
        raw[12] = h0.x; raw[13] = h0.y; raw[14] = h0.z; raw[15] = h0.w;
        raw[16] = h1.x; raw[17] = h1.y; raw[18] = h1.z; raw[19] = h1.w;
    }
    // acc[0..1] low-nibble codes (even / odd dwords), acc[2..3] high
    static constexpr int NACC = 4;
    __device__ static void accum(const uint32_t (&raw)[NRAW], int t, int jp, const float *xl, const float *xh,
                                 float (&acc)[NACC]) {
        const int e = t & 1;
        acc[e] = q5x4(raw[4 + t], raw[12 + t], 0, 2 * jp, xl, acc[e]);
        acc[2 + e] = q5x4(raw[4 + t], raw[12 + t], 4, 2 * jp + 1, xh, acc[2 + e]);
    }
    static constexpr int NDW = 8;  // dwords of codes per lane
    __device__ static float finish(const uint32_t (&raw)[NRAW], int jp, const float (&acc)[NACC],
                                   const float (&xs)[NG]) {
        const float d = h2f(raw[0] & 0xFFFF), dmin = h2f(raw[0] >> 16);
        uint32_t sa, sb, ma, mb;
        q4k_pair_scale_bytes(raw, jp, sa, sb, ma, mb);
        float a = (d * static_cast<float>(sa) * kTwo24) * (acc[0] + acc[1]);
        a = __builtin_fmaf(d * static_cast<float>(sb) * kTwo24, acc[2] + acc[3], a);
        a = __builtin_fmaf(-dmin * static_cast<float>(ma), xs[0], a);
        return __builtin_fmaf(-dmin * static_cast<float>(mb), xs[1], a);
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int jp, const float (&xv)[64],
                                const float (&xs)[NG]) {
        float acc[NACC] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < NDW; t++) accum(raw, t, jp, &xv[4 * t], &xv[32 + 4 * t], acc);
        return finish(raw, jp, acc, xs);
    }
};

template <> struct WaveFmt<DT_Q6_K> {
    // lane slot jp: half h = jp/2, l0 = 16 (jp & 1): values 128h + 32qd + l0 + t,
    // qd = 0..3, t = 0..15 (four runs of 16); scales sc[8h + (jp&1) + 2qd]
    static constexpr int LPB = 4, BPS = 16, NG = 4, RUN = 16, NRUN = 4, NRAW = 15;
    __device__ static int blk_of(int lane) { return lane >> 2; }
    __device__ static int slot_of(int lane) { return lane & 3; }
    __device__ static int run_start(int jp, int r) { return 128 * (jp >> 1) + 32 * r + 16 * (jp & 1); }
    __device__ static int group_of(int i) { return i >> 4; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int jp) {
        const int h = jp >> 1, l0 = 16 * (jp & 1);
        uint32_t a[4], b[4], q[4], s[2];
        load_bytes2<4>(blk + 64 * h + l0, a);
        load_bytes2<4>(blk + 64 * h + 32 + l0, b);
        load_bytes2<4>(blk + 128 + 32 * h + l0, q);
        load_bytes2<2>(blk + 192 + 8 * h, s);
        raw[14] = ld32_at(blk + 208);
#pragma unroll
        for (int k = 0; k < 4; k++) { raw[k] = a[k]; raw[4 + k] = b[k]; raw[8 + k] = q[k]; }
        raw[12] = s[0]; raw[13] = s[1];
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int jp, const float (&xv)[64],
                                const float (&xs)[NG]) {
        const float d = h2f(raw[14] & 0xFFFF);
        float sq[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t A = raw[t], B = raw[4 + t], H = raw[8 + t];
            const uint32_t q[4] = {(A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u),
                                   (B & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u),
                                   ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u),
                                   ((B >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u)};
#pragma unroll
            for (int qd = 0; qd < 4; qd++) {
                const float *x = &xv[16 * qd + 4 * t];
                sq[qd] = mix2(q[qd] & 0x003F003Fu, x[0], x[2], sq[qd]);
                sq[qd] = mix2((q[qd] >> 8) & 0x003F003Fu, x[1], x[3], sq[qd]);
            }
        }
        // scale bytes (jp&1) + {0,2} in raw[12], (jp&1) + {4,6} in raw[13]
        const uint32_t sel = 8u * static_cast<uint32_t>(jp & 1);
        const uint32_t w0 = raw[12] >> sel, w1 = raw[13] >> sel;
        const int sc[4] = {static_cast<int8_t>(w0 & 0xFF), static_cast<int8_t>((w0 >> 16) & 0xFF),
                           static_cast<int8_t>(w1 & 0xFF), static_cast<int8_t>((w1 >> 16) & 0xFF)};
        float a = 0.0f;
#pragma unroll
        for (int qd = 0; qd < 4; qd++) {
            const float ds = d * static_cast<float>(sc[qd]);
            a = __builtin_fmaf(ds * kTwo24, sq[qd], a);
            a = __builtin_fmaf(-32.0f * ds, xs[qd], a);
        }
        return a;
    }
};

// Q2_K / Q3_K wave view, as Q6_K's: slot jp, half h = jp / 2, s = jp % 2,
// values 128h + 32j + 16s + t (plane j = run, t = 0..15), code bytes
// 32h + 16s .. +16
template <> struct WaveFmt<DT_Q2_K> {
    static constexpr int LPB = 4, BPS = 16, NG = 4, RUN = 16, NRUN = 4, NRAW = 7;
    __device__ static int blk_of(int lane) { return lane >> 2; }
    __device__ static int slot_of(int lane) { return lane & 3; }
    __device__ static int run_start(int jp, int r) { return 128 * (jp >> 1) + 32 * r + 16 * (jp & 1); }
    __device__ static int group_of(int i) { return i >> 4; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int jp) {
        const int h = jp >> 1, s = jp & 1;
        const u32x4 q = ld128(blk + 16 + 32 * h + 16 * s);
        const u32x2 sc = ld64(blk + 8 * h);
        raw[0] = q.x; raw[1] = q.y; raw[2] = q.z; raw[3] = q.w;
        raw[4] = sc.x; raw[5] = sc.y; raw[6] = ld32(blk + 80);
    }
    __device__ static void plane_sums(const uint32_t (&raw)[NRAW], const float (&xv)[64], float (&sq)[4]) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float a = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t q = plane2(raw[t], j);
                const float *x = &xv[16 * j + 4 * t];
                a = mix2(q & 0x00030003u, x[0], x[2], a);
                a = mix2((q >> 8) & 0x00030003u, x[1], x[3], a);
            }
            sq[j] = a;
        }
    }
    __device__ static float fold(const uint32_t (&raw)[NRAW], int jp, const float (&sq)[4], const float (&xs)[NG]) {
        const float d = h2f(raw[6] & 0xFFFF), dmin = h2f(raw[6] >> 16);
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t sc = byte_of(raw[4], raw[5], 2 * j + (jp & 1));
            a = __builtin_fmaf(d * static_cast<float>(sc & 0xF) * kTwo24, sq[j], a);
            a = __builtin_fmaf(-(dmin * static_cast<float>(sc >> 4)), xs[j], a);
        }
        return a;
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int jp, const float (&xv)[64],
                                const float (&xs)[NG]) {
        float sq[4];
        plane_sums(raw, xv, sq);
        return fold(raw, jp, sq, xs);
    }
};

template <> struct WaveFmt<DT_Q3_K> {
    static constexpr int LPB = 4, BPS = 16, NG = 4, RUN = 16, NRUN = 4, NRAW = 12;
    __device__ static int blk_of(int lane) { return lane >> 2; }
    __device__ static int slot_of(int lane) { return lane & 3; }
    __device__ static int run_start(int jp, int r) { return 128 * (jp >> 1) + 32 * r + 16 * (jp & 1); }
    __device__ static int group_of(int i) { return i >> 4; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int jp) {
        const int h = jp >> 1, s = jp & 1;
        uint32_t q[4], m[4], sc[3];
        load_bytes2<4>(blk + 32 + 32 * h + 16 * s, q);
        load_bytes2<4>(blk + 16 * s, m);
        load_bytes2<3>(blk + 96, sc);
#pragma unroll
        for (int k = 0; k < 4; k++) { raw[k] = q[k]; raw[4 + k] = m[k]; }
        raw[8] = sc[0]; raw[9] = sc[1]; raw[10] = sc[2];
        raw[11] = q3k_d_word(blk);
    }
    __device__ static void plane_sums(const uint32_t (&raw)[NRAW], int jp, const float (&xv)[64], float (&sq)[4]) {
        const int h = jp >> 1;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float a = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const uint32_t q = plane3(raw[t] >> (2 * j), raw[4 + t], 4 * h + j);
                const float *x = &xv[16 * j + 4 * t];
                a = mix2(q & 0x00070007u, x[0], x[2], a);
                a = mix2((q >> 8) & 0x00070007u, x[1], x[3], a);
            }
            sq[j] = a;
        }
    }
    __device__ static float fold(const uint32_t (&raw)[NRAW], int jp, const float (&sq)[4], const float (&xs)[NG]) {
        const float d = h2f(raw[11] & 0xFFFF);
        const int h = jp >> 1;
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float dl = d * static_cast<float>(q3k_scale_w(raw[8], raw[9], raw[10], h, 2 * j + (jp & 1)) - 32);
            a = __builtin_fmaf(dl * kTwo24, sq[j], a);
            a = __builtin_fmaf(-4.0f * dl, xs[j], a);
        }
        return a;
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int jp, const float (&xv)[64],
                                const float (&xs)[NG]) {
        float sq[4];
        plane_sums(raw, jp, xv, sq);
        return fold(raw, jp, sq, xs);
    }
};

template <> struct WaveFmt<DT_Q4_0> {
    // lane owns blocks 2*lane, 2*lane+1 of the step: 64 contiguous values
    static constexpr int LPB = 1, BPS = 128, NG = 2, RUN = 64, NRUN = 1, NRAW = 10;
    __device__ static int blk_of(int lane) { return 2 * lane; }
    __device__ static int slot_of(int) { return 0; }
    __device__ static int run_start(int, int) { return 0; }
    __device__ static int group_of(int i) { return i >> 5; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const uint8_t *b = blk + 18 * u;
            uint32_t q[4];
            load_bytes2<4>(b + 2, q);
            raw[5 * u + 4] = ld32_at(b);
#pragma unroll
            for (int k = 0; k < 4; k++) raw[5 * u + k] = q[k];
        }
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int, const float (&xv)[64],
                                const float (&xs)[NG]) {
        float a = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const float d = h2f(raw[5 * u + 4] & 0xFFFF);
            float sl = 0.0f, shi = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++)
                nib8(raw[5 * u + t], &xv[32 * u + 4 * t], &xv[32 * u + 16 + 4 * t], sl, shi);
            a = __builtin_fmaf(d * kTwo24, sl, a);
            a = __builtin_fmaf(d * kTwo20, shi, a);
            a = __builtin_fmaf(-8.0f * d, xs[u], a);
        }
        return a;
    }
};

template <> struct WaveFmt<DT_IQ4_NL> {
    // lane owns blocks 2*lane, 2*lane+1 of the step: 64 contiguous values
    static constexpr int LPB = 1, BPS = 128, NG = 2, RUN = 64, NRUN = 1, NRAW = 10;
    __device__ static int blk_of(int lane) { return 2 * lane; }
    __device__ static int slot_of(int) { return 0; }
    __device__ static int run_start(int, int) { return 0; }
    __device__ static int group_of(int i) { return i >> 5; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int p) {
        WaveFmt<DT_Q4_0>::load(raw, blk, p);
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int, const float (&xv)[64],
                                const float (&xs)[NG]) {
        float a = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const float d = h2f(raw[5 * u + 4] & 0xFFFF);
            float s = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++) s = iq4x8(raw[5 * u + t], &xv[32 * u + 4 * t], &xv[32 * u + 16 + 4 * t], s);
            a = __builtin_fmaf(d * kTwo24, s, a);
            a = __builtin_fmaf(-128.0f * d, xs[u], a);
        }
        return a;
    }
};

template <> struct WaveFmt<DT_MXFP4> {
    // lane owns blocks 2*lane, 2*lane+1 of the step: 64 contiguous values
    static constexpr int LPB = 1, BPS = 128, NG = 2, RUN = 64, NRUN = 1, NRAW = 10;
    __device__ static int blk_of(int lane) { return 2 * lane; }
    __device__ static int slot_of(int) { return 0; }
    __device__ static int run_start(int, int) { return 0; }
    __device__ static int group_of(int i) { return i >> 5; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            uint32_t q[4];
            load_bytes2<4>(blk + 17 * u + 1, q);
#pragma unroll
            for (int k = 0; k < 4; k++) raw[5 * u + k] = q[k];
            raw[5 * u + 4] = byte_at(blk + 17 * u);
        }
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int, const float (&xv)[64],
                                const float (&xs)[NG]) {
        float a = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const float d = e8m0_half(raw[5 * u + 4]);
            float s = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++)
                s = iq4x8<true>(raw[5 * u + t], &xv[32 * u + 4 * t], &xv[32 * u + 16 + 4 * t], s);
            a = __builtin_fmaf(d * kTwo24, s, a);
            a = __builtin_fmaf(-12.0f * d, xs[u], a);
        }
        return a;
    }
};

template <int DT> struct WaveFmtL32 {
    // lane owns blocks 2*lane, 2*lane+1 of the step: 64 contiguous values
    static constexpr int LPB = 1, BPS = 128, NG = 2, RUN = 64, NRUN = 1, NRAW = 12;
    __device__ static int blk_of(int lane) { return 2 * lane; }
    __device__ static int slot_of(int) { return 0; }
    __device__ static int run_start(int, int) { return 0; }
    __device__ static int group_of(int i) { return i >> 5; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) {
        load_l32<DT>(blk, &raw[0]);
        load_l32<DT>(blk + L32<DT>::BB, &raw[6]);
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int, const float (&xv)[64],
                                const float (&xs)[NG]) {
        float a = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++)
            a = l32_fold<DT>(&raw[6 * u], l32_sum<DT>(&raw[6 * u], &xv[32 * u], &xv[32 * u + 16], 0.0f), xs[u], a);
        return a;
    }
};
template <> struct WaveFmt<DT_Q4_1> : WaveFmtL32<DT_Q4_1> {};
template <> struct WaveFmt<DT_Q5_0> : WaveFmtL32<DT_Q5_0> {};
template <> struct WaveFmt<DT_Q5_1> : WaveFmtL32<DT_Q5_1> {};

template <int DT> struct WaveFmtFloat {
    // lane owns pseudo-blocks 2*lane, 2*lane+1 of the step: 64 contiguous values
    static constexpr int LPB = 1, BPS = 128, NG = 1, RUN = 64, NRUN = 1, NRAW = 32;
    __device__ static int blk_of(int lane) { return 2 * lane; }
    __device__ static int slot_of(int) { return 0; }
    __device__ static int run_start(int, int) { return 0; }
    __device__ static int group_of(int) { return 0; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const u32x4 v = ld128(blk + 16 * k);
            raw[4 * k] = v.x; raw[4 * k + 1] = v.y; raw[4 * k + 2] = v.z; raw[4 * k + 3] = v.w;
        }
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int, const float (&xv)[64], const float (&)[NG]) {
        float a = 0.0f, b = 0.0f;
#pragma unroll
        for (int k = 0; k < 32; k += 2) {
            a = LaneFmtFloat<DT>::pair(raw[k], xv[2 * k], xv[2 * k + 1], a);
            b = LaneFmtFloat<DT>::pair(raw[k + 1], xv[2 * k + 2], xv[2 * k + 3], b);
        }
        return a + b;
    }
};
template <> struct WaveFmt<DT_F16> : WaveFmtFloat<DT_F16> {};
template <> struct WaveFmt<DT_BF16> : WaveFmtFloat<DT_BF16> {};

template <> struct WaveFmt<DT_IQ4_XS> {
    // lane slot jp = lane % 4 of block lane / 4: sub-blocks 2jp, 2jp+1 (index
    // bytes 8 + 32jp .. +32), 64 contiguous values
    static constexpr int LPB = 4, BPS = 16, NG = 2, RUN = 64, NRUN = 1, NRAW = 10;
    __device__ static int blk_of(int lane) { return lane >> 2; }
    __device__ static int slot_of(int lane) { return lane & 3; }
    __device__ static int run_start(int jp, int) { return 64 * jp; }
    __device__ static int group_of(int i) { return i >> 5; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int jp) {
        const u32x2 h = ld64(blk);
        const u32x4 a = ld128(blk + 8 + 32 * jp), b = ld128(blk + 24 + 32 * jp);
        raw[0] = a.x; raw[1] = a.y; raw[2] = a.z; raw[3] = a.w;
        raw[4] = b.x; raw[5] = b.y; raw[6] = b.z; raw[7] = b.w;
        raw[8] = h.x; raw[9] = h.y;
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int jp, const float (&xv)[64],
                                const float (&xs)[NG]) {
        float a = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const float dl = iq4xs_scale(raw[8], raw[9], 2 * jp + u);
            float s = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++) s = iq4x8(raw[4 * u + t], &xv[32 * u + 4 * t], &xv[32 * u + 16 + 4 * t], s);
            a = __builtin_fmaf(dl * kTwo24, s, a);
            a = __builtin_fmaf(-128.0f * dl, xs[u], a);
        }
        return a;
    }
};

template <> struct WaveFmt<DT_Q8_0> {
    static constexpr int LPB = 1, BPS = 128, NG = 2, RUN = 64, NRUN = 1, NRAW = 18;
    __device__ static int blk_of(int lane) { return 2 * lane; }
    __device__ static int slot_of(int) { return 0; }
    __device__ static int run_start(int, int) { return 0; }
    __device__ static int group_of(int i) { return i >> 5; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const uint8_t *b = blk + 34 * u;
            uint32_t q[8];
            load_bytes2<8>(b + 2, q);
            raw[9 * u + 8] = ld32_at(b);
#pragma unroll
            for (int k = 0; k < 8; k++) raw[9 * u + k] = q[k];
        }
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int, const float (&xv)[64],
                                const float (&xs)[NG]) {
        float a = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const float d = h2f(raw[9 * u + 8] & 0xFFFF);
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const uint32_t v = raw[9 * u + t] ^ 0x80808080u;
                const float *x = &xv[32 * u + 4 * t];
                s0 = mix2(v & 0x00FF00FFu, x[0], x[2], s0);
                s1 = mix2((v >> 8) & 0x00FF00FFu, x[1], x[3], s1);
            }
            a = __builtin_fmaf(d * kTwo24, s0 + s1, a);
            a = __builtin_fmaf(-128.0f * d, xs[u], a);
        }
        return a;
    }
};

// ---------------------------------------------------- generic chunk lane ----
// The GEMV view of a generic-chunk format: one lane per 32-value chunk (LPB
// lanes per block), the lane keeps its block's address and decodes its chunk
// with dequant_chunk when it is dotted; the dot is one f32 fma chain over the
// chunk's values in order.
template <int DT> struct ChunkLane {
    static constexpr int LPB = blk_vals(DT) / 32, NG = 1, RUN = 32, NRUN = 1, NRAW = 2;
    __device__ static int run_start(int p, int) { return 32 * p; }
    __device__ static int group_of(int) { return 0; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) {
        const uint64_t a = reinterpret_cast<uint64_t>(blk);
        raw[0] = static_cast<uint32_t>(a);
        raw[1] = static_cast<uint32_t>(a >> 32);
    }
    __device__ static float dot(const uint32_t (&raw)[NRAW], int p, const float (&xv)[32], const float (&)[NG]) {
        const uint8_t *blk = reinterpret_cast<const uint8_t *>(static_cast<uint64_t>(raw[0]) |
                                                               (static_cast<uint64_t>(raw[1]) << 32));
        float y[32];
        dequant_chunk<DT>(blk, p, y);
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) s = __builtin_fmaf(y[i], xv[i], s);
        return s;
    }
};
#define KRK_CHUNK_LANE(D) template <> struct LaneFmt<D> : ChunkLane<D> {};
KRK_CHUNK_FORMATS(KRK_CHUNK_LANE)
#undef KRK_CHUNK_LANE

}  // namespace krk
