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
__host__ __device__ constexpr int blk_vals(int dt) {
    return dt == DT_Q4_K || dt == DT_Q6_K ? 256 : (dt == DT_Q4_0 || dt == DT_Q8_0) ? 32 : 1;
}
__host__ __device__ constexpr int blk_bytes(int dt) {
    return dt == DT_Q4_K ? 144 : dt == DT_Q6_K ? 210 : dt == DT_Q4_0 ? 18
         : dt == DT_Q8_0 ? 34 : dt == DT_F16 ? 2 : 4;
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

// ----------------------------------------------------- aligned raw loads ----
// NW dwords holding bytes [p, p + 4*NW) of a 2-byte aligned pointer.  Only
// dwords overlapping that range are read; a 4-aligned dword never crosses a
// page, so a block's bytes can be fetched without reading past the buffer.
template <int NW>
__device__ __forceinline__ void load_bytes2(const uint8_t *p, uint32_t (&o)[NW]) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint8_t *base = reinterpret_cast<const uint8_t *>(a & ~uintptr_t(3));
    const uint32_t s = static_cast<uint32_t>(a & 3);
    uint32_t d[NW + 1];
#pragma unroll
    for (int k = 0; k < NW; k++) d[k] = ld32(base + 4 * k);
    d[NW] = s ? ld32(base + 4 * NW) : 0u;
#pragma unroll
    for (int k = 0; k < NW; k++) o[k] = align_bytes(d[k + 1], d[k], s);
}

// --------------------------------------------------------------- LaneFmt ----
// The lane view: LPB lanes per block, each owning 32 values ("a piece"), NG
// groups sharing one (scale, off) pair.  pos(p, i) is the position inside the
// block of the piece's i-th value; runs(p, r) the start of its r-th run of
// RUN consecutive values (the x loads).
template <int DT> struct LaneFmt;

// Q4_K: piece p covers qs bytes [16p, 16p+16): sub-block 2j low nibbles
// (values 64j + 16(p&1) + i) and sub-block 2j+1 high nibbles, j = p/2.
template <> struct LaneFmt<DT_Q4_K> {
    static constexpr int LPB = 8, NG = 2, RUN = 16, NRUN = 2, NRAW = 8;
    __device__ static int run_start(int p, int r) { return 64 * (p >> 1) + 32 * r + 16 * (p & 1); }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int p) {
        const u32x4 h = ld128(blk);
        const u32x4 q = ld128(blk + 16 + 16 * p);
        raw[0] = h.x; raw[1] = h.y; raw[2] = h.z; raw[3] = h.w;
        raw[4] = q.x; raw[5] = q.y; raw[6] = q.z; raw[7] = q.w;
    }
    // wq[i]: i < 16 -> q (low nibble), i >= 16 -> 16*q (high nibble, masked in place)
    __device__ static void decode(const uint32_t (&raw)[NRAW], int p, float (&wq)[32],
                                  float (&sc)[NG], float (&off)[NG]) {
        const float d = h2f(raw[0] & 0xFFFF), dmin = h2f(raw[0] >> 16);
        const uint32_t sh = 16u * static_cast<uint32_t>((p >> 1) & 1);  // j & 1
        const uint32_t Y = raw[1] >> sh, Z = raw[2] >> sh, W = raw[3] >> sh;
        int sa, sb, ma, mb;
        if (p < 4) {  // sub-blocks 0..3: 6-bit fields stored directly
            sa = Y & 63; sb = (Y >> 8) & 63; ma = Z & 63; mb = (Z >> 8) & 63;
        } else {      // sub-blocks 4..7: low 4 bits in scales[8..11], top 2 in the high bits
            sa = (W & 0xF) | (((Y >> 6) & 3) << 4);
            sb = ((W >> 8) & 0xF) | (((Y >> 14) & 3) << 4);
            ma = ((W >> 4) & 0xF) | (((Z >> 6) & 3) << 4);
            mb = ((W >> 12) & 0xF) | (((Z >> 14) & 3) << 4);
        }
        sc[0] = d * static_cast<float>(sa);
        off[0] = dmin * static_cast<float>(ma);
        sc[1] = d * static_cast<float>(sb) * 0.0625f;
        off[1] = dmin * static_cast<float>(mb);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t lo = raw[4 + t] & 0x0F0F0F0Fu, hi = raw[4 + t] & 0xF0F0F0F0u;
            wq[4 * t + 0] = ubyte_f<0>(lo); wq[4 * t + 1] = ubyte_f<1>(lo);
            wq[4 * t + 2] = ubyte_f<2>(lo); wq[4 * t + 3] = ubyte_f<3>(lo);
            wq[16 + 4 * t + 0] = ubyte_f<0>(hi); wq[16 + 4 * t + 1] = ubyte_f<1>(hi);
            wq[16 + 4 * t + 2] = ubyte_f<2>(hi); wq[16 + 4 * t + 3] = ubyte_f<3>(hi);
        }
    }
    __device__ static int group_of(int i) { return i >> 4; }
};

// Q6_K: piece p = (half h = p/4, sub = p%4): values 128h + 32qd + 8sub + t for
// quadrant qd (0..3) and t (0..7).  Needs ql[64h+8sub..+8], ql[64h+32+8sub..+8],
// qh[32h+8sub..+8], scales sc[8h + sub/2 + 2qd] and d.
template <> struct LaneFmt<DT_Q6_K> {
    static constexpr int LPB = 8, NG = 4, RUN = 8, NRUN = 4, NRAW = 9;
    __device__ static int run_start(int p, int r) { return 128 * (p >> 2) + 32 * r + 8 * (p & 3); }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int p) {
        const int h = p >> 2, o = 8 * (p & 3);
        uint32_t a[2], b[2], q[2], s[2], dd[1];
        load_bytes2<2>(blk + 64 * h + o, a);
        load_bytes2<2>(blk + 64 * h + 32 + o, b);
        load_bytes2<2>(blk + 128 + 32 * h + o, q);
        load_bytes2<2>(blk + 192 + 8 * h, s);
        // d is the last two bytes of the block; read the dword that holds them
        // without touching anything past the block.
        const uintptr_t da = reinterpret_cast<uintptr_t>(blk + 208);
        dd[0] = ld32(reinterpret_cast<const uint8_t *>(da & ~uintptr_t(3))) >> (8 * (da & 3));
        raw[0] = a[0]; raw[1] = a[1]; raw[2] = b[0]; raw[3] = b[1];
        raw[4] = q[0]; raw[5] = q[1]; raw[6] = s[0]; raw[7] = s[1]; raw[8] = dd[0];
    }
    // wq = q6 code in [0, 63]; value = (d*sc) * (q - 32).
    __device__ static void decode(const uint32_t (&raw)[NRAW], int p, float (&wq)[32],
                                  float (&sc)[NG], float (&off)[NG]) {
        const float d = h2f(raw[8] & 0xFFFF);
        const uint32_t sub2 = static_cast<uint32_t>((p & 3) >> 1);
#pragma unroll
        for (int qd = 0; qd < 4; qd++) {
            const int idx = static_cast<int>(sub2) + 2 * qd;  // byte in the 8 scale bytes
            const uint32_t sw = idx < 4 ? raw[6] : raw[7];
            const int s8 = static_cast<int32_t>(sw << (24 - 8 * (idx & 3))) >> 24;
            const float ds = d * static_cast<float>(s8);
            sc[qd] = ds;
            off[qd] = 32.0f * ds;
        }
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const uint32_t A = raw[t], B = raw[2 + t], H = raw[4 + t];
            const uint32_t q0 = (A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
            const uint32_t q1 = (B & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
            const uint32_t q2 = ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u);
            const uint32_t q3 = ((B >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
            const uint32_t qq[4] = {q0, q1, q2, q3};
#pragma unroll
            for (int qd = 0; qd < 4; qd++) {
                wq[8 * qd + 4 * t + 0] = ubyte_f<0>(qq[qd]);
                wq[8 * qd + 4 * t + 1] = ubyte_f<1>(qq[qd]);
                wq[8 * qd + 4 * t + 2] = ubyte_f<2>(qq[qd]);
                wq[8 * qd + 4 * t + 3] = ubyte_f<3>(qq[qd]);
            }
        }
    }
    __device__ static int group_of(int i) { return i >> 3; }
};

// Q4_0: one lane per 32-value block.  Low nibbles are values 0..15, high
// nibbles 16..31; value = d * (q - 8).
template <> struct LaneFmt<DT_Q4_0> {
    static constexpr int LPB = 1, NG = 2, RUN = 32, NRUN = 1, NRAW = 5;
    __device__ static int run_start(int, int) { return 0; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) {
        uint32_t q[4];
        load_bytes2<4>(blk + 2, q);
        const uintptr_t da = reinterpret_cast<uintptr_t>(blk);
        raw[4] = ld32(reinterpret_cast<const uint8_t *>(da & ~uintptr_t(3))) >> (8 * (da & 3));
        raw[0] = q[0]; raw[1] = q[1]; raw[2] = q[2]; raw[3] = q[3];
    }
    __device__ static void decode(const uint32_t (&raw)[NRAW], int, float (&wq)[32],
                                  float (&sc)[NG], float (&off)[NG]) {
        const float d = h2f(raw[4] & 0xFFFF);
        sc[0] = d; off[0] = 8.0f * d;
        sc[1] = d * 0.0625f; off[1] = 8.0f * d;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t lo = raw[t] & 0x0F0F0F0Fu, hi = raw[t] & 0xF0F0F0F0u;
            wq[4 * t + 0] = ubyte_f<0>(lo); wq[4 * t + 1] = ubyte_f<1>(lo);
            wq[4 * t + 2] = ubyte_f<2>(lo); wq[4 * t + 3] = ubyte_f<3>(lo);
            wq[16 + 4 * t + 0] = ubyte_f<0>(hi); wq[16 + 4 * t + 1] = ubyte_f<1>(hi);
            wq[16 + 4 * t + 2] = ubyte_f<2>(hi); wq[16 + 4 * t + 3] = ubyte_f<3>(hi);
        }
    }
    __device__ static int group_of(int i) { return i >> 4; }
};

// Q8_0: one lane per 32-value block; value = d * (int8)q.
template <> struct LaneFmt<DT_Q8_0> {
    static constexpr int LPB = 1, NG = 1, RUN = 32, NRUN = 1, NRAW = 9;
    __device__ static int run_start(int, int) { return 0; }
    __device__ static void load(uint32_t (&raw)[NRAW], const uint8_t *blk, int) {
        uint32_t q[8];
        load_bytes2<8>(blk + 2, q);
        const uintptr_t da = reinterpret_cast<uintptr_t>(blk);
        raw[8] = ld32(reinterpret_cast<const uint8_t *>(da & ~uintptr_t(3))) >> (8 * (da & 3));
#pragma unroll
        for (int k = 0; k < 8; k++) raw[k] = q[k];
    }
    __device__ static void decode(const uint32_t (&raw)[NRAW], int, float (&wq)[32],
                                  float (&sc)[NG], float (&off)[NG]) {
        sc[0] = h2f(raw[8] & 0xFFFF);
        off[0] = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            wq[4 * t + 0] = sbyte_f<0>(raw[t]); wq[4 * t + 1] = sbyte_f<1>(raw[t]);
            wq[4 * t + 2] = sbyte_f<2>(raw[t]); wq[4 * t + 3] = sbyte_f<3>(raw[t]);
        }
    }
    __device__ static int group_of(int) { return 0; }
};

}  // namespace krk
