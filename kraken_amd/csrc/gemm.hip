// gemm.hip -- prefill GEMM for rows > 8: out[M, N] = X[M, K] . deq(W)[N, K]^T
// on gfx950 MFMA.  Replaces the reference's gemm_wmma_kernel / gemm_simt_kernel
// / gemm_reduce_kernel (src/hip/kernels/gemm.hpp:286-1140) and the int8 rung
// gemm_dp4a_kernel (src/hip/kernels/gemm_dp4a.hpp:161-610).
//
// f16 path (KRK_PATH_MFMA):
//   * workgroup tile 256 (M) x 256 (N), K consumed 32 values (one GGUF chunk)
//     per step; 8 waves, each a 128 x 64 sub-tile of 4 x 2
//     v_mfma_f32_32x32x16_f16 accumulators (128 f32 registers per lane);
//   * every step the workgroup decodes its 256 weight rows x 32 values with
//     the host oracle's arithmetic (bit-identical f32), rounds them to f16
//     into LDS, and stages the activation tile (f16, or f32 rounded to f16)
//     beside it; rows padded to 80 B so the b128 fragment reads are
//     bank-conflict free;
//   * the two wave groups run out of phase (ping-pong): one group's MFMAs
//     overlap the other group's decode and LDS stores, and each thread
//     fetches the raw bytes of the step after next (two register sets) while
//     the other group computes;
//   * tiles are ordered XCD-first: workgroup g runs on XCD g % 8, so the
//     launch order is remapped to give each XCD a contiguous run of tiles,
//     M fastest, so that the workgroups an XCD runs together share a few
//     weight tiles in its own L2;
//   * split-K (z dimension) when the tile count cannot fill 256 CUs: two
//     splits summed inside the GEMM by the one that arrives second (per-tile
//     counters), more splits as f32 partials summed in a fixed order by a
//     second kernel.
//
// int8 path (KRK_PATH_INT8, Q8_0 weights only): activations quantized per 32
// with the host rule (quantize_q8_32_d), v_mfma_i32_32x32x32_i8 per 32-value
// block, and the block fold acc = fma((f32)isum, d_w * d_x, acc) of
// dot_q8_0_q8_scalar (src/quant.cpp:3261-3279).
#include <type_traits>

#include "krk_formats.hpp"
#include "krk_kernels.hpp"
#include "krk_mi355x.h"

namespace krk {

constexpr int GB_M = 256, GB_N = 256, GB_K = 64;
constexpr int G_THREADS = 512;
constexpr int LDS_ROW = 72;  // halves per LDS row: 64 + 8 pad (144 B)

// ------------------------------------------------- weight half-chunk staging
// Thread view: 16 consecutive values of one weight row, values
// [32*kt + 16*hf, +16) of the row.  Raw bytes are fetched in fetch() and
// decoded to f16 in decode(); the f32 intermediate equals the host decoder's.
template <int DT> struct WStage;

template <> struct WStage<DT_Q4_K> {
    uint32_t hdr[4], q[4];
    __device__ void fetch(const uint8_t *row, int kt, int hf) {
        const int blk = kt >> 3, c = kt & 7;
        const uint8_t *b = row + blk * 144;
        const u32x4 h = ld128(b);
        hdr[0] = h.x; hdr[1] = h.y; hdr[2] = h.z; hdr[3] = h.w;
        const u32x4 v = ld128(b + 16 + 32 * (c >> 1) + 16 * hf);
        q[0] = v.x; q[1] = v.y; q[2] = v.z; q[3] = v.w;
    }
    __device__ void decode(int kt, _Float16 (&o)[16]) const {
        const int c = kt & 7;
        const float d = h2f(hdr[0] & 0xFFFF), dmin = h2f(hdr[0] >> 16);
        uint32_t sbytes[3] = {hdr[1], hdr[2], hdr[3]};
        auto sb = [&](int j) { return (sbytes[j >> 2] >> (8 * (j & 3))) & 0xFFu; };
        int sc, mn;
        if (c < 4) { sc = sb(c) & 63; mn = sb(c + 4) & 63; }
        else {
            sc = (sb(c + 4) & 0xF) | ((sb(c - 4) >> 6) << 4);
            mn = (sb(c + 4) >> 4) | ((sb(c) >> 6) << 4);
        }
        const float d1 = d * static_cast<float>(sc), m1 = dmin * static_cast<float>(mn);
        const int sh = (c & 1) * 4;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float qv = static_cast<float>((q[t] >> (8 * k + sh)) & 0xFu);
                o[4 * t + k] = static_cast<_Float16>(__builtin_fmaf(d1, qv, -m1));
            }
    }
};

// Q4_K by chunk pair: step p (64 values) is sub-blocks 2(p%4), 2(p%4)+1 of
// block p/4, which share the 32 code bytes (low nibbles: the even chunk,
// high nibbles: the odd one).  The thread with slice h takes code bytes
// [16h, 16h+16): values 16h .. 16h+15 of both chunks.  All lanes extract
// the same nibbles, so one mask serves four values.
struct Q4KPair {
    uint32_t hdr[4], q[4];
    __device__ void fetch(const uint8_t *row, int p, int h) {
        const uint8_t *b = row + (p >> 2) * 144;
        const u32x4 hv = ld128(b);
        hdr[0] = hv.x; hdr[1] = hv.y; hdr[2] = hv.z; hdr[3] = hv.w;
        const u32x4 v = ld128(b + 16 + 32 * (p & 3) + 16 * h);
        q[0] = v.x; q[1] = v.y; q[2] = v.z; q[3] = v.w;
    }
    // lo / hi: the slice of the even / odd chunk, f16 of the host decoder's f32
    __device__ void decode(int p, _Float16 (&lo)[16], _Float16 (&hi)[16]) const {
        const float d = h2f(hdr[0] & 0xFFFF), dmin = h2f(hdr[0] >> 16);
        // sub-blocks 2jp, 2jp+1 (get_scale_min_k4, quant.cpp:427-435), no branches
        const int jp = p & 3;
        const uint32_t sh = 16u * static_cast<uint32_t>(jp & 1);
        const uint32_t Y = hdr[1] >> sh, Z = hdr[2] >> sh, W = hdr[3] >> sh;
        const bool up = jp >= 2;
        const uint32_t A = up ? W : Y, Am = up ? (W >> 4) : Z, s2 = up ? 2u : 0u;
        const uint32_t sa = (A & 15u) | ((Y >> s2) & 0x30u);
        const uint32_t sb = ((A >> 8) & 15u) | ((Y >> (8u + s2)) & 0x30u);
        const uint32_t ma = (Am & 15u) | ((Z >> s2) & 0x30u);
        const uint32_t mb = ((Am >> 8) & 15u) | ((Z >> (8u + s2)) & 0x30u);
        const float d1a = d * static_cast<float>(sa), m1a = dmin * static_cast<float>(ma);
        const float d1b = d * static_cast<float>(sb), m1b = dmin * static_cast<float>(mb);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t l = q[t] & 0x0F0F0F0Fu, u = (q[t] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                lo[4 * t + k] = static_cast<_Float16>(
                    __builtin_fmaf(d1a, static_cast<float>((l >> (8 * k)) & 0xFFu), -m1a));
                hi[4 * t + k] = static_cast<_Float16>(
                    __builtin_fmaf(d1b, static_cast<float>((u >> (8 * k)) & 0xFFu), -m1b));
            }
        }
    }
};

template <> struct WStage<DT_Q6_K> {
    uint32_t ql[4], qh[4], sw, dw;
    __device__ void fetch(const uint8_t *row, int kt, int hf) {
        const int blk = kt >> 3, c = kt & 7, h = c >> 2, qd = c & 3;
        const uint8_t *b = row + blk * 210;
        load_bytes2<4>(b + 64 * h + 32 * (qd & 1) + 16 * hf, ql);
        load_bytes2<4>(b + 128 + 32 * h + 16 * hf, qh);
        // scale byte sc[8h + 2qd + hf] and d (bytes 208..209)
        sw = ld32_at(b + 192 + 8 * h + 2 * qd + hf);
        dw = ld32_at(b + 208);
    }
    __device__ void decode(int kt, _Float16 (&o)[16]) const {
        const int c = kt & 7, qd = c & 3;
        const float d = h2f(dw & 0xFFFF);
        const float ds = d * static_cast<float>(static_cast<int8_t>(sw & 0xFF));
        const int nsh = (qd >> 1) * 4, hsh = 2 * qd;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int qv = ((ql[t] >> (8 * k + nsh)) & 0xF) | (((qh[t] >> (8 * k + hsh)) & 3) << 4);
                o[4 * t + k] = static_cast<_Float16>(ds * static_cast<float>(qv - 32));
            }
    }
};

// Q5_K: Q4_K's staging plus the 16 high-bit bytes qh[16 hf .. +16) of the
// same positions; chunk c takes bit c of each as bit 4 of its code
// (quant.cpp:462-489).
template <> struct WStage<DT_Q5_K> {
    uint32_t hdr[4], q[4], h[4];
    __device__ void fetch(const uint8_t *row, int kt, int hf) {
        const int blk = kt >> 3, c = kt & 7;
        const uint8_t *b = row + blk * 176;
        const u32x4 hv = ld128(b);
        hdr[0] = hv.x; hdr[1] = hv.y; hdr[2] = hv.z; hdr[3] = hv.w;
        const u32x4 qv = ld128(b + 48 + 32 * (c >> 1) + 16 * hf);
        q[0] = qv.x; q[1] = qv.y; q[2] = qv.z; q[3] = qv.w;
        const u32x4 bv = ld128(b + 16 + 16 * hf);
        h[0] = bv.x; h[1] = bv.y; h[2] = bv.z; h[3] = bv.w;
    }
    __device__ void decode(int kt, _Float16 (&o)[16]) const {
        const int c = kt & 7;
        const float d = h2f(hdr[0] & 0xFFFF), dmin = h2f(hdr[0] >> 16);
        uint32_t sa, sb, ma, mb;
        q4k_pair_scale_bytes(hdr, c >> 1, sa, sb, ma, mb);
        const bool odd = c & 1;
        const float d1 = d * static_cast<float>(odd ? sb : sa), m1 = dmin * static_cast<float>(odd ? mb : ma);
        const int sh = odd ? 4 : 0;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t qv = ((q[t] >> (8 * k + sh)) & 0xFu) | (((h[t] >> (8 * k + c)) & 1u) << 4);
                o[4 * t + k] = static_cast<_Float16>(__builtin_fmaf(d1, static_cast<float>(qv), -m1));
            }
    }
};

template <> struct WStage<DT_Q8_0> {
    uint32_t q[4], dw;
    __device__ void fetch(const uint8_t *row, int kt, int hf) {
        const uint8_t *b = row + kt * 34;
        load_bytes2<4>(b + 2 + 16 * hf, q);
        dw = ld32_at(b);
    }
    __device__ void decode(int, _Float16 (&o)[16]) const {
        const float d = h2f(dw & 0xFFFF);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int k = 0; k < 4; k++)
                o[4 * t + k] = static_cast<_Float16>(
                    d * static_cast<float>(static_cast<int8_t>((q[t] >> (8 * k)) & 0xFF)));
    }
};

template <> struct WStage<DT_Q4_0> {
    uint32_t q[4], dw;
    int hf_;
    __device__ void fetch(const uint8_t *row, int kt, int hf) {
        const uint8_t *b = row + kt * 18;
        load_bytes2<4>(b + 2, q);
        dw = ld32_at(b);
        hf_ = hf;
    }
    __device__ void decode(int, _Float16 (&o)[16]) const {
        const float d = h2f(dw & 0xFFFF);
        const int sh = hf_ * 4;
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int k = 0; k < 4; k++)
                o[4 * t + k] = static_cast<_Float16>(
                    d * static_cast<float>(static_cast<int>((q[t] >> (8 * k + sh)) & 0xF) - 8));
    }
};

// IQ4_NL: Q4_0's staging, each nibble an index into the grid (value d * grid[q],
// quant.cpp:566-574), looked up four at a time
template <> struct WStage<DT_IQ4_NL> {
    uint32_t q[4], dw;
    int hf_;
    __device__ void fetch(const uint8_t *row, int kt, int hf) {
        const uint8_t *b = row + kt * 18;
        load_bytes2<4>(b + 2, q);
        dw = ld32_at(b);
        hf_ = hf;
    }
    __device__ void decode(int, _Float16 (&o)[16]) const {
        const float d = h2f(dw & 0xFFFF);
        const int sh = hf_ * 4;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t g = iq4_lookup((q[t] >> sh) & 0x0F0F0F0Fu);   // grid + 128 per byte
#pragma unroll
            for (int k = 0; k < 4; k++)
                o[4 * t + k] = static_cast<_Float16>(
                    d * static_cast<float>(static_cast<int>((g >> (8 * k)) & 0xFF) - 128));
        }
    }
};

// IQ4_XS: chunk kt is sub-block kt % 8 of block kt / 8: the 8-byte header and
// the sub-block's 16 index bytes; half hf takes the low (0) or high nibbles
template <> struct WStage<DT_IQ4_XS> {
    uint32_t q[4], h0, h1;
    int hf_;
    __device__ void fetch(const uint8_t *row, int kt, int hf) {
        const uint8_t *b = row + (kt >> 3) * 136;
        const u32x2 h = ld64(b);
        h0 = h.x;
        h1 = h.y;
        const u32x4 v = ld128(b + 8 + 16 * (kt & 7));
        q[0] = v.x; q[1] = v.y; q[2] = v.z; q[3] = v.w;
        hf_ = hf;
    }
    __device__ void decode(int kt, _Float16 (&o)[16]) const {
        const float dl = iq4xs_scale(h0, h1, kt & 7);
        const int sh = hf_ * 4;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t g = iq4_lookup((q[t] >> sh) & 0x0F0F0F0Fu);
#pragma unroll
            for (int k = 0; k < 4; k++)
                o[4 * t + k] = static_cast<_Float16>(
                    dl * static_cast<float>(static_cast<int>((g >> (8 * k)) & 0xFF) - 128));
        }
    }
};

// Q4_1 / Q5_0 / Q5_1: chunk kt is block kt; half hf takes the low (0) or
// high nibbles and qh bits 16hf + k; value d*q + m or d*(q - 16), to f16
template <int DT> struct WStageL32 {
    uint32_t raw[6];
    int hf_;
    __device__ void fetch(const uint8_t *row, int kt, int hf) {
        load_l32<DT>(row + kt * L32<DT>::BB, raw);
        hf_ = hf;
    }
    __device__ void decode(int, _Float16 (&o)[16]) const {
        const float d = h2f(raw[5] & 0xFFFF), m = h2f(raw[5] >> 16);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t c = l32_codes<DT>(raw, t, hf_);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int q = static_cast<int>((c >> (8 * k)) & 0xFF);
                const float v = L32<DT>::M ? __builtin_fmaf(d, static_cast<float>(q), m)
                                           : d * static_cast<float>(q - L32<DT>::BIAS);
                o[4 * t + k] = static_cast<_Float16>(v);
            }
        }
    }
};
template <> struct WStage<DT_Q4_1> : WStageL32<DT_Q4_1> {};
template <> struct WStage<DT_Q5_0> : WStageL32<DT_Q5_0> {};
template <> struct WStage<DT_Q5_1> : WStageL32<DT_Q5_1> {};

// F16 / BF16: chunk kt is pseudo-block kt (64 bytes); half hf its 16 values
// at 32 hf bytes, F16 as they are, BF16 rounded once to f16
template <int DT> struct WStageFloat {
    uint32_t v[8];
    __device__ void fetch(const uint8_t *row, int kt, int hf) {
        const u32x4 a = ld128(row + kt * 64 + 32 * hf), b = ld128(row + kt * 64 + 32 * hf + 16);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    __device__ void decode(int, _Float16 (&o)[16]) const {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if constexpr (DT == DT_F16) {
                const half2v h = __builtin_bit_cast(half2v, v[k]);
                o[2 * k] = h.x;
                o[2 * k + 1] = h.y;
            } else {
                o[2 * k] = static_cast<_Float16>(__builtin_bit_cast(float, v[k] << 16));
                o[2 * k + 1] = static_cast<_Float16>(__builtin_bit_cast(float, v[k] & 0xFFFF0000u));
            }
        }
    }
};
template <> struct WStage<DT_F16> : WStageFloat<DT_F16> {};
template <> struct WStage<DT_BF16> : WStageFloat<DT_BF16> {};

// MXFP4: chunk kt is block kt (byte aligned, 17 bytes); half hf takes the
// low (0) or high nibbles; value grid[q] * 2^(e - 128), rounded once to f16
template <> struct WStage<DT_MXFP4> {
    uint32_t q[4], e;
    int hf_;
    __device__ void fetch(const uint8_t *row, int kt, int hf) {
        const uint8_t *b = row + kt * 17;
        load_bytes2<4>(b + 1, q);
        e = byte_at(b);
        hf_ = hf;
    }
    __device__ void decode(int, _Float16 (&o)[16]) const {
        const float d = e8m0_half(e);
        const int sh = hf_ * 4;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const uint32_t g = fp4_lookup((q[t] >> sh) & 0x0F0F0F0Fu);   // grid + 12 per byte
#pragma unroll
            for (int k = 0; k < 4; k++)
                o[4 * t + k] = static_cast<_Float16>(
                    static_cast<float>(static_cast<int>((g >> (8 * k)) & 0xFF) - 12) * d);
        }
    }
};

// Q2_K: chunk kt = plane j of half h of block kt / 8 (c = 4h + j); half hf
// takes code bytes 32h + 16hf .. +16 and scale byte 8h + 2j + hf
template <> struct WStage<DT_Q2_K> {
    uint32_t q[4], sw, dw;
    __device__ void fetch(const uint8_t *row, int kt, int hf) {
        const int c = kt & 7, h = c >> 2, j = c & 3;
        const uint8_t *b = row + (kt >> 3) * 84;
        const u32x4 v = ld128(b + 16 + 32 * h + 16 * hf);
        q[0] = v.x; q[1] = v.y; q[2] = v.z; q[3] = v.w;
        sw = byte_at(b + 8 * h + 2 * j + hf);
        dw = ld32(b + 80);
    }
    __device__ void decode(int kt, _Float16 (&o)[16]) const {
        const int j = kt & 3;
        const float dl = h2f(dw & 0xFFFF) * static_cast<float>(sw & 0xF);
        const float ml = h2f(dw >> 16) * static_cast<float>(sw >> 4);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int k = 0; k < 4; k++)
                o[4 * t + k] = static_cast<_Float16>(
                    __builtin_fmaf(dl, static_cast<float>((q[t] >> (8 * k + 2 * j)) & 3), -ml));
    }
};

// Q3_K: as Q2_K, plus the hmask bytes 16hf .. +16 (bit 4h + j) and the
// packed 6-bit scale 8h + 2j + hf
template <> struct WStage<DT_Q3_K> {
    uint32_t q[4], m[4], lo, hi, dw;
    int hf_;
    __device__ void fetch(const uint8_t *row, int kt, int hf) {
        const int c = kt & 7, h = c >> 2, j = c & 3;
        const uint8_t *b = row + (kt >> 3) * 110;
        load_bytes2<4>(b + 32 + 32 * h + 16 * hf, q);
        load_bytes2<4>(b + 16 * hf, m);
        lo = byte_at(b + 96 + 2 * j + hf);
        hi = byte_at(b + 104 + ((2 * j + hf) & 3));
        dw = q3k_d_word(b);
        hf_ = hf;
    }
    __device__ void decode(int kt, _Float16 (&o)[16]) const {
        const int c = kt & 7, h = c >> 2, j = c & 3, i = 8 * h + 2 * j + hf_;
        const int sc = static_cast<int>(((lo >> (4 * h)) & 0xF) | (((hi >> (2 * (i >> 2))) & 3) << 4));
        const float dl = h2f(dw & 0xFFFF) * static_cast<float>(sc - 32);
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int code = static_cast<int>((q[t] >> (8 * k + 2 * j)) & 3) -
                                 (((m[t] >> (8 * k + 4 * h + j)) & 1) ? 0 : 4);
                o[4 * t + k] = static_cast<_Float16>(dl * static_cast<float>(code));
            }
    }
};

// Generic-chunk formats: the thread keeps its block's address; decode runs
// the chunk contract and takes its 16-value half.
template <int DT> struct WStageChunk {
    const uint8_t *blk;
    int c, hf;
    __device__ void fetch(const uint8_t *row, int kt, int h) {
        constexpr int CPB = blk_vals(DT) / 32;
        blk = row + static_cast<int64_t>(kt / CPB) * blk_bytes(DT);
        c = kt % CPB;
        hf = h;
    }
    __device__ void decode(int, _Float16 (&o)[16]) const {
        float y[32];
        dequant_chunk<DT>(blk, c, y);
#pragma unroll
        for (int i = 0; i < 16; i++) o[i] = static_cast<_Float16>(hf ? y[16 + i] : y[i]);
    }
};
#define KRK_CHUNK_WSTAGE(D) template <> struct WStage<D> : WStageChunk<D> {};
KRK_CHUNK_FORMATS(KRK_CHUNK_WSTAGE)
#undef KRK_CHUNK_WSTAGE

// ------------------------------------------------------- activation staging
template <typename XT> struct XStage;
template <> struct XStage<_Float16> {
    u32x4 v[2];
    __device__ void fetch(const _Float16 *p, bool ok) {
        if (ok) {
            v[0] = *reinterpret_cast<const u32x4 *>(p);
            v[1] = *reinterpret_cast<const u32x4 *>(p + 8);
        } else {
            v[0] = u32x4{0, 0, 0, 0};
            v[1] = u32x4{0, 0, 0, 0};
        }
    }
    __device__ void store(_Float16 *lds) const {
        *reinterpret_cast<u32x4 *>(lds) = v[0];
        *reinterpret_cast<u32x4 *>(lds + 8) = v[1];
    }
};
template <> struct XStage<float> {
    floatx4 v[4];
    __device__ void fetch(const float *p, bool ok) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            v[i] = ok ? *reinterpret_cast<const floatx4 *>(p + 4 * i) : floatx4{0, 0, 0, 0};
    }
    __device__ void store(_Float16 *lds) const {
        half8 a, b;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            a[i] = static_cast<_Float16>(v[0][i]);
            a[4 + i] = static_cast<_Float16>(v[1][i]);
            b[i] = static_cast<_Float16>(v[2][i]);
            b[4 + i] = static_cast<_Float16>(v[3][i]);
        }
        *reinterpret_cast<half8 *>(lds) = a;
        *reinterpret_cast<half8 *>(lds + 8) = b;
    }
};

// XCD-aware tile order: the hardware hands workgroup g to XCD g % 8.  Give
// XCD x the contiguous tile range [x*per, (x+1)*per) so its workgroups share
// operand rows in that XCD's L2.
__device__ __forceinline__ int xcd_remap(int g, int G) {
    const int per = G / 8;
    if (g >= per * 8) return g;  // tail when G is not a multiple of 8
    return (g & 7) * per + (g >> 3);
}

// Raw operand bytes of one thread for one K step (64 values): the two
// 16-value halves of its weight chunk and its 32 activations.
template <int DT, typename XT> struct StepRegs {
    WStage<DT> w0, w1;
    XStage<XT> x0, x1;
};
template <typename XT> struct StepRegs<DT_Q4_K, XT> {
    Q4KPair w;
    XStage<XT> x0, x1;
};

// Whether a (format, activation type) pair keeps two steps of raw bytes in
// registers without spilling (256 VGPRs at two waves per SIMD; measured on
// the compiled kernels: the f32-activation staging of the wider formats and
// the 16-bit-weight and Q3_K stagings do not fit).
template <int DT, typename XT> constexpr bool deep_prefetch() {
    if constexpr (std::is_same<XT, float>::value)
        return !(DT == DT_Q5_K || DT == DT_Q6_K || DT == DT_Q8_0 || DT == DT_Q3_K || DT == DT_F16 ||
                 DT == DT_BF16);
    return !(DT == DT_Q3_K || DT == DT_F16);
}

template <int DT, typename XT, typename OT>
__global__ void __launch_bounds__(G_THREADS, 1)
    gemm_f16_kernel(const uint8_t *__restrict__ w, int64_t row_bytes, const XT *__restrict__ x,
                    OT *__restrict__ out, float *__restrict__ part, unsigned *__restrict__ cnt,
                    int M, int N, int K, int k_per_split, int tiles_n) {
    // two LDS stages of a 256 x 64 activation tile and a 256 x 64 weight tile
    __shared__ _Float16 Xs[2][GB_M * LDS_ROW];
    __shared__ _Float16 Ws[2][GB_N * LDS_ROW];

    const int G = gridDim.x;
    const int g = xcd_remap(static_cast<int>(blockIdx.x), G);
    const int tiles_m = G / tiles_n;
    const int tm = g % tiles_m, tn = g / tiles_m;
    const int m0 = tm * GB_M, n0 = tn * GB_N;
    const int kb = static_cast<int>(blockIdx.z) * k_per_split;
    const int ke = min(K, kb + k_per_split);
    const int nk = (ke - kb + GB_K - 1) / GB_K;   // a K of 32 mod 64 ends in a half step
    const int cend = ke / 32;                      // first chunk past this split

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;  // 2 x 4 waves, 128 x 64 each (wm = group)

    // Two wave groups (waves 0-3 and 4-7; each SIMD holds one wave of each)
    // run out of phase: while one group's MFMAs consume a stage, the other
    // decodes and stores its half of the next stage.  Group gp computes
    // output rows 128 gp .. +127 and stages activation rows and weight rows
    // 128 gp .. +127: thread role row = 128 gp + (tid % 256) / 2, values
    // [64 kt + 32 shf, +32) of the row (one 32-value GGUF chunk).
    const int gp = wave >> 2;
    const int srow = gp * 128 + ((tid & 255) >> 1), shf = tid & 1;
    const int wr = min(n0 + srow, N - 1);
    const uint8_t *wrow = w + static_cast<int64_t>(wr) * row_bytes;
    const bool xok = m0 + srow < M;
    const XT *xrow = x + static_cast<int64_t>(xok ? m0 + srow : 0) * K + shf * 32;
    const int c0 = kb / 32 + shf;  // chunk index of step 0

    auto fetch = [&](StepRegs<DT, XT> &r, int it) {
        const int c = c0 + 2 * it;
        const bool ok = c < cend;
        const int cc = ok ? c : cend - 1;          // stay inside the row
        if constexpr (DT == DT_Q4_K) {
            const int pp = c >> 1;                  // chunk pair of this step
            r.w.fetch(wrow, 2 * pp < cend ? pp : (cend - 1) >> 1, shf);
        } else {
            r.w0.fetch(wrow, cc, 0);
            r.w1.fetch(wrow, cc, 1);
        }
        const XT *xp = xrow + kb + (ok ? it * GB_K : 0);
        r.x0.fetch(xp, xok && ok);
        r.x1.fetch(xp + 16, xok && ok);
    };
    auto stage = [&](const StepRegs<DT, XT> &r, int it, int s) {
        const int c = c0 + 2 * it;
        _Float16 a[16], b[16];
        // a, b: the two 16-value runs this thread stores, at wo and wo + 16
        // (Q4_K: slice shf of the even chunk at 16 shf, of the odd at 32 + 16 shf)
        int wo = shf * 32, bo = shf * 32 + 16;
        if constexpr (DT == DT_Q4_K) {
            const int pp = c >> 1;
            r.w.decode(pp, a, b);
            if (2 * pp + 1 >= cend) {   // the half step past K: zero the odd chunk
#pragma unroll
                for (int i = 0; i < 16; i++) b[i] = static_cast<_Float16>(0.0f);
            }
            wo = 16 * shf;
            bo = 32 + 16 * shf;
        } else {
            r.w0.decode(c, a);
            r.w1.decode(c, b);
            if (c >= cend) {   // the half step past K: zero weights (the activations are zero too)
#pragma unroll
                for (int i = 0; i < 16; i++) { a[i] = static_cast<_Float16>(0.0f); b[i] = a[i]; }
            }
        }
        _Float16 *wd = &Ws[s][srow * LDS_ROW + wo];
        _Float16 *wb = &Ws[s][srow * LDS_ROW + bo];
        half8 h;
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = a[i];
        *reinterpret_cast<half8 *>(wd) = h;
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = a[8 + i];
        *reinterpret_cast<half8 *>(wd + 8) = h;
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = b[i];
        *reinterpret_cast<half8 *>(wb) = h;
#pragma unroll
        for (int i = 0; i < 8; i++) h[i] = b[8 + i];
        *reinterpret_cast<half8 *>(wb + 8) = h;
        r.x0.store(&Xs[s][srow * LDS_ROW + shf * 32]);
        r.x1.store(&Xs[s][srow * LDS_ROW + shf * 32 + 16]);
    };

    floatx16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    auto mfma_step = [&](int s) {
#pragma unroll
        for (int kk = 0; kk < GB_K; kk += 16) {
            half8 af[4], bf[2];
            const int ko = kk + (lane >> 5) * 8;
#pragma unroll
            for (int i = 0; i < 4; i++)
                af[i] = *reinterpret_cast<const half8 *>(&Xs[s][(wm * 128 + i * 32 + (lane & 31)) * LDS_ROW + ko]);
#pragma unroll
            for (int j = 0; j < 2; j++)
                bf[j] = *reinterpret_cast<const half8 *>(&Ws[s][(wn * 64 + j * 32 + (lane & 31)) * LDS_ROW + ko]);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    // Pipeline (phases separated by workgroup barriers):
    //   group 0:  C0 | M1 | C1 | M2 | C2 | ...
    //   group 1:  M1 | C0 | M2 | C1 | M3 | ...
    // Ct = MFMAs over stage t % 2, Mt = decode and store this group's half
    // of step t into stage t % 2, then fetch step t + 1's raw bytes.  A stage
    // is complete one phase before either group reads it, and rewritten only
    // after both groups have read it.  Both groups pass 2 nk barriers.
    // Raw bytes are double-buffered in registers where the budget allows
    // (deep_prefetch): group gp keeps step s in set (s + gp) % 2 (ra = 0,
    // rb = 1), and a step's bytes are requested right after the step two
    // earlier was staged from the same set, so each load has a full step
    // (two phases) to land.  In loop iteration t both groups stage from set
    // (t + 1) % 2, so unrolling the loop by two makes every set choice static
    // (no register arrays indexed at run time).  Otherwise one set: a step's
    // bytes are requested after the previous step was staged.
    constexpr bool DEEP = deep_prefetch<DT, XT>();
    StepRegs<DT, XT> ra;
    std::conditional_t<DEEP, StepRegs<DT, XT>, StepRegs<DT, XT> &> rb = ra;
    constexpr int DIST = DEEP ? 2 : 1;
    auto stage_fetch = [&](StepRegs<DT, XT> &r, int ms) {
        stage(r, ms, ms & 1);
        if (ms + DIST < nk) fetch(r, ms + DIST);
    };
    if (nk > 0) {
        if (DEEP && gp == 1) {
            fetch(rb, 0);
            if (nk > 1) fetch(ra, 1);
            stage_fetch(rb, 0);
        } else {
            fetch(ra, 0);
            if (DEEP && nk > 1) fetch(rb, 1);
            stage_fetch(ra, 0);
        }
    }
    __syncthreads();
    if (gp == 1) {
        if (1 < nk) stage_fetch(ra, 1);
        __syncthreads();
    }
    auto iter = [&](StepRegs<DT, XT> &r, int t) {
        __builtin_amdgcn_s_setprio(1);
        mfma_step(t & 1);
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
        const int ms = t + 1 + gp;
        if (ms < nk) stage_fetch(r, ms);
        if (t + 1 < nk || gp == 0) __syncthreads();
    };
    for (int t = 0; t < nk; t += 2) {
        iter(rb, t);
        if (t + 1 < nk) iter(ra, t + 1);
    }

    // Split-K fix-up (cnt set, two splits): each split stores its
    // accumulators as a fragment image (register-major, 256 B per wave and
    // register), waits for the stores to complete, and counts itself in the
    // tile's counter; the split that arrives second adds the other's image
    // to its registers (a + b = b + a: the result does not depend on which
    // split arrives first), writes the output and clears the counter for the
    // next call.  Images and counter go through agent-scope atomics, which
    // are coherent across the XCDs' L2s without a cache write-back or
    // invalidate.
    if (cnt) {
        __shared__ int is_last;
        const int z = static_cast<int>(blockIdx.z);
        float *img = part + static_cast<int64_t>(g) * (2 * 65536) + tid;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    __hip_atomic_store(img + (z * 128 + (i * 2 + j) * 16 + r) * 512, acc[i][j][r],
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // the image stores stay above the wait (a compiler barrier), and the
        // wait holds the count back until every store has completed
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0)
            is_last = __hip_atomic_fetch_add(cnt + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1u;
        __syncthreads();
        if (!is_last) return;
        const float *other = img + (1 - z) * 128 * 512;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    acc[i][j][r] += __hip_atomic_load(other + ((i * 2 + j) * 16 + r) * 512, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
        if (tid == 0) __hip_atomic_store(cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        part = nullptr;
    }

    // C fragment: lane holds column j = lane % 32, rows 8*(r/4) + 4*(lane/32) + r%4
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn * 64 + j * 32 + (lane & 31);
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m >= M) continue;
                const float v = acc[i][j][r];
                if (part)
                    part[(static_cast<int64_t>(blockIdx.z) * M + m) * N + n] = v;
                else
                    out[static_cast<int64_t>(m) * N + n] = static_cast<OT>(v);
            }
        }
}

// Fixed-order sum of the split-K partials: 8 consecutive outputs per thread
// (two 16-byte loads per split, one 16- or 32-byte store), the tail of MN
// not a multiple of 8 (and every output of a shape or output pointer the
// 16-byte accesses do not fit) one by one.
template <typename OT>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const float *__restrict__ part,
                                                            OT *__restrict__ out, int64_t MN,
                                                            int splits) {
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 8;
    if (i >= MN) return;
    // 16-byte accesses need every slice (z MN floats into the 256-byte
    // aligned workspace) and the output 16-byte aligned; other shapes and
    // outputs are summed value by value
    const bool vec = (MN & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    if (vec && i + 8 <= MN) {
        floatx4 a = {0.0f, 0.0f, 0.0f, 0.0f}, b = a;
        for (int z = 0; z < splits; z++) {
            const floatx4 u = *reinterpret_cast<const floatx4 *>(part + z * MN + i);
            const floatx4 v = *reinterpret_cast<const floatx4 *>(part + z * MN + i + 4);
            a += u;
            b += v;
        }
        if constexpr (sizeof(OT) == 2) {
            half8 h;
#pragma unroll
            for (int k = 0; k < 4; k++) { h[k] = static_cast<_Float16>(a[k]); h[4 + k] = static_cast<_Float16>(b[k]); }
            *reinterpret_cast<half8 *>(out + i) = h;
        } else {
            *reinterpret_cast<floatx4 *>(out + i) = a;
            *reinterpret_cast<floatx4 *>(out + i + 4) = b;
        }
        return;
    }
    for (int64_t j = i; j < (i + 8 < MN ? i + 8 : MN); j++) {
        float s = 0.0f;
        for (int z = 0; z < splits; z++) s += part[z * MN + j];
        out[j] = static_cast<OT>(s);
    }
}

static int pick_split(int64_t M, int64_t N, int64_t K, int dt) {
    const int64_t tiles = ((M + GB_M - 1) / GB_M) * ((N + GB_N - 1) / GB_N);
    const int64_t kblk = blk_vals(dt) < GB_K ? GB_K : blk_vals(dt);
    const int64_t cus = device_cus();
    // Estimated time of a split (us): rounds of resident workgroups x K per
    // split at ~0.034 us per K value and round (a 256 x 256 tile, measured),
    // plus the partials' traffic -- written and read back, 8 s M N bytes --
    // at ~4 TB/s.  Splits keep at least 1024 K in whole blocks; ties keep
    // the smaller split.
    auto cost = [&](int64_t s) {
        const double rounds = static_cast<double>((tiles * s + cus - 1) / cus);
        const double part = s > 1 ? 8.0 * static_cast<double>(s) * M * N / 4.0e6 : 0.0;
        return rounds * static_cast<double>(K / s) * 0.034 + part;
    };
    int best = 1;
    double best_cost = cost(1);
    for (int s = 2; s <= 64 && K / s >= 1024 && K % s == 0 && (K / s) % kblk == 0; s *= 2) {
        const double c = cost(s);
        if (c < best_cost) {
            best_cost = c;
            best = s;
        }
    }
    return best;
}

// Batches of up to kStreamGemmRows rows take the weight-streaming kernel of
// the grouped expert GEMM in its dense mode: the 256 x 256 tiles would be
// mostly padding, and the weights, not the MFMAs, bound these.
constexpr int64_t kStreamGemmRows = 128;
static bool stream_gemm(int dt, int64_t M, int64_t N, int64_t K) {
    return M <= kStreamGemmRows && K % 256 == 0 && N < (1LL << 31) && K < (1LL << 31) && moe_gemm_ok(dt);
}

// K ranges of a dense streaming launch: the largest divisor of the block
// count up to what brings the workgroups to one per CU (two per CU measured
// slower from 9 to 64 rows: 16 rows 17.8 -> 19.4 us up, 20.8 -> 24.6 down)
static int stream_split(int64_t M, int64_t N, int64_t K) {
    const int64_t mt = M <= 32 ? 32 : 64;
    const int64_t wgs = ((M + mt - 1) / mt) * ((N + 255) / 256);
    const int64_t want = (device_cus() + wgs - 1) / wgs;
    const int64_t nb = K / 256;
    int best = 1;
    for (int s = 1; s <= nb && s <= want; s++)
        if (nb % s == 0) best = s;
    return best;
}
static size_t al256(size_t v) { return (v + 255) & ~size_t(255); }

// Split-K scratch of the tile GEMM: the reduce kernel's slices (flat,
// s M N floats) and the two-split fix-up's fragment images (one 256 x 256
// image per tile and split; more than flat when M or N ends in a partial
// tile)
static size_t splitk_floats(int64_t M, int64_t N, int s, bool images) {
    if (s == 1) return 0;
    if (!images) return static_cast<size_t>(s) * M * N;
    const size_t tiles = static_cast<size_t>((M + GB_M - 1) / GB_M) * ((N + GB_N - 1) / GB_N);
    return tiles * s * GB_M * GB_N;
}

size_t gemm_mfma_workspace(int dt, int64_t M, int64_t N, int64_t K, bool minimal) {
    if (stream_gemm(dt, M, N, K)) {   // f32 rows as f16, and the split partials
        const int s = stream_split(M, N, K);
        return al256(static_cast<size_t>(M * K) * sizeof(_Float16)) +
               (s > 1 ? static_cast<size_t>(s) * M * N * sizeof(float) : 0);
    }
    const int s = pick_split(M, N, K, dt);
    const size_t flat = splitk_floats(M, N, s, false), imgs = splitk_floats(M, N, s, true);
    return (minimal || flat > imgs ? flat : imgs) * sizeof(float);
}

template <int DT, typename XT, typename OT>
static hipError_t launch_f16(const void *w, int64_t rb, const void *x, void *out, int64_t M,
                             int64_t N, int64_t K, void *ws, size_t ws_bytes, unsigned *cnt,
                             hipStream_t st) {
    const int tiles_m = static_cast<int>((M + GB_M - 1) / GB_M);
    const int tiles_n = static_cast<int>((N + GB_N - 1) / GB_N);
    const int s = pick_split(M, N, K, DT);
    const int kps = static_cast<int>(K / s);
    float *part = nullptr;
    if (s > 1) {
        if (ws_bytes < splitk_floats(M, N, s, false) * sizeof(float)) return hipErrorInvalidValue;
        part = static_cast<float *>(ws);
    }
    // two splits sum inside the GEMM when the caller brings tile counters
    // (zero between calls) and scratch for the images; more splits would
    // leave the serial sum of the last to arrive long, and take the reduce
    // kernel
    const bool fix = s == 2 && cnt && tiles_m * tiles_n <= kTileCounters &&
                     ws_bytes >= splitk_floats(M, N, s, true) * sizeof(float);
    dim3 grid(static_cast<unsigned>(tiles_m * tiles_n), 1, static_cast<unsigned>(s));
    hipLaunchKernelGGL((gemm_f16_kernel<DT, XT, OT>), grid, dim3(G_THREADS), 0, st,
                       static_cast<const uint8_t *>(w), rb, static_cast<const XT *>(x),
                       static_cast<OT *>(out), part, fix ? cnt : nullptr, static_cast<int>(M),
                       static_cast<int>(N), static_cast<int>(K), kps, tiles_n);
    if (s > 1 && !fix) {
        const int64_t MN = M * N;
        hipLaunchKernelGGL((splitk_reduce_kernel<OT>), dim3(static_cast<unsigned>((MN + 2047) / 2048)),
                           dim3(256), 0, st, part, static_cast<OT *>(out), MN, s);
    }
    return hipGetLastError();
}

hipError_t gemm_mfma(int dt, const void *w, int64_t row_bytes, const void *x, bool act_f16,
                     void *out, int64_t M, int64_t N, int64_t K, void *ws, size_t ws_bytes,
                     unsigned *cnt, hipStream_t st) {
    if (stream_gemm(dt, M, N, K)) {
        if (ws_bytes < gemm_mfma_workspace(dt, M, N, K, false)) return hipErrorInvalidValue;
        const int split = stream_split(M, N, K);
        float *part = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) +
                                                al256(static_cast<size_t>(M * K) * sizeof(_Float16)));
        MoeGemmArgs g{};
        g.x = x;
        if (!act_f16) {   // the rows as f16 (the operand rounding of every MFMA path)
            const hipError_t e = moe_gather_f16(static_cast<const float *>(x), K, nullptr, nullptr, M,
                                                static_cast<_Float16 *>(ws), st);
            if (e != hipSuccess) return e;
            g.x = ws;
        }
        g.w = w;
        g.ksplit = split;
        g.out = split > 1 ? static_cast<void *>(part) : out;
        g.out_f16 = act_f16;
        g.row_bytes = row_bytes;
        g.K = static_cast<int>(K);
        g.N = static_cast<int>(N);
        g.M = static_cast<int>(M);
        g.mi = M <= 32 ? 1 : 2;
        hipError_t e = moe_gemm(dt, g, st);
        if (e != hipSuccess || split == 1) return e;
        const int64_t MN = M * N;
        if (act_f16)
            hipLaunchKernelGGL((splitk_reduce_kernel<_Float16>), dim3(static_cast<unsigned>((MN + 2047) / 2048)),
                               dim3(256), 0, st, part, static_cast<_Float16 *>(out), MN, split);
        else
            hipLaunchKernelGGL((splitk_reduce_kernel<float>), dim3(static_cast<unsigned>((MN + 2047) / 2048)),
                               dim3(256), 0, st, part, static_cast<float *>(out), MN, split);
        return hipGetLastError();
    }
#define KRK_GEMM_CASE(D)                                                                       \
    case D:                                                                                   \
        return act_f16 ? launch_f16<D, _Float16, _Float16>(w, row_bytes, x, out, M, N, K, ws,  \
                                                           ws_bytes, cnt, st)                  \
                       : launch_f16<D, float, float>(w, row_bytes, x, out, M, N, K, ws,        \
                                                     ws_bytes, cnt, st);
    switch (dt) {
        KRK_GEMM_CASE(DT_Q4_K)
        KRK_GEMM_CASE(DT_Q5_K)
        KRK_GEMM_CASE(DT_Q6_K)
        KRK_GEMM_CASE(DT_Q8_0)
        KRK_GEMM_CASE(DT_Q4_0)
        KRK_GEMM_CASE(DT_IQ4_NL)
        KRK_GEMM_CASE(DT_IQ4_XS)
        KRK_GEMM_CASE(DT_Q2_K)
        KRK_GEMM_CASE(DT_Q3_K)
        KRK_GEMM_CASE(DT_MXFP4)
        KRK_GEMM_CASE(DT_Q4_1)
        KRK_GEMM_CASE(DT_Q5_0)
        KRK_GEMM_CASE(DT_Q5_1)
        KRK_GEMM_CASE(DT_F16)
        KRK_GEMM_CASE(DT_BF16)
        KRK_CHUNK_FORMATS(KRK_GEMM_CASE)
        default: return hipErrorInvalidValue;
    }
#undef KRK_GEMM_CASE
}

// ------------------------------------------------------ grouped expert GEMM
// Prefill-sized MoE batches: each plan item (one expert, up to MT = 32 MI of
// its (token, slot) pairs, activation rows gathered to f16 in plan order)
// against one N tile of that expert's bank, on v_mfma_f32_16x16x32_f16.
// The weights go from HBM straight into the MFMA B operand: each wave owns
// two 16-row column blocks (gate/up: 16 gate rows and the same 16 up rows,
// so both dots of an output land in one lane), and per 256-value block lane
// group g = lane / 16 of row j = lane % 16 takes code bytes [16 g, 16 g + 16)
// and [64 + 16 g, +16): the four groups of a row read its code bytes as two
// whole 64-byte lines.  Slice s = 4 u + 2 nib + ih of a block (8 MFMAs of 32
// values) takes, in group g, values 64 (2 u + g / 2) + 32 nib + 16 (g % 2)
// + 8 ih + e, e < 8 (u: which 64 code bytes, nib: low or high nibbles); the
// activation fragments are read from LDS at the same positions, so every
// block's sum is unchanged by the permutation.  Raw weight bytes of the
// next block are in flight while a block computes; the f16 activation rows
// are staged a block at a time in two LDS buffers, one barrier per block.
// An item holds all of an expert's pairs up to MT, so a batch reads each
// active expert's weights about once.
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));

// One lane's share of one 256-value block of one weight row.  bf[0], bf[1]:
// slices 4 u + ih and 4 u + 2 + ih.
template <int DT> struct LaneBlk {
    // value 128 u + NIB nib + gofs(g) + 8 ih + e of the block in slice
    // 4 u + 2 nib + ih of lane group g (the activation side reads the same)
    static constexpr int NIB = 32;
    static constexpr int LOADS = -1;   // vector loads per fetch: not counted
    __device__ static int gofs(int g) { return 64 * (g >> 1) + 16 * (g & 1); }
    WStage<DT> w[4];   // (u, nib) = chunk 4 u + 2 (g / 2) + nib, half g % 2
    __device__ void fetch(const uint8_t *row, int blk, int g) {
#pragma unroll
        for (int i = 0; i < 4; i++) w[i].fetch(row, 8 * blk + 4 * (i >> 1) + 2 * (g >> 1) + (i & 1), g & 1);
    }
    __device__ void decode(int blk, int g, int u, int ih, half8 (&bf)[2]) const {
#pragma unroll
        for (int nib = 0; nib < 2; nib++) {
            _Float16 o[16];
            w[2 * u + nib].decode(8 * blk + 4 * u + 2 * (g >> 1) + nib, o);
#pragma unroll
            for (int e = 0; e < 8; e++) bf[nib][e] = o[8 * ih + e];
        }
    }
};
// Q4_K: code byte pairs become the f16 pairs (1024 + q0, 1024 + q1) by one
// byte permute (0x64 is the high byte of 1024.0 in f16, where the ulp is 1),
// and each value is one mixed-precision FMA, f16(d1 (1024 + q) - c) with
// c = 1024 d1 + m1 in f32 (1024 d1 exact).
template <> struct LaneBlk<DT_Q4_K> {
    static constexpr int NIB = 32;
    static constexpr int LOADS = 3;
    __device__ static int gofs(int g) { return 64 * (g >> 1) + 16 * (g & 1); }
    uint32_t hdr[4], q[2][4];
    __device__ void fetch(const uint8_t *row, int blk, int g) {
        const uint8_t *b = row + static_cast<int64_t>(blk) * 144;
        const u32x4 hv = ldg128(b);
        hdr[0] = hv.x; hdr[1] = hv.y; hdr[2] = hv.z; hdr[3] = hv.w;
        const u32x4 v0 = ldg128(b + 16 + 16 * g), v1 = ldg128(b + 80 + 16 * g);
        q[0][0] = v0.x; q[0][1] = v0.y; q[0][2] = v0.z; q[0][3] = v0.w;
        q[1][0] = v1.x; q[1][1] = v1.y; q[1][2] = v1.z; q[1][3] = v1.w;
    }
    __device__ void decode(int, int g, int u, int ih, half8 (&bf)[2]) const {
        const float d = h2f(hdr[0] & 0xFFFF), dmin = h2f(hdr[0] >> 16);
        // sub-blocks 2 jp, 2 jp + 1 with jp = 2 u + g / 2 (get_scale_min_k4,
        // quant.cpp:427-435, as Q4KPair)
        const uint32_t sh = 16u * static_cast<uint32_t>((g >> 1) & 1);
        const uint32_t Y = hdr[1] >> sh, Z = hdr[2] >> sh, W = hdr[3] >> sh;
        const uint32_t A = u ? W : Y, Am = u ? (W >> 4) : Z, s2 = u ? 2u : 0u;
        const uint32_t sa = (A & 15u) | ((Y >> s2) & 0x30u);
        const uint32_t sb = ((A >> 8) & 15u) | ((Y >> (8u + s2)) & 0x30u);
        const uint32_t ma = (Am & 15u) | ((Z >> s2) & 0x30u);
        const uint32_t mb = ((Am >> 8) & 15u) | ((Z >> (8u + s2)) & 0x30u);
        const float d1a = d * static_cast<float>(sa), d1b = d * static_cast<float>(sb);
        const float ca = 1024.0f * d1a + dmin * static_cast<float>(ma);
        const float cb = 1024.0f * d1b + dmin * static_cast<float>(mb);
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            const uint32_t w = q[u][2 * ih + tt];
            const uint32_t l = w & 0x0F0F0F0Fu, hn = (w >> 4) & 0x0F0F0F0Fu;
            const uint32_t pr[4] = {__builtin_amdgcn_perm(0x64646464u, l, 0x04010400u),
                                    __builtin_amdgcn_perm(0x64646464u, l, 0x04030402u),
                                    __builtin_amdgcn_perm(0x64646464u, hn, 0x04010400u),
                                    __builtin_amdgcn_perm(0x64646464u, hn, 0x04030402u)};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const h16x2 hp = __builtin_bit_cast(h16x2, pr[k]);
                const float dk = k < 2 ? d1a : d1b, ck = k < 2 ? ca : cb;
                const int o = 4 * tt + 2 * (k & 1);
                bf[k >> 1][o] = static_cast<_Float16>(__builtin_fmaf(dk, static_cast<float>(hp[0]), -ck));
                bf[k >> 1][o + 1] = static_cast<_Float16>(__builtin_fmaf(dk, static_cast<float>(hp[1]), -ck));
            }
        }
    }
};

// Q6_K (210-byte blocks, 2-byte aligned rows): in half u of the block,
// lane group g takes ql bytes [64 u + 16 g, +16) -- the four groups read
// the half's 64 ql bytes as one line -- and the qh bytes of the same
// positions l = 16 (g % 2) + i: low nibbles are quadrant g / 2 (values
// 128 u + 16 g + i), high nibbles quadrant 2 + g / 2 (values + 64), with
// scales sc[8 u + g] and sc[8 u + 4 + g].  Values are
// f16(ds (1024 + q) - 1056 ds), ds = d sc (the host's (d sc) (q - 32)).
template <> struct LaneBlk<DT_Q6_K> {
    static constexpr int NIB = 64;
    static constexpr int LOADS = 6;
    __device__ static int gofs(int g) { return 16 * g; }
    uint32_t ql[2][4], qh[2][4], sc[4], dw;
    __device__ void fetch(const uint8_t *row, int blk, int g) {
        gbyte *b = to_global(row + static_cast<int64_t>(blk) * 210);
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const u32x4 l = ld128_a2(b + 64 * u + 16 * g), h = ld128_a2(b + 128 + 32 * u + 16 * (g & 1));
            ql[u][0] = l.x; ql[u][1] = l.y; ql[u][2] = l.z; ql[u][3] = l.w;
            qh[u][0] = h.x; qh[u][1] = h.y; qh[u][2] = h.z; qh[u][3] = h.w;
        }
        const u32x4 s = ld128_a2(b + 192);
        sc[0] = s.x; sc[1] = s.y; sc[2] = s.z; sc[3] = s.w;
        dw = ld16g(b + 208);
    }
    __device__ void decode(int, int g, int u, int ih, half8 (&bf)[2]) const {
        const float d = h2f(dw);
        // scale bytes 8 u + g and 8 u + 4 + g: dwords 2 u and 2 u + 1, byte g
        const int sa = static_cast<int8_t>((sc[2 * u] >> (8 * g)) & 0xFFu);
        const int sb = static_cast<int8_t>((sc[2 * u + 1] >> (8 * g)) & 0xFFu);
        const float da = d * static_cast<float>(sa), db = d * static_cast<float>(sb);
        const float ca = 1056.0f * da, cb = 1056.0f * db;
        const uint32_t s0 = 2u * static_cast<uint32_t>(g >> 1);
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            const uint32_t lw = ql[u][2 * ih + tt], hw = qh[u][2 * ih + tt];
            const uint32_t lo = (lw & 0x0F0F0F0Fu) | (((hw >> s0) & 0x03030303u) << 4);
            const uint32_t hi = ((lw >> 4) & 0x0F0F0F0Fu) | (((hw >> (s0 + 4u)) & 0x03030303u) << 4);
            const uint32_t pr[4] = {__builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u),
                                    __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u),
                                    __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u),
                                    __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u)};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const h16x2 hp = __builtin_bit_cast(h16x2, pr[k]);
                const float dk = k < 2 ? da : db, ck = k < 2 ? ca : cb;
                const int o = 4 * tt + 2 * (k & 1);
                bf[k >> 1][o] = static_cast<_Float16>(__builtin_fmaf(dk, static_cast<float>(hp[0]), -ck));
                bf[k >> 1][o + 1] = static_cast<_Float16>(__builtin_fmaf(dk, static_cast<float>(hp[1]), -ck));
            }
        }
    }
};

constexpr int MG_THREADS = 512;

// s_waitcnt vmcnt(N) alone (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt[5:4] << 14)
template <int N> __device__ __forceinline__ void mg_wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int DT, bool GU, int MI>
__global__ void __launch_bounds__(MG_THREADS) __attribute__((amdgpu_waves_per_eu(DT == DT_Q4_K || (DT == DT_Q6_K && MI == 1) ? 4 : 2)))
    moe_gemm_kernel(MoeGemmArgs a, int ntiles) {
    constexpr int MT = 32 * MI;        // item rows
    constexpr int MB = 2 * MI;         // 16-row M blocks
    constexpr int NI = MT / 16;        // activation DMA instructions per wave and block
    // two buffers of MT rows x 256 halves; 16-byte chunk c of row r at slot
    // c ^ (r % 16), so the 16 rows a fragment read touches at one chunk hit
    // distinct bank groups
    __shared__ __attribute__((aligned(1024))) _Float16 Xs[2][MT * 256];

    // blockIdx -> (item, N tile): the hardware gives workgroup g to XCD
    // g % 8, so every N tile of an item runs on one XCD (its activation rows
    // stay in that L2) and the items, empty ones included, are dealt evenly
    // over the XCDs.
    // Dense mode: every N tile's row items run on one XCD (they share its
    // weights in that L2).
    const int gi = static_cast<int>(blockIdx.x), slot = gi >> 3;
    const bool dense = !GU && a.w != nullptr;
    int item, nt, pb, rows, ks = 0;
    const krk_moe_entry *en = nullptr;
    if (dense) {
        // slot -> (item fastest, N tile group, K range)
        const int nit = (a.M + MT - 1) / MT, ntg = (ntiles + 7) / 8;
        item = slot % nit;
        nt = (gi & 7) + 8 * ((slot / nit) % ntg);
        ks = (slot / nit) / ntg;
        if (nt >= ntiles) return;
        pb = item * MT;
        rows = a.M - pb < MT ? a.M - pb : MT;
    } else {
        item = (gi & 7) + 8 * (slot / ntiles);
        nt = slot % ntiles;
        if (item >= *a.n_items) return;
        const int32_t *it = a.items + 4 * item;
        pb = it[1];
        rows = it[2];
        en = static_cast<const krk_moe_entry *>(a.tab) + it[0];
    }

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, g = lane >> 4;
    int row[2];
    const uint8_t *wrow[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const uint8_t *wb;
        if constexpr (GU) {
            row[c] = nt * 128 + wave * 16 + j;
            wb = static_cast<const uint8_t *>(en->p[c == 0 ? KRK_MOE_GATE : KRK_MOE_UP]);
        } else {
            row[c] = nt * 256 + wave * 32 + 16 * c + j;
            wb = dense ? static_cast<const uint8_t *>(a.w) : static_cast<const uint8_t *>(en->p[KRK_MOE_DOWN]);
        }
        wrow[c] = wb + static_cast<int64_t>(row[c] < a.N ? row[c] : a.N - 1) * a.row_bytes;
    }
    // a dense launch's K range: its blocks start kb0 blocks into every row
    const int nblk = a.K / 256 / (dense ? a.ksplit : 1);
    const int64_t kb0 = static_cast<int64_t>(ks) * nblk;
    if (ks) {
        const int64_t bb = a.row_bytes / (a.K / 256);   // bytes per 256 values
#pragma unroll
        for (int c = 0; c < 2; c++) wrow[c] += kb0 * bb;
    }

    // activation rows by LDS DMA (global_load_lds, 16 bytes a lane): wave
    // w's instruction i fills rows 2 (NI w + i) + lane / 32, slots lane % 32
    // (rows past the item re-read its first row; their outputs are dropped)
    gbyte *dsrc[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int r = 2 * (NI * wave + i) + (lane >> 5);
        const int c = (lane & 31) ^ (r & 15);
        const int pr = pb + (r < rows ? r : 0);
        const int64_t xr = a.xtok ? static_cast<int64_t>(a.xtok[pr]) : pr;
        dsrc[i] = to_global(reinterpret_cast<const uint8_t *>(static_cast<const _Float16 *>(a.x) + xr * a.K +
                                                              256 * kb0 + 8 * c));
    }
    auto xdma = [&](int blk, int buf) {
#pragma unroll
        for (int i = 0; i < NI; i++)
            __builtin_amdgcn_global_load_lds(
                (const __attribute__((address_space(1))) void *)(dsrc[i] + 512 * static_cast<int64_t>(blk)),
                (__attribute__((address_space(3))) void *)(&Xs[buf][(2 * (NI * wave + i)) * 256]), 16, 0, 0);
    };
    // this wave's DMA of a block has landed once at most the `later` vector
    // loads issued after it are outstanding (in-order completion); then a
    // bare barrier (__syncthreads would also wait for the weight prefetch)
    auto publish = [&](bool fetched) {
        constexpr int L = LaneBlk<DT>::LOADS;
        if (L > 0 && fetched) mg_wait_vm<2 * (L > 0 ? L : 0)>();
        else mg_wait_vm<0>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    // A fragment of (u, nib, ih) for lane (j, g): row j of an M block, chunk
    // 16 u + (NIB / 8) nib + ih + gofs(g) / 8 (disjoint bits), swizzled
    const int cd = LaneBlk<DT>::gofs(g) >> 3;
    auto a_off = [&](int u, int nib, int ih) {
        const int c = 16 * u + (LaneBlk<DT>::NIB / 8) * nib + ih + cd;
        return j * 256 + ((c ^ j) << 3);
    };

    floatx4 acc[MB][2];
#pragma unroll
    for (int i = 0; i < MB; i++)
#pragma unroll
        for (int c = 0; c < 2; c++) acc[i][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    // Q4_K keeps two blocks of raw bytes in registers (the next block's
    // requests are issued a whole block before it is decoded); the wider
    // formats keep one (requested right after the block before is decoded).
    constexpr bool DEEP = DT == DT_Q4_K && MI == 1;
    struct Set { LaneBlk<DT> r[2]; };
    auto block = [&](Set &ws, int blk) {
        LaneBlk<DT>(&wr)[2] = ws.r;
        const bool next = blk + 1 < nblk;
        if (next) xdma(blk + 1, (blk + 1) & 1);
        const _Float16 *xb = Xs[blk & 1];
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int ih = 0; ih < 2; ih++) {
                half8 bf[2][2];
                wr[0].decode(blk, g, u, ih, bf[0]);
                wr[1].decode(blk, g, u, ih, bf[1]);
                if (!DEEP && u == 1 && ih == 1 && next) {
                    wr[0].fetch(wrow[0], blk + 1, g);
                    wr[1].fetch(wrow[1], blk + 1, g);
                }
#pragma unroll
                for (int nib = 0; nib < 2; nib++)
#pragma unroll
                    for (int mb = 0; mb < MB; mb++) {
                        if (mb > 0 && 16 * mb >= rows) break;   // M blocks past the item: no work
                        const half8 af = *reinterpret_cast<const half8 *>(xb + mb * 16 * 256 + a_off(u, nib, ih));
#pragma unroll
                        for (int c = 0; c < 2; c++)
                            acc[mb][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[c][nib], acc[mb][c], 0, 0, 0);
                    }
            }
        const bool deep_fetch = DEEP && blk + 2 < nblk;
        if (deep_fetch) {
            wr[0].fetch(wrow[0], blk + 2, g);
            wr[1].fetch(wrow[1], blk + 2, g);
        }
        if (next) publish(deep_fetch || !DEEP);
    };

    Set ra;
    std::conditional_t<DEEP, Set, Set &> rb = ra;
    xdma(0, 0);
    ra.r[0].fetch(wrow[0], 0, g);
    ra.r[1].fetch(wrow[1], 0, g);
    if (DEEP && nblk > 1) {
        rb.r[0].fetch(wrow[0], 1, g);
        rb.r[1].fetch(wrow[1], 1, g);
    }
    publish(true);
    for (int blk = 0; blk < nblk; blk += 2) {
        block(ra, blk);
        if (blk + 1 < nblk) block(rb, blk + 1);
    }

    // C fragment (16 x 16): lane holds column j, rows 4 g .. 4 g + 3 of each
    // M block
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = mb * 16 + 4 * g + r;
            if (m >= rows) continue;
            if constexpr (GU) {
                if (row[0] < a.N) {
                    const float gt = acc[mb][0][r], up = acc[mb][1][r];
                    static_cast<_Float16 *>(a.out)[static_cast<int64_t>(pb + m) * a.N + row[0]] =
                        static_cast<_Float16>((gt / (1.0f + expf(-gt))) * up);
                }
            } else {
#pragma unroll
                for (int c = 0; c < 2; c++)
                    if (row[c] < a.N) {
                        const int64_t o = static_cast<int64_t>(pb + m) * a.N + row[c];
                        if (a.ksplit > 1)   // (dense) this K range's f32 partial
                            static_cast<float *>(a.out)[static_cast<int64_t>(ks) * a.M * a.N + o] = acc[mb][c][r];
                        else if (a.out_f16)
                            static_cast<_Float16 *>(a.out)[o] = static_cast<_Float16>(acc[mb][c][r]);
                        else
                            static_cast<float *>(a.out)[o] = acc[mb][c][r];
                    }
            }
        }
}

// Activation rows as f16 (the GEMM's operand rounding): row pos =
// x[plan_tok[pos]] for the live plan positions, or without plan_tok row pos
// = x[pos] (the tokens' rows, or a dense GEMM's).
__global__ void __launch_bounds__(256) moe_gather_f16_kernel(const float *__restrict__ x, int64_t n,
                                                              const int32_t *__restrict__ plan_tok,
                                                              const int32_t *__restrict__ n_live,
                                                              _Float16 *__restrict__ xg) {
    const int64_t pos = blockIdx.x;
    if (n_live && pos >= *n_live) return;
    const float *src = x + (plan_tok ? static_cast<int64_t>(plan_tok[pos]) : pos) * n;
    _Float16 *dst = xg + pos * n;
    for (int64_t i = 8 * static_cast<int64_t>(threadIdx.x); i < n; i += 8 * 256) {
        const floatx4 v0 = *reinterpret_cast<const floatx4 *>(src + i);
        const floatx4 v1 = *reinterpret_cast<const floatx4 *>(src + i + 4);
        half8 h;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            h[k] = static_cast<_Float16>(v0[k]);
            h[4 + k] = static_cast<_Float16>(v1[k]);
        }
        *reinterpret_cast<half8 *>(dst + i) = h;
    }
}

hipError_t moe_gather_f16(const float *x, int64_t n, const int32_t *plan_tok, const int32_t *n_live,
                          int64_t max_rows, _Float16 *xg, hipStream_t st) {
    if (n % 8 || max_rows <= 0 || max_rows > (1LL << 31) - 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(moe_gather_f16_kernel, dim3(static_cast<unsigned>(max_rows)), dim3(256), 0, st, x, n,
                       plan_tok, n_live, xg);
    return hipGetLastError();
}

#define KRK_MOE_GEMM_TYPES(X) X(DT_Q4_K) X(DT_Q5_K) X(DT_Q6_K) X(DT_Q8_0) X(DT_Q4_0) X(DT_MXFP4)

bool moe_gemm_ok(int dt) {
    switch (dt) {
#define KRK_MG_OK(D) case D:
        KRK_MOE_GEMM_TYPES(KRK_MG_OK)
#undef KRK_MG_OK
        return true;
        default: return false;
    }
}

template <int DT, bool GU>
static hipError_t launch_moe_gemm(const MoeGemmArgs &a, hipStream_t st) {
    if (a.K % 256 || a.N <= 0 ||
        (a.w ? (GU || a.M <= 0 || a.ksplit < 1 || (a.K / 256) % a.ksplit) : a.max_items <= 0))
        return hipErrorInvalidValue;
    const int ntiles = (a.N + (GU ? 127 : 255)) / (GU ? 128 : 256);
    const int64_t blocks = a.w ? 8LL * ((a.M + 32 * a.mi - 1) / (32 * a.mi)) * ((ntiles + 7) / 8) * a.ksplit
                               : 8LL * ntiles * ((a.max_items + 7) / 8);
    if (blocks > (1LL << 31) - 1) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(blocks));
    switch (a.mi) {
        case 1: hipLaunchKernelGGL((moe_gemm_kernel<DT, GU, 1>), grid, dim3(MG_THREADS), 0, st, a, ntiles); break;
        case 2: hipLaunchKernelGGL((moe_gemm_kernel<DT, GU, 2>), grid, dim3(MG_THREADS), 0, st, a, ntiles); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t moe_gemm(int dt, const MoeGemmArgs &a, hipStream_t st) {
    switch (dt) {
#define KRK_MG_CASE(D) \
    case D: return a.gate_up ? launch_moe_gemm<D, true>(a, st) : launch_moe_gemm<D, false>(a, st);
        KRK_MOE_GEMM_TYPES(KRK_MG_CASE)
#undef KRK_MG_CASE
        default: return hipErrorInvalidValue;
    }
}

}  // namespace krk
