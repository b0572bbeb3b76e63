// gemm_i8.hip -- the int8 rung (rows > 8, KRK_PATH_INT8): Q8_0, Q4_K, Q5_K
// and Q6_K weights x activations quantized per 32 values.
//
// The reference's int8 rung (gemm_dp4a.hpp:161-610; CPU twin
// dot_q8_0_q8_scalar, src/quant.cpp:3261-3279) quantizes every activation
// row per 32 values (quantize_q8_32_d, quant.cpp:2167-2197) and computes, per
// output, the exact integer dot of each 32-value block and folds it as
//     acc = fma((f32) isum_b, dw_b * dx_b, acc)        for b = 0, 1, ...
// The fold is the cost on MI355X: a wave64 VALU op issues in 4 cycles, so
// convert + scale product + fma per output per block (48 ops a lane per
// 32x32 block patch, ~192 cycles) outweighs the int8 MFMA (32 cycles) six to
// one and held an all-VALU fold to ~210 TOP/s.  Here two of the three ops
// move to the matrix core, and the outputs stay bit-identical:
//   - isum comes from two v_mfma_f32_32x32x16_f16 on the codes as f16: every
//     code is exact in f16, every product is exact, and every partial sum is
//     an integer below 32*127*127 < 2^24, so the f32 result is isum exactly;
//   - dw * dx comes from v_mfma_f32_32x32x1_2b_f32 (two 32x32 outer products
//     of rank one): one product plus zeros, rounded once to nearest even,
//     which is the f32 multiply, in the same 32x32 layout as the sums;
// leaving one fma per output per block on the VALU (~64 cycles a patch)
// against ~96 cycles of MFMA, in block order, so each output's fold is the
// reference's sequence of roundings.
//
// Q4_K / Q5_K fold as the reference's GPU rung does (gemm_dp4a.hpp 532-552):
// per 32-value sub-block with integer dot I, activation code sum S, weight
// scale bsc = d*s and min bmin = dmin*m,
//     acc = fma(dx * bsc, I, acc);  acc = fma(-(dx * S), bmin, acc)
// I comes from the f16 MFMA on the unsigned codes, dx * bsc from the
// outer-product MFMA, and the second term from an outer-product MFMA of
// -(dx * S) and bmin that accumulates straight into the accumulators.
// Q6_K takes its offset 32 inside the integer dot as the CPU twin does
// (t = I - 32 S, dot_q6_K_q8_d): codes are staged as q - 32 (exact in f16)
// and each 16-value half is one K = 16 MFMA, folded as
// acc = fma(dx * bsc, t, acc).  One VALU fma per output per half.
//
// Tiles: 128 x 128 outputs per 256-thread workgroup (4 waves in 2 x 2, each
// 64 x 64 = 2 x 2 patches), two Q8_0 blocks (64 values) per LDS stage, the
// next stage prefetched into registers; codes sit in LDS as f16 rows padded
// to 144 bytes so the 16-byte operand reads of 16 consecutive rows hit
// distinct banks.  Two workgroups share a CU (78 KB of LDS each).  The
// activation codes arrive as f16 from the quantizer; weight codes are
// widened at staging (xor 0x80, v_perm into 1024 + u as f16 bits, one
// packed f16 subtract).
#include "krk_formats.hpp"
#include "krk_kernels.hpp"
#include "gemv_core.hpp"

namespace krk {

namespace {

typedef float floatx32 __attribute__((ext_vector_type(32)));

constexpr int TM = 128, TN = 128, LS = 72;  // f16 LDS row: 64 codes + 8 pad

__device__ __forceinline__ int xcd_map(int g, int G) {
    // consecutive tiles land on one XCD (and its L2)
    const int per = G / 8;
    if (g >= per * 8) return g;
    return (g & 7) * per + (g >> 3);
}

// four int8 codes -> four exact f16 values (two dwords, code order kept)
__device__ __forceinline__ void widen_i8x4(uint32_t w, uint32_t &lo, uint32_t &hi) {
    const uint32_t u = w ^ 0x80808080u;  // biased 0..255
    const half2v off = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - off);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - off);
}

// four Q6_K codes q (0..63) -> the four exact f16 values q - 32: bytes
// q + 96 (no carries) in the low byte of 1024 + u, less 1152
__device__ __forceinline__ void widen_q6x4(uint32_t c, uint32_t &lo, uint32_t &hi) {
    const uint32_t u = c + 0x60606060u;
    const half2v off = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - off);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - off);
}

// four code bytes (unsigned 0..63) -> four exact f16 values (two dwords)
__device__ __forceinline__ void widen_u8x4(uint32_t c, uint32_t &lo, uint32_t &hi) {
    const half2v off = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, c, 0x04010400u)) - off);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, c, 0x04030402u)) - off);
}

// get_scale_min_k4 (quant.cpp:427-435) of sub-block j from the 12 scale
// bytes held in header dwords h1..h3 (bytes 4..15 of the block)
__device__ __forceinline__ void kq_scale_min(uint32_t h1, uint32_t h2, uint32_t h3, int j, uint32_t &sc,
                                             uint32_t &mn) {
    const uint32_t q[3] = {h1, h2, h3};
    auto byte = [&](int i) { return (q[i >> 2] >> (8 * (i & 3))) & 0xFFu; };
    if (j < 4) {
        sc = byte(j) & 63;
        mn = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
        mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// One 32-value block's weight codes (as 8 dwords of bytes), scales and mins
// for staging, per weight type.  bb is the row's 32-value block index.
template <int WT> struct I8W;
template <> struct I8W<DT_Q8_0> {
    static constexpr int G = 1;
    uint32_t q[8];
    float bsc;
    __device__ void fetch(const uint8_t *row, int bb) {
        const uint8_t *blk = row + static_cast<int64_t>(bb) * 34;
        load_bytes2<8>(blk + 2, q);
        bsc = h2f(static_cast<uint32_t>(*reinterpret_cast<const uint16_t *>(blk)));
    }
    __device__ void widen(uint32_t (&hv)[16]) const {
#pragma unroll
        for (int k = 0; k < 8; k++) widen_i8x4(q[k], hv[2 * k], hv[2 * k + 1]);
    }
    __device__ float scale(int) const { return bsc; }
    __device__ float minv(int) const { return 0.0f; }
};
template <int WT> struct I8WK45 {
    // Q4_K (Q5_K): sub-block b32 of block bb / 8; codes the nibble b32 & 1 of
    // the 32 bytes at 16 (48) + 32 (b32 / 2), plus (Q5_K) bit b32 of qh[l]
    static constexpr int G = 1;
    uint32_t q[8];
    float bsc, bmin;
    __device__ void fetch(const uint8_t *row, int bb) {
        constexpr int BB = WT == DT_Q4_K ? 144 : 176, QS = WT == DT_Q4_K ? 16 : 48;
        const uint8_t *blk = row + static_cast<int64_t>(bb >> 3) * BB;
        const int b32 = bb & 7;
        const u32x4 hdr = ld128(blk);
        const u32x4 c0 = ld128(blk + QS + 32 * (b32 >> 1)), c1 = ld128(blk + QS + 32 * (b32 >> 1) + 16);
        const uint32_t raw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        const int sh = 4 * (b32 & 1);
#pragma unroll
        for (int k = 0; k < 8; k++) q[k] = (raw[k] >> sh) & 0x0F0F0F0Fu;
        if constexpr (WT == DT_Q5_K) {
            const u32x4 h0 = ld128(blk + 16), h1 = ld128(blk + 32);
            const uint32_t qh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
            for (int k = 0; k < 8; k++) q[k] |= ((qh[k] >> b32) & 0x01010101u) << 4;
        }
        uint32_t sc, mn;
        kq_scale_min(hdr.y, hdr.z, hdr.w, b32, sc, mn);
        bsc = h2f(hdr.x & 0xFFFF) * static_cast<float>(sc);
        bmin = h2f(hdr.x >> 16) * static_cast<float>(mn);
    }
    __device__ void widen(uint32_t (&hv)[16]) const {
#pragma unroll
        for (int k = 0; k < 8; k++) widen_u8x4(q[k], hv[2 * k], hv[2 * k + 1]);
    }
    __device__ float scale(int) const { return bsc; }
    __device__ float minv(int) const { return bmin; }
};
template <> struct I8W<DT_Q4_K> : I8WK45<DT_Q4_K> {};
template <> struct I8W<DT_Q5_K> : I8WK45<DT_Q5_K> {};
template <> struct I8W<DT_Q6_K> {
    // 32 values 32 b32 .. of block bb / 8: half n = b32 / 4, quadrant
    // qd = b32 % 4; low 4 bits the nibble qd / 2 of ql[64n + 32 (qd & 1) + l],
    // high 2 bits bits 2qd of qh[32n + l]; scale groups sc[8n + 2qd + g].
    // Codes are staged as q - 32, so each half's MFMA dot is I - 32 S.
    static constexpr int G = 2;
    uint32_t q[8];
    float bsc[2];
    __device__ void fetch(const uint8_t *row, int bb) {
        const uint8_t *blk = row + static_cast<int64_t>(bb >> 3) * 210;
        const int b32 = bb & 7, n = b32 >> 2, qd = b32 & 3;
        uint32_t ql[8], qh[8];
        load_bytes2<8>(blk + 64 * n + 32 * (qd & 1), ql);
        load_bytes2<8>(blk + 128 + 32 * n, qh);
        const int ns = 4 * (qd >> 1), hs = 2 * qd;
#pragma unroll
        for (int k = 0; k < 8; k++) q[k] = ((ql[k] >> ns) & 0x0F0F0F0Fu) | (((qh[k] >> hs) & 0x03030303u) << 4);
        const float d = h2f((ld32_at(blk + 208)) & 0xFFFF);
#pragma unroll
        for (int g = 0; g < 2; g++)
            bsc[g] = d * static_cast<float>(static_cast<int8_t>(byte_at(blk + 192 + 8 * n + 2 * qd + g)));
    }
    __device__ void widen(uint32_t (&hv)[16]) const {
#pragma unroll
        for (int k = 0; k < 8; k++) widen_q6x4(q[k], hv[2 * k], hv[2 * k + 1]);
    }
    __device__ float scale(int g) const { return bsc[g]; }
    __device__ float minv(int) const { return 0.0f; }
};

template <int WT, typename OT>
__global__ void __launch_bounds__(256, 2) gemm_i8_kernel(const _Float16 *__restrict__ xh,
                                                         const float *__restrict__ dx,
                                                         const float *__restrict__ sx16,
                                                         const uint8_t *__restrict__ w, int64_t rb,
                                                         OT *__restrict__ out, int M, int N, int K,
                                                         int tiles_n) {
    constexpr int G = I8W<WT>::G;
    constexpr bool AFF = WT == DT_Q4_K || WT == DT_Q5_K;   // a min term to fold
    constexpr int GM = AFF ? G : 1;
    __shared__ __align__(16) _Float16 As[2][TM * LS];
    __shared__ __align__(16) _Float16 Bs[2][TN * LS];
    __shared__ float dxs[2][2][TM];
    __shared__ float nss[2][2][GM][AFF ? TM : 1];   // -(dx * S) per half (min term)
    __shared__ float bscs[2][2][G][TN];
    __shared__ float bmins[2][2][GM][AFF ? TN : 1];

    const int Gd = static_cast<int>(gridDim.x);
    const int g = xcd_map(static_cast<int>(blockIdx.x), Gd);
    // M fastest: the tiles an XCD runs together share weight tiles (a few
    // hundred KB each, kept in its L2) and stream the activations
    const int tiles_m = Gd / tiles_n;
    const int m0 = (g % tiles_m) * TM, n0 = (g / tiles_m) * TN;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = (wv >> 1) * 64, wn = (wv & 1) * 64;
    const int nb = K / 32, nst = (nb + 1) / 2;

    // staging roles: thread t stages block sh = t % 2 of the stage for
    // activation row t / 2 and weight row t / 2; rows past the matrix read
    // its last row and are never stored, a missing second block (odd nb,
    // Q8_0 only) re-reads the last block and is never used
    const int sr = tid >> 1, sh = tid & 1;
    const int am = min(m0 + sr, M - 1), bn = min(n0 + sr, N - 1);
    const _Float16 *arow = xh + static_cast<int64_t>(am) * K;
    const uint8_t *brow = w + static_cast<int64_t>(bn) * rb;
    const float *dxrow = dx + static_cast<int64_t>(am) * nb;
    const float *sxrow = AFF ? sx16 + static_cast<int64_t>(am) * (K / 16) : nullptr;   // Q4_K / Q5_K

    half8 ra[4];
    I8W<WT> rw;
    float rdx, rs[2];
    auto fetch = [&](int st) {
        const int bb = min(2 * st + sh, nb - 1);
        const half8 *ap = reinterpret_cast<const half8 *>(arow + 32 * bb);
#pragma unroll
        for (int k = 0; k < 4; k++) ra[k] = ap[k];
        rw.fetch(brow, bb);
        rdx = dxrow[bb];
        if constexpr (AFF) {
            rs[0] = sxrow[2 * bb];
            rs[1] = sxrow[2 * bb + 1];
        }
    };
    auto stash = [&](int s) {
        half8 *ad = reinterpret_cast<half8 *>(&As[s][sr * LS + 32 * sh]);
#pragma unroll
        for (int k = 0; k < 4; k++) ad[k] = ra[k];
        uint32_t hv[16];
        rw.widen(hv);
        u32x4 *bd = reinterpret_cast<u32x4 *>(&Bs[s][sr * LS + 32 * sh]);
#pragma unroll
        for (int k = 0; k < 4; k++) bd[k] = u32x4{hv[4 * k], hv[4 * k + 1], hv[4 * k + 2], hv[4 * k + 3]};
        dxs[s][sh][sr] = rdx;
#pragma unroll
        for (int h = 0; h < G; h++) {
            bscs[s][sh][h][sr] = rw.scale(h);
            if constexpr (AFF) {
                bmins[s][sh][h][sr] = rw.minv(h);
                nss[s][sh][h][sr] = -(rdx * (rs[0] + rs[1]));
            }
        }
    };

    // accumulators: acc[j] holds patches (i = 0, j) in elements 0..15 and
    // (i = 1, j) in 16..31 -- the layout of the two-block outer product
    floatx32 acc[2];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int e = 0; e < 32; e++) acc[j][e] = 0.0f;

    // MFMA operand rows: lane l supplies row l % 32, codes 8 (l / 32) .. +7 of
    // each 16-code step; C element e of lane l is row 8 (e / 4) + rsub + e % 4,
    // column l % 32
    const int orow = lane & 31, ko = 8 * (lane >> 5);
    const int rsub = 4 * (lane >> 5);
    const floatx16 z16 = {};
    const floatx32 z32 = {};

    fetch(0);
    stash(0);
    __syncthreads();
    for (int st = 0; st < nst; st++) {
        const int s = st & 1;
        if (st + 1 < nst) fetch(st + 1);
        const int nu = min(2, nb - 2 * st);
#pragma unroll
        for (int u = 0; u < 2; u++) {
            if (u >= nu) break;
            // outer-product operands: lanes 0..31 feed block 0 (patch row i = 0),
            // lanes 32..63 block 1 (i = 1); both blocks take the same columns j
            const int arow_l = wm + 32 * (lane >> 5) + orow;
            const float ax = dxs[s][u][arow_l];
            if constexpr (G == 1) {
                half8 A[2][2], B[2][2];
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        A[i][h] = *reinterpret_cast<const half8 *>(&As[s][(wm + 32 * i + orow) * LS + 32 * u + 16 * h + ko]);
                        B[i][h] = *reinterpret_cast<const half8 *>(&Bs[s][(wn + 32 * i + orow) * LS + 32 * u + 16 * h + ko]);
                    }
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int bcol = wn + 32 * j + orow;
                    const floatx32 P = __builtin_amdgcn_mfma_f32_32x32x1f32(ax, bscs[s][u][0][bcol], z32, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        floatx16 c = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[i][0], B[j][0], z16, 0, 0, 0);
                        c = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[i][1], B[j][1], c, 0, 0, 0);
#pragma unroll
                        for (int e = 0; e < 16; e++)
                            acc[j][16 * i + e] = __builtin_fmaf(c[e], P[16 * i + e], acc[j][16 * i + e]);
                    }
                    if constexpr (AFF)
                        acc[j] = __builtin_amdgcn_mfma_f32_32x32x1f32(nss[s][u][0][arow_l], bmins[s][u][0][bcol],
                                                                      acc[j], 0, 0, 0);
                }
            } else {
                // two 16-value halves, each one K = 16 MFMA, folded in order
#pragma unroll
                for (int h = 0; h < G; h++) {
                    half8 A[2], B[2];
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        A[i] = *reinterpret_cast<const half8 *>(&As[s][(wm + 32 * i + orow) * LS + 32 * u + 16 * h + ko]);
                        B[i] = *reinterpret_cast<const half8 *>(&Bs[s][(wn + 32 * i + orow) * LS + 32 * u + 16 * h + ko]);
                    }
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const int bcol = wn + 32 * j + orow;
                        const floatx32 P = __builtin_amdgcn_mfma_f32_32x32x1f32(ax, bscs[s][u][h][bcol], z32, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 2; i++) {
                            const floatx16 c = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[i], B[j], z16, 0, 0, 0);
#pragma unroll
                            for (int e = 0; e < 16; e++)
                                acc[j][16 * i + e] = __builtin_fmaf(c[e], P[16 * i + e], acc[j][16 * i + e]);
                        }
                    }
                }
            }
        }
        if (st + 1 < nst) {
            stash(s ^ 1);
            __syncthreads();
        }
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + wn + 32 * j + orow;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = m0 + wm + 32 * i + 8 * (e >> 2) + rsub + (e & 3);
                if (m < M) store_out<OT>(out + static_cast<int64_t>(m) * N + n, acc[j][16 * i + e], SEG_PLAIN, 1.0f);
            }
        }
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

template <int WT>
void launch_i8(dim3 grid, hipStream_t st, bool f16, const _Float16 *xq, const float *dx, const float *sx,
               const uint8_t *wb, int64_t rb, void *out, int M, int N, int K, int tiles_n) {
    if (f16)
        hipLaunchKernelGGL((gemm_i8_kernel<WT, _Float16>), grid, dim3(256), 0, st, xq, dx, sx, wb, rb,
                           static_cast<_Float16 *>(out), M, N, K, tiles_n);
    else
        hipLaunchKernelGGL((gemm_i8_kernel<WT, float>), grid, dim3(256), 0, st, xq, dx, sx, wb, rb,
                           static_cast<float *>(out), M, N, K, tiles_n);
}

}  // namespace

size_t gemm_int8_workspace(int64_t M, int64_t K) {
    return align256(static_cast<size_t>(M * K) * sizeof(_Float16)) +
           align256(static_cast<size_t>(M * (K / 32)) * sizeof(float)) +
           align256(static_cast<size_t>(M * (K / 16)) * sizeof(float));
}

bool gemm_int8_serves(int wt) { return wt == DT_Q8_0 || wt == DT_Q4_K || wt == DT_Q5_K || wt == DT_Q6_K; }

hipError_t gemm_int8(int wt, const void *w, int64_t row_bytes, const void *x, bool act_f16, void *out,
                     int64_t rows, int64_t n_out, int64_t n_in, void *ws, size_t ws_bytes, hipStream_t st) {
    if (!gemm_int8_serves(wt)) return hipErrorInvalidValue;
    if (n_in % 32 || rows < 1 || n_out < 1) return hipErrorInvalidValue;
    if (wt != DT_Q8_0 && n_in % 256) return hipErrorInvalidValue;
    if (ws_bytes < gemm_int8_workspace(rows, n_in)) return hipErrorInvalidValue;
    if (rows > (1 << 30) || n_out > (1 << 30) || n_in > (1 << 30)) return hipErrorInvalidValue;
    uint8_t *p = static_cast<uint8_t *>(ws);
    _Float16 *xq = reinterpret_cast<_Float16 *>(p);
    p += align256(static_cast<size_t>(rows * n_in) * sizeof(_Float16));
    float *dx = reinterpret_cast<float *>(p);
    p += align256(static_cast<size_t>(rows * (n_in / 32)) * sizeof(float));
    float *sx = wt == DT_Q8_0 ? nullptr : reinterpret_cast<float *>(p);
    hipError_t e = quantize_q8_rows_f16codes(x, act_f16, rows, n_in, xq, dx, sx, st);
    if (e != hipSuccess) return e;
    const int M = static_cast<int>(rows), N = static_cast<int>(n_out), K = static_cast<int>(n_in);
    const int tiles_m = (M + TM - 1) / TM, tiles_n = (N + TN - 1) / TN;
    const dim3 grid(static_cast<unsigned>(tiles_m * tiles_n));
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    switch (wt) {
        case DT_Q8_0: launch_i8<DT_Q8_0>(grid, st, act_f16, xq, dx, sx, wb, row_bytes, out, M, N, K, tiles_n); break;
        case DT_Q4_K: launch_i8<DT_Q4_K>(grid, st, act_f16, xq, dx, sx, wb, row_bytes, out, M, N, K, tiles_n); break;
        case DT_Q5_K: launch_i8<DT_Q5_K>(grid, st, act_f16, xq, dx, sx, wb, row_bytes, out, M, N, K, tiles_n); break;
        default: launch_i8<DT_Q6_K>(grid, st, act_f16, xq, dx, sx, wb, row_bytes, out, M, N, K, tiles_n); break;
    }
    return hipGetLastError();
}

}  // namespace krk
