// gemm_i8.hip -- the Q8_0 x Q8 int8 rung (rows > 8, KRK_PATH_INT8).
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
    // consecutive tiles (which share activation rows) land on one XCD's L2
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

template <typename OT>
__global__ void __launch_bounds__(256, 2) gemm_q8_kernel(const _Float16 *__restrict__ xh,
                                                         const float *__restrict__ dx,
                                                         const uint8_t *__restrict__ w, int64_t rb,
                                                         OT *__restrict__ out, int M, int N, int K,
                                                         int tiles_n) {
    __shared__ __align__(16) _Float16 As[2][TM * LS];
    __shared__ __align__(16) _Float16 Bs[2][TN * LS];
    __shared__ float dxs[2][2][TM];
    __shared__ float dws[2][2][TN];

    const int G = static_cast<int>(gridDim.x);
    const int g = xcd_map(static_cast<int>(blockIdx.x), G);
    const int m0 = (g / tiles_n) * TM, n0 = (g % tiles_n) * TN;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = (wv >> 1) * 64, wn = (wv & 1) * 64;
    const int nb = K / 32, nst = (nb + 1) / 2;

    // staging roles: thread t stages block sh = t % 2 of the stage for
    // activation row t / 2 and weight row t / 2; rows past the matrix read
    // its last row and are never stored, a missing second block (odd nb)
    // re-reads the last block and is never used
    const int sr = tid >> 1, sh = tid & 1;
    const int am = min(m0 + sr, M - 1), bn = min(n0 + sr, N - 1);
    const _Float16 *arow = xh + static_cast<int64_t>(am) * K;
    const uint8_t *brow = w + static_cast<int64_t>(bn) * rb;
    const float *dxrow = dx + static_cast<int64_t>(am) * nb;

    half8 ra[4];
    uint32_t rq[8];
    float rdx, rdw;
    auto fetch = [&](int st) {
        const int bb = min(2 * st + sh, nb - 1);
        const half8 *ap = reinterpret_cast<const half8 *>(arow + 32 * bb);
#pragma unroll
        for (int k = 0; k < 4; k++) ra[k] = ap[k];
        const uint8_t *blk = brow + static_cast<int64_t>(bb) * 34;
        load_bytes2<8>(blk + 2, rq);
        rdw = h2f(static_cast<uint32_t>(*reinterpret_cast<const uint16_t *>(blk)));
        rdx = dxrow[bb];
    };
    auto stash = [&](int s) {
        half8 *ad = reinterpret_cast<half8 *>(&As[s][sr * LS + 32 * sh]);
#pragma unroll
        for (int k = 0; k < 4; k++) ad[k] = ra[k];
        uint32_t hv[16];
#pragma unroll
        for (int k = 0; k < 8; k++) widen_i8x4(rq[k], hv[2 * k], hv[2 * k + 1]);
        u32x4 *bd = reinterpret_cast<u32x4 *>(&Bs[s][sr * LS + 32 * sh]);
#pragma unroll
        for (int k = 0; k < 4; k++) bd[k] = u32x4{hv[4 * k], hv[4 * k + 1], hv[4 * k + 2], hv[4 * k + 3]};
        dxs[s][sh][sr] = rdx;
        dws[s][sh][sr] = rdw;
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

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
            half8 A[2][2], B[2][2];
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    A[i][h] = *reinterpret_cast<const half8 *>(&As[s][(wm + 32 * i + orow) * LS + 32 * u + 16 * h + ko]);
                    B[i][h] = *reinterpret_cast<const half8 *>(&Bs[s][(wn + 32 * i + orow) * LS + 32 * u + 16 * h + ko]);
                }
            // outer-product operands: lanes 0..31 feed block 0 (patch row i = 0),
            // lanes 32..63 block 1 (i = 1); both blocks take the same columns j
            const float ax = dxs[s][u][wm + 32 * (lane >> 5) + orow];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const float bw = dws[s][u][wn + 32 * j + orow];
                const floatx32 P = __builtin_amdgcn_mfma_f32_32x32x1f32(ax, bw, z32, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    floatx16 c = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[i][0], B[j][0], z16, 0, 0, 0);
                    c = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[i][1], B[j][1], c, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 16; e++) acc[i][j][e] = __builtin_fmaf(c[e], P[16 * i + e], acc[i][j][e]);
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
                if (m < M) store_out<OT>(out + static_cast<int64_t>(m) * N + n, acc[i][j][e], SEG_PLAIN, 1.0f);
            }
        }
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

}  // namespace

size_t gemm_int8_workspace(int64_t M, int64_t K) {
    return align256(static_cast<size_t>(M * K) * sizeof(_Float16)) +
           align256(static_cast<size_t>(M * (K / 32)) * sizeof(float));
}

hipError_t gemm_int8_q8_0(const void *w, int64_t row_bytes, const void *x, bool act_f16, void *out,
                          int64_t rows, int64_t n_out, int64_t n_in, void *ws, size_t ws_bytes,
                          hipStream_t st) {
    if (n_in % 32 || rows < 1 || n_out < 1) return hipErrorInvalidValue;
    if (ws_bytes < gemm_int8_workspace(rows, n_in)) return hipErrorInvalidValue;
    if (rows > (1 << 30) || n_out > (1 << 30) || n_in > (1 << 30)) return hipErrorInvalidValue;
    _Float16 *xq = static_cast<_Float16 *>(ws);
    float *dx = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) +
                                          align256(static_cast<size_t>(rows * n_in) * sizeof(_Float16)));
    hipError_t e = quantize_q8_rows_f16codes(x, act_f16, rows, n_in, xq, dx, st);
    if (e != hipSuccess) return e;
    const int M = static_cast<int>(rows), N = static_cast<int>(n_out), K = static_cast<int>(n_in);
    const int tiles_m = (M + TM - 1) / TM, tiles_n = (N + TN - 1) / TN;
    const dim3 grid(static_cast<unsigned>(tiles_m * tiles_n));
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    if (act_f16)
        hipLaunchKernelGGL(gemm_q8_kernel<_Float16>, grid, dim3(256), 0, st, xq, dx, wb, row_bytes,
                           static_cast<_Float16 *>(out), M, N, K, tiles_n);
    else
        hipLaunchKernelGGL(gemm_q8_kernel<float>, grid, dim3(256), 0, st, xq, dx, wb, row_bytes,
                           static_cast<float *>(out), M, N, K, tiles_n);
    return hipGetLastError();
}

}  // namespace krk
