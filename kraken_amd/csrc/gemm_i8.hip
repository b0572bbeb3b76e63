// gemm_i8.hip -- the Q8_0 x Q8 int8 rung (rows > 8, KRK_PATH_INT8).
//
// The reference's int8 rung (gemm_dp4a.hpp:161-610; CPU twin
// dot_q8_0_q8_scalar, src/quant.cpp:3261-3279) quantizes every activation
// row per 32 values (quantize_q8_32_d, quant.cpp:2167-2197) and computes, per
// output, the exact integer dot of each 32-value block and folds it as
//     acc = fma((f32) isum_b, dw_b * dx_b, acc)        for b = 0, 1, ...
// Here the integer block dots come from v_mfma_i32_32x32x32_i8: one MFMA's K
// of 32 is exactly one Q8_0 block, so every MFMA result is a block's isum for
// a 32x32 patch of outputs, and each lane folds its 16 results in block
// order with the same fma -- the outputs equal the CPU oracle's bit for bit.
//
// Roofline: the fold is 3 VALU ops (convert, scale product, fma) per output
// per 32-value block against 32 MACs on the matrix core, so the rung is VALU
// bound at ~1/6 of the int8 peak (~0.84 POP/s on MI355X), below the f16 MFMA
// path's reach.  It exists for its semantics (the reference's lossy int8
// mode), not for speed on this part.
//
// Tiles: 128 x 128 outputs per 256-thread workgroup (4 waves in 2 x 2, each
// 64 x 64 = 2 x 2 MFMA tiles), one Q8_0 block per LDS stage, the next
// block's operands prefetched into registers.
#include "krk_formats.hpp"
#include "krk_kernels.hpp"
#include "gemv_core.hpp"

namespace krk {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int TM = 128, TN = 128;

__device__ __forceinline__ int xcd_map(int g, int G) {
    // consecutive tiles (which share activation rows) land on one XCD's L2
    const int per = G / 8;
    if (g >= per * 8) return g;
    return (g & 7) * per + (g >> 3);
}

template <typename OT>
__global__ void __launch_bounds__(256) gemm_q8_kernel(const int8_t *__restrict__ xq,
                                                      const float *__restrict__ dx,
                                                      const uint8_t *__restrict__ w, int64_t rb,
                                                      OT *__restrict__ out, int M, int N, int K,
                                                      int tiles_n) {
    __shared__ __align__(16) int8_t As[2][TM * 32];
    __shared__ __align__(16) int8_t Bs[2][TN * 32];
    __shared__ float dxs[2][TM];
    __shared__ float dws[2][TN];

    const int G = static_cast<int>(gridDim.x);
    const int g = xcd_map(static_cast<int>(blockIdx.x), G);
    const int m0 = (g / tiles_n) * TM, n0 = (g % tiles_n) * TN;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = (wv >> 1) * 64, wn = (wv & 1) * 64;
    const int nb = K / 32;

    // staging roles: thread t loads 16 activation bytes of row t/2 and 16
    // weight codes of row t/2 (half t%2 of the block); rows past the matrix
    // read its last row and are never stored
    const int sr = tid >> 1, sh = tid & 1;
    const int am = min(m0 + sr, M - 1), bn = min(n0 + sr, N - 1);
    const int8_t *arow = xq + static_cast<int64_t>(am) * K + 16 * sh;
    const uint8_t *brow = w + static_cast<int64_t>(bn) * rb;
    const float *dxrow = dx + static_cast<int64_t>(min(m0 + tid, M - 1)) * nb;

    v4i ra, rbv;
    float rdx = 0.0f, rdw = 0.0f;
    auto fetch = [&](int b) {
        ra = *reinterpret_cast<const v4i *>(arow + b * 32);
        uint32_t q[4];
        load_bytes2<4>(brow + static_cast<int64_t>(b) * 34 + 2 + 16 * sh, q);
        rbv = v4i{static_cast<int>(q[0]), static_cast<int>(q[1]), static_cast<int>(q[2]),
                  static_cast<int>(q[3])};
        if (tid < TM) rdx = dxrow[b];
        if (sh == 0) rdw = h2f(static_cast<uint32_t>(*reinterpret_cast<const uint16_t *>(
                                   brow + static_cast<int64_t>(b) * 34)));
    };
    auto stash = [&](int s) {
        *reinterpret_cast<v4i *>(&As[s][sr * 32 + 16 * sh]) = ra;
        *reinterpret_cast<v4i *>(&Bs[s][sr * 32 + 16 * sh]) = rbv;
        if (tid < TM) dxs[s][tid] = rdx;
        if (sh == 0) dws[s][sr] = rdw;
    };

    float acc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    // MFMA operand rows: lane l supplies row l % 32, bytes 16 (l / 32) .. +15
    const int orow = lane & 31, ok16 = 16 * (lane >> 5);
    const int rsub = 4 * (lane >> 5);  // C rows 8 (e / 4) + rsub + e % 4, column lane % 32

    fetch(0);
    stash(0);
    __syncthreads();
    for (int b = 0; b < nb; b++) {
        const int s = b & 1;
        if (b + 1 < nb) fetch(b + 1);
        v4i A[2], B[2];
#pragma unroll
        for (int i = 0; i < 2; i++) A[i] = *reinterpret_cast<const v4i *>(&As[s][(wm + 32 * i + orow) * 32 + ok16]);
#pragma unroll
        for (int j = 0; j < 2; j++) B[j] = *reinterpret_cast<const v4i *>(&Bs[s][(wn + 32 * j + orow) * 32 + ok16]);
        float dwv[2], dxv[2][16];
#pragma unroll
        for (int j = 0; j < 2; j++) dwv[j] = dws[s][wn + 32 * j + orow];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const floatx4 v = *reinterpret_cast<const floatx4 *>(&dxs[s][wm + 32 * i + 8 * q + rsub]);
                dxv[i][4 * q] = v.x; dxv[i][4 * q + 1] = v.y; dxv[i][4 * q + 2] = v.z; dxv[i][4 * q + 3] = v.w;
            }
        const v16i z = {};
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const v16i c = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[i], B[j], z, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 16; e++)
                    acc[i][j][e] = __builtin_fmaf(static_cast<float>(c[e]), dwv[j] * dxv[i][e], acc[i][j][e]);
            }
        if (b + 1 < nb) {
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
    return align256(static_cast<size_t>(M * K)) + align256(static_cast<size_t>(M * (K / 32)) * sizeof(float));
}

hipError_t gemm_int8_q8_0(const void *w, int64_t row_bytes, const void *x, bool act_f16, void *out,
                          int64_t rows, int64_t n_out, int64_t n_in, void *ws, size_t ws_bytes,
                          hipStream_t st) {
    if (n_in % 32 || rows < 1 || n_out < 1) return hipErrorInvalidValue;
    if (ws_bytes < gemm_int8_workspace(rows, n_in)) return hipErrorInvalidValue;
    if (rows > (1 << 30) || n_out > (1 << 30) || n_in > (1 << 30)) return hipErrorInvalidValue;
    int8_t *xq = static_cast<int8_t *>(ws);
    float *dx = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) + align256(static_cast<size_t>(rows * n_in)));
    hipError_t e = quantize_q8_rows(x, act_f16, rows, n_in, xq, dx, st);
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
