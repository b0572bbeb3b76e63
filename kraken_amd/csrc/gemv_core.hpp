// gemv_core.hpp -- the wave64 GEMV core shared by the dense GEMV launches
// (gemv.hip) and the MoE expert launches (moe.hip).  See gemv.hip for the
// work layout.
#pragma once

#include "krk_formats.hpp"
#include "krk_kernels.hpp"

namespace krk {

template <typename T> __device__ __forceinline__ float to_f(T v) { return static_cast<float>(v); }

// x run loader: RUN consecutive activations starting at p (RUN = 8/16/32).
template <int RUN>
__device__ __forceinline__ void load_run(const float *p, float *o) {
#pragma unroll
    for (int i = 0; i < RUN; i += 4) {
        const floatx4 v = *reinterpret_cast<const floatx4 *>(p + i);
        o[i] = v.x; o[i + 1] = v.y; o[i + 2] = v.z; o[i + 3] = v.w;
    }
}
template <int RUN>
__device__ __forceinline__ void load_run(const _Float16 *p, float *o) {
#pragma unroll
    for (int i = 0; i < RUN; i += 8) {
        const half8 v = *reinterpret_cast<const half8 *>(p + i);
#pragma unroll
        for (int k = 0; k < 8; k++) o[i + k] = static_cast<float>(v[k]);
    }
}

template <typename OT>
__device__ __forceinline__ void store_out(OT *o, float v, int kind, float inv);

template <>
__device__ __forceinline__ void store_out<float>(float *o, float v, int kind, float inv) {
    if (kind == SEG_ACC) *o = __builtin_fmaf(v, inv, *o);
    else *o = v;
}
template <>
__device__ __forceinline__ void store_out<_Float16>(_Float16 *o, float v, int kind, float inv) {
    if (kind == SEG_ACC) {
        // backend_hip.hip gemv_kernel<ACC> (gemm.hpp:96-108): the product is
        // rounded to f16 first, scaled by 2^-rexp, added in f32, saturated.
        const float pv = static_cast<float>(static_cast<_Float16>(v));
        *o = sat_f16(static_cast<float>(*o) + pv * inv);
    } else {
        *o = static_cast<_Float16>(v);
    }
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

// The core: one workgroup, one segment, RB weight rows [n0, n0+RB) of W
// against MR activation rows [m0, m0+MR).  Results land in red[] (per-wave
// partials, LDS) and are combined by the caller.
template <int DT, typename XT, int MR, int RB>
__device__ __forceinline__ void gemv_rows(const uint8_t *__restrict__ w, int64_t row_bytes,
                                          int64_t n_out, int n_in, const XT *const (&xr)[MR],
                                          int64_t n0, const uint8_t *__restrict__ w2,
                                          float (&acc)[MR][RB], int wv = -1, int nw = 0) {
    // wv / nw: this wave's share of K (default: the workgroup's waves split it)
    using F = LaneFmt<DT>;
    constexpr int BV = blk_vals(DT), BB = blk_bytes(DT);
    constexpr int BPS = kWave / F::LPB;
    const int lane = threadIdx.x & 63;
    if (wv < 0) { wv = threadIdx.x >> 6; nw = blockDim.x >> 6; }
    const int p = lane % F::LPB, bl = lane / F::LPB;
    const int nb = n_in / BV;
    const int nsteps = (nb + BPS - 1) / BPS;
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int r = 0; r < RB; r++) acc[m][r] = 0.0f;

    for (int st = wv; st < nsteps; st += nw) {
        const int b = st * BPS + bl;
        if (b >= nb) continue;
        // activations for this lane's piece, and their per-group sums
        float xv[MR][32], xs[MR][F::NG];
#pragma unroll
        for (int m = 0; m < MR; m++) {
            if (xr[m]) {
                const XT *xb = xr[m] + static_cast<int64_t>(b) * BV;
#pragma unroll
                for (int r = 0; r < F::NRUN; r++)
                    load_run<F::RUN>(xb + F::run_start(p, r), &xv[m][r * F::RUN]);
            } else {
#pragma unroll
                for (int i = 0; i < 32; i++) xv[m][i] = 0.0f;
            }
#pragma unroll
            for (int g = 0; g < F::NG; g++) xs[m][g] = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i++) xs[m][F::group_of(i)] += xv[m][i];
        }
        // every row's piece in flight before any is decoded
        uint32_t raw[RB][F::NRAW];
#pragma unroll
        for (int r = 0; r < RB; r++) {
            int64_t n = n0 + (w2 ? (r % (RB / 2)) : r);
            if (n >= n_out) n = n_out - 1;
            const uint8_t *wb = (w2 && r >= RB / 2) ? w2 : w;
            F::load(raw[r], wb + n * row_bytes + static_cast<int64_t>(b) * BB, p);
        }
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int m = 0; m < MR; m++) acc[m][r] += F::dot(raw[r], p, xv[m], xs[m]);
    }
}

}  // namespace krk
