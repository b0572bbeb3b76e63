// gemv.hip -- decode GEMV for Q4_0 / Q8_0 / Q4_K / Q6_K on gfx950 (wave64).
//
// Replaces the reference's gemv_kernel / gemv_m / gemv_mw / gemv_grid
// (src/hip/kernels/gemm.hpp:76-272) and the fused decode groups
// (src/hip/kernels/fused.hpp:71-169).  The arithmetic contract differs from
// the reference GPU path on purpose: weights are decoded to f32 registers, x
// is read in the handle's activation type and widened to f32, and the dot is
// accumulated in f32, so the result tracks the f32 CPU oracle to ~1e-7
// relative instead of the reference GPU's f16 rounding (2e-3..1.5e-2).
//
// Layout of the work (MI355X-first, not a wave32 translation):
//   * a "step" is 2048 consecutive values of K: 64 lanes x 32 values.  For the
//     256-value K-quants 8 lanes share a block (lane piece = 16 B of Q4_K
//     nibbles / 24 B of Q6_K planes); Q4_0 / Q8_0 give each lane one block.
//   * one wave per step, so a workgroup is ceil(K/2048) waves (K = 4096 -> 2,
//     14336 -> 7).  A lane loads its x values once (32 f32 registers per
//     x-row) and keeps them while the workgroup walks RB weight rows: the
//     activation never re-crosses LDS or L1 per weight byte, which is what
//     keeps VALU, not bandwidth, from being the limit.
//   * all RB rows' pieces are loaded before any is decoded (RB x 32 B of
//     loads in flight per lane), the per-row partials of a wave are reduced
//     in one transposed butterfly (wave_reduce_multi), and the waves' partials
//     are added in wave order through LDS.  No atomics: the result is
//     deterministic for a given shape.
#include "gemv_core.hpp"

namespace krk {

template <int DT, typename XT, typename OT, int MR, int RB>
__global__ void __launch_bounds__(512) gemv_seg_kernel(SegTable t) {
    __shared__ float red[8][MR * RB];
    // find this block's segment
    int si = 0;
#pragma unroll 1
    while (si + 1 < t.n && static_cast<int64_t>(blockIdx.x) >= t.seg[si + 1].blk_begin) si++;
    const Seg &s = t.seg[si];
    const int kind = s.kind;
    const bool pair = kind == SEG_SILU;
    const int64_t rows_per_blk = pair ? RB / 2 : RB;
    const int64_t n0 = (static_cast<int64_t>(blockIdx.x) - s.blk_begin) * rows_per_blk;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * MR;
    if (m0 >= t.rows) return;
    const int rows_avail = static_cast<int>(t.rows - m0 < MR ? t.rows - m0 : MR);
    const XT *x = static_cast<const XT *>(s.x) + m0 * t.x_stride;
    const XT *xr[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) xr[m] = m < rows_avail ? x + m * t.x_stride : nullptr;

    float acc[MR][RB];
    gemv_rows<DT, XT, MR, RB>(static_cast<const uint8_t *>(s.w), t.row_bytes, s.n_out, t.n_in, xr,
                              n0, pair ? static_cast<const uint8_t *>(s.w2) : nullptr, acc);

    float v[MR * RB];
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int r = 0; r < RB; r++) v[m * RB + r] = acc[m][r];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    wave_reduce_multi<MR * RB>(v, lane);
    if (reduce_owner<MR * RB>(lane)) red[wv][reduce_owner_index<MR * RB>(lane)] = v[0];
    __syncthreads();
    const int tid = threadIdx.x;
    const float inv = (kind == SEG_ACC && t.rexp) ? exp2f(-static_cast<float>(t.rexp[0])) : 1.0f;
    OT *out = static_cast<OT *>(s.out);
    if (!pair) {
        if (tid < MR * RB) {
            const int m = tid / RB, r = tid % RB;
            float sum = 0.0f;
            for (int k = 0; k < nw; k++) sum += red[k][tid];
            const int64_t n = n0 + r;
            if (m < rows_avail && n < s.n_out)
                store_out<OT>(out + (m0 + m) * t.out_stride + n, sum, kind, inv);
        }
    } else {
        constexpr int H = RB / 2;
        if (tid < MR * H) {
            const int m = tid / H, r = tid % H;
            float g = 0.0f, u = 0.0f;
            for (int k = 0; k < nw; k++) {
                g += red[k][m * RB + r];
                u += red[k][m * RB + H + r];
            }
            const int64_t n = n0 + r;
            if (m < rows_avail && n < s.n_out) {
                OT *o = out + (m0 + m) * t.out_stride + n;
                if constexpr (sizeof(OT) == 2) {
                    // fused_gate_silu_kernel (fused.hpp:161-166): both dots
                    // rounded to f16, activation in f32, saturated store.
                    const float hg = static_cast<float>(static_cast<_Float16>(g));
                    const float hu = static_cast<float>(static_cast<_Float16>(u));
                    *o = sat_f16(silu_f(hg) * hu);
                } else {
                    // silu_mul on f32 (backend_cpu.cpp:2401-2406)
                    *o = (g / (1.0f + expf(-g))) * u;
                }
            }
        }
    }
}

// ------------------------------------------------------------- launcher ----
template <int DT, typename XT, typename OT, int MR, int RB>
static hipError_t launch_seg(const SegTable &t, int64_t total_blocks, hipStream_t st) {
    const int nb = t.n_in / blk_vals(DT);
    const int bps = kWave / LaneFmt<DT>::LPB;
    int nsteps = (nb + bps - 1) / bps;
    int nw = nsteps < 8 ? nsteps : 8;
    if (nw < 1) nw = 1;
    dim3 grid(static_cast<unsigned>(total_blocks), static_cast<unsigned>((t.rows + MR - 1) / MR));
    hipLaunchKernelGGL((gemv_seg_kernel<DT, XT, OT, MR, RB>), grid, dim3(nw * 64), 0, st, t);
    return hipGetLastError();
}

template <int DT, typename XT, typename OT>
static hipError_t dispatch_mr(SegTable t, hipStream_t st) {
    // rows per x pass and weight rows per block, MR*RB = 8 values per lane
    int mr = t.rows <= 1 ? 1 : t.rows == 2 ? 2 : 4;
    const int rb = 8 / mr;
    int64_t blk = 0;
    for (int i = 0; i < t.n; i++) {
        t.seg[i].blk_begin = blk;
        const int64_t per = t.seg[i].kind == SEG_SILU ? rb / 2 : rb;
        blk += (t.seg[i].n_out + per - 1) / per;
    }
    switch (mr) {
        case 1: return launch_seg<DT, XT, OT, 1, 8>(t, blk, st);
        case 2: return launch_seg<DT, XT, OT, 2, 4>(t, blk, st);
        default: return launch_seg<DT, XT, OT, 4, 2>(t, blk, st);
    }
}

template <typename XT, typename OT>
static hipError_t dispatch_dt(int dt, const SegTable &t, hipStream_t st) {
    switch (dt) {
        case DT_Q4_K: return dispatch_mr<DT_Q4_K, XT, OT>(t, st);
        case DT_Q6_K: return dispatch_mr<DT_Q6_K, XT, OT>(t, st);
        case DT_Q4_0: return dispatch_mr<DT_Q4_0, XT, OT>(t, st);
        case DT_Q8_0: return dispatch_mr<DT_Q8_0, XT, OT>(t, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t gemv_segments(int dt, bool act_f16, const SegTable &t, hipStream_t st) {
    if (act_f16) return dispatch_dt<_Float16, _Float16>(dt, t, st);
    return dispatch_dt<float, float>(dt, t, st);
}

}  // namespace krk
