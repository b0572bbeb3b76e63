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

// --------------------------------------------------- persistent decode GEMV --
// rows == 1: a fixed grid of workgroups (as many as the chip keeps resident)
// walks all row groups of all segments.  Each wave loads its 2048-value step
// of x ONCE into registers for the whole kernel (the non-persistent form
// re-read x -- 16 KB at K = 4096 -- for every 4..8 weight rows, more bytes
// than the weights themselves), and the next group's weight pieces are in
// flight while the current group is decoded and reduced.
template <int DT, typename XT, typename OT, int RB>
__global__ void __launch_bounds__(512) gemv_persist_kernel(SegTable t, int64_t total) {
    using F = LaneFmt<DT>;
    constexpr int BV = blk_vals(DT), BB = blk_bytes(DT);
    constexpr int BPS = kWave / F::LPB;
    constexpr int H = RB / 2;
    __shared__ float red[2][8][RB];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int p = lane % F::LPB;
    const int b = wv * BPS + lane / F::LPB;  // this lane's block (one step per wave)
    const int nb = t.n_in / BV;
    const bool active = b < nb;

    // (segment, first row) of a global group index
    auto locate = [&](int64_t g, int &si, int64_t &n0) {
        si = 0;
        while (si + 1 < t.n && g >= t.seg[si + 1].blk_begin) si++;
        n0 = (g - t.seg[si].blk_begin) * (t.seg[si].kind == SEG_SILU ? H : RB);
    };
    auto fetch = [&](uint32_t (&raw)[RB][F::NRAW], int si, int64_t n0) {
        const Seg &s = t.seg[si];
        const bool pair = s.kind == SEG_SILU;
        const uint8_t *w = static_cast<const uint8_t *>(s.w);
        const uint8_t *w2 = static_cast<const uint8_t *>(s.w2);
#pragma unroll
        for (int r = 0; r < RB; r++) {
            int64_t n = n0 + (pair ? (r % H) : r);
            if (n >= s.n_out) n = s.n_out - 1;
            const uint8_t *wb = (pair && r >= H) ? w2 : w;
            F::load(raw[r], wb + n * t.row_bytes + static_cast<int64_t>(b) * BB, p);
        }
    };

    float xv[32], xs[F::NG];
    const void *xcur = nullptr;
    uint32_t rawA[RB][F::NRAW], rawB[RB][F::NRAW];
    int64_t g = blockIdx.x;
    int si;
    int64_t n0;
    if (g < total) {
        locate(g, si, n0);
        if (active) fetch(rawA, si, n0);
    }
    int par = 0;
    for (; g < total; g += gridDim.x, par ^= 1) {
        const Seg &s = t.seg[si];
        // next group's bytes travel while this one is decoded
        const int64_t gn = g + gridDim.x;
        int sn = si;
        int64_t nn = 0;
        if (gn < total) {
            locate(gn, sn, nn);
            if (active) fetch(rawB, sn, nn);
        }
        if (s.x != xcur) {  // once per workgroup unless segments read different x
            xcur = s.x;
            if (active) {
                const XT *xb = static_cast<const XT *>(s.x) + static_cast<int64_t>(b) * BV;
#pragma unroll
                for (int r = 0; r < F::NRUN; r++) load_run<F::RUN>(xb + F::run_start(p, r), &xv[r * F::RUN]);
            } else {
#pragma unroll
                for (int i = 0; i < 32; i++) xv[i] = 0.0f;
            }
#pragma unroll
            for (int q = 0; q < F::NG; q++) xs[q] = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i++) xs[F::group_of(i)] += xv[i];
        }
        float v[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) v[r] = active ? F::dot(rawA[r], p, xv, xs) : 0.0f;
        wave_reduce_multi<RB>(v, lane);
        if (reduce_owner<RB>(lane)) red[par][wv][reduce_owner_index<RB>(lane)] = v[0];
        __syncthreads();
        const int tid = threadIdx.x;
        const int kind = s.kind;
        OT *out = static_cast<OT *>(s.out);
        if (kind != SEG_SILU) {
            if (tid < RB) {
                float sum = 0.0f;
                for (int k = 0; k < nw; k++) sum += red[par][k][tid];
                const int64_t n = n0 + tid;
                const float inv = (kind == SEG_ACC && t.rexp) ? exp2f(-static_cast<float>(t.rexp[0])) : 1.0f;
                if (n < s.n_out) store_out<OT>(out + n, sum, kind, inv);
            }
        } else if (tid < H) {
            float gs = 0.0f, us = 0.0f;
            for (int k = 0; k < nw; k++) {
                gs += red[par][k][tid];
                us += red[par][k][H + tid];
            }
            const int64_t n = n0 + tid;
            if (n < s.n_out) {
                if constexpr (sizeof(OT) == 2) {
                    const float hg = static_cast<float>(static_cast<_Float16>(gs));
                    const float hu = static_cast<float>(static_cast<_Float16>(us));
                    out[n] = sat_f16(silu_f(hg) * hu);
                } else {
                    out[n] = (gs / (1.0f + expf(-gs))) * us;
                }
            }
        }
        // red[par] is rewritten two groups later; the barrier of the next
        // group orders those writes after these reads.
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int k = 0; k < F::NRAW; k++) rawA[r][k] = rawB[r][k];
        si = sn;
        n0 = nn;
    }
}

// ------------------------------------------------- independent-wave GEMV ----
// rows == 1.  Every wave is its own unit of work: a lane owns 64 weights of a
// row (WaveFmt), so one wave covers 4096 values of K with no other wave --
// no LDS, no barrier, no cross-wave reduction.  Waves are persistent: each
// loads its activations once (K <= 4096; longer rows re-read x per 4096-value
// step from L1/L2) and walks groups of RB rows, with the next group's weight
// bytes in flight while the current group is decoded.  A group's RB partial
// sums are reduced across the wave by one transposed butterfly and written
// by their owner lanes.
template <int DT, typename XT, typename OT, int RB>
__global__ void __launch_bounds__(256) gemv_wave_kernel(SegTable t, int64_t total) {
    using F = WaveFmt<DT>;
    constexpr int BV = blk_vals(DT), BB = blk_bytes(DT);
    constexpr int H = RB / 2;
    const int lane = threadIdx.x & 63;
    const int64_t W = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t NW = static_cast<int64_t>(gridDim.x) * (blockDim.x >> 6);
    const int slot = F::slot_of(lane);
    const int nb = t.n_in / BV;
    const int nsteps = (nb + F::BPS - 1) / F::BPS;

    auto locate = [&](int64_t g, int &si, int64_t &n0) {
        si = 0;
        while (si + 1 < t.n && g >= t.seg[si + 1].blk_begin) si++;
        n0 = (g - t.seg[si].blk_begin) * (t.seg[si].kind == SEG_SILU ? H : RB);
    };
    auto fetch = [&](uint32_t (&raw)[RB][F::NRAW], int si, int64_t n0, int st) {
        const Seg &s = t.seg[si];
        const bool pair = s.kind == SEG_SILU;
        // a lane past the row end re-reads the last block(s) and is masked
        // out of the sum (Q4_0 / Q8_0 lanes own two blocks; K % 64 == 0 there)
        int b = st * F::BPS + F::blk_of(lane);
        constexpr int per_lane = (blk_vals(DT) == 32) ? 2 : 1;
        if (b > nb - per_lane) b = nb - per_lane;
#pragma unroll
        for (int r = 0; r < RB; r++) {
            int64_t n = n0 + (pair ? (r % H) : r);
            if (n >= s.n_out) n = s.n_out - 1;
            const uint8_t *wb = static_cast<const uint8_t *>((pair && r >= H) ? s.w2 : s.w);
            F::load(raw[r], wb + n * t.row_bytes + static_cast<int64_t>(b) * BB, slot);
        }
    };
    auto load_x = [&](const void *xp, int st, float (&xv)[64], float (&xs)[F::NG]) {
        const int b = st * F::BPS + F::blk_of(lane);
        const bool ok = b < nb;
        const XT *xb = static_cast<const XT *>(xp) + static_cast<int64_t>(ok ? b : 0) * BV;
#pragma unroll
        for (int r = 0; r < F::NRUN; r++) load_run<F::RUN>(xb + F::run_start(slot, r), &xv[r * F::RUN]);
#pragma unroll
        for (int q = 0; q < F::NG; q++) xs[q] = 0.0f;
#pragma unroll
        for (int i = 0; i < 64; i++) {
            if (!ok) xv[i] = 0.0f;
            xs[F::group_of(i)] += xv[i];
        }
    };

    float xv[64], xs[F::NG];
    const void *xcur = nullptr;
    uint32_t rawA[RB][F::NRAW], rawB[RB][F::NRAW];
    int64_t g = W;
    int si = 0;
    int64_t n0 = 0;
    if (g < total) {
        locate(g, si, n0);
        fetch(rawA, si, n0, 0);
    }
    for (; g < total; g += NW) {
        const Seg &s = t.seg[si];
        float v[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) v[r] = 0.0f;
        const int64_t gn = g + NW;
        int sn = si;
        int64_t nn = 0;
        for (int st = 0; st < nsteps; st++) {
            if (st + 1 < nsteps) {
                fetch(rawB, si, n0, st + 1);
            } else if (gn < total) {  // the next group's first step
                locate(gn, sn, nn);
                fetch(rawB, sn, nn, 0);
            }
            if (nsteps > 1 || s.x != xcur) {
                xcur = s.x;
                load_x(s.x, st, xv, xs);
            }
            const bool ok = st * F::BPS + F::blk_of(lane) < nb;
            if constexpr (DT == DT_Q4_K) {
                // code dword outer, row inner: RB x 4 independent chains
                float acc[RB][F::NACC];
#pragma unroll
                for (int r = 0; r < RB; r++)
#pragma unroll
                    for (int q = 0; q < F::NACC; q++) acc[r][q] = 0.0f;
#pragma unroll
                for (int tt = 0; tt < F::NDW; tt++)
#pragma unroll
                    for (int r = 0; r < RB; r++) F::accum(rawA[r], tt, xv, acc[r]);
#pragma unroll
                for (int r = 0; r < RB; r++) {
                    const float d = F::finish(rawA[r], slot, acc[r], xs);
                    v[r] += ok ? d : 0.0f;
                }
            } else
#pragma unroll
            for (int r = 0; r < RB; r++) {
                const float d = F::dot(rawA[r], slot, xv, xs);
                v[r] += ok ? d : 0.0f;
            }
#pragma unroll
            for (int r = 0; r < RB; r++)
#pragma unroll
                for (int k = 0; k < F::NRAW; k++) rawA[r][k] = rawB[r][k];
        }
        wave_reduce_multi<RB>(v, lane);
        const int idx = reduce_owner_index<RB>(lane);
        const int kind = s.kind;
        OT *out = static_cast<OT *>(s.out);
        if (kind != SEG_SILU) {
            if (reduce_owner<RB>(lane)) {
                const int64_t n = n0 + idx;
                const float inv = (kind == SEG_ACC && t.rexp) ? exp2f(-static_cast<float>(t.rexp[0])) : 1.0f;
                if (n < s.n_out) store_out<OT>(out + n, v[0], kind, inv);
            }
        } else {
            // up row r sits with the owner of index H + r
            constexpr int SH = 64 / RB;  // lanes per owned index
            const float u = __shfl(v[0], (lane + H * SH) & 63, 64);
            if (reduce_owner<RB>(lane) && idx < H) {
                const int64_t n = n0 + idx;
                if (n < s.n_out) {
                    const float gs = v[0];
                    if constexpr (sizeof(OT) == 2) {
                        const float hg = static_cast<float>(static_cast<_Float16>(gs));
                        const float hu = static_cast<float>(static_cast<_Float16>(u));
                        out[n] = sat_f16(silu_f(hg) * hu);
                    } else {
                        out[n] = (gs / (1.0f + expf(-gs))) * u;
                    }
                }
            }
        }
        si = sn;
        n0 = nn;
    }
}

template <int DT, typename XT, typename OT, int RB>
static hipError_t launch_wave(SegTable t, hipStream_t st) {
    int64_t total = 0;
    for (int i = 0; i < t.n; i++) {
        t.seg[i].blk_begin = total;
        const int64_t per = t.seg[i].kind == SEG_SILU ? RB / 2 : RB;
        total += (t.seg[i].n_out + per - 1) / per;
    }
    static thread_local int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cus = 256;
    }
    static thread_local int per_cu = 0;
    if (!per_cu &&
        (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_wave_kernel<DT, XT, OT, RB>, 256, 0) !=
             hipSuccess || per_cu < 1))
        per_cu = 1;
    const int64_t waves = total;  // one wave per group at most
    int64_t grid = static_cast<int64_t>(cus) * per_cu;
    if (grid * 4 > waves) grid = (waves + 3) / 4;
    hipLaunchKernelGGL((gemv_wave_kernel<DT, XT, OT, RB>), dim3(static_cast<unsigned>(grid)), dim3(256),
                       0, st, t, total);
    return hipGetLastError();
}

// ------------------------------------------------------- LDS-staged GEMV ----
// rows == 1, the decode shape.  Measured on MI355X: with x held in registers,
// every wave must pull its whole 16 KB slice of x through L2/L1 once, and
// with the few rows per wave that latency hiding needs, that is as many
// bytes as the weights (7x at one row per wave).  So x is staged ONCE per
// workgroup into LDS (f32, padded 4 floats per 64 so the b128 reads of the
// 64 lanes spread over the banks), and waves read it back in 4-value runs,
// each run applied to RB rows.  A lane owns 64 weights of a row (WaveFmt
// layout), a wave covers 4096 values of K with no other wave, waves are
// persistent and independent (no barrier after the staging), and the next
// group's weight bytes are in flight while the current group is decoded.
__device__ __forceinline__ int xpad(int k) { return k + 4 * (k >> 6); }

template <int DT> struct XRuns;  // where dword t of a lane's codes finds its x
template <> struct XRuns<DT_Q4_K> {
    // lane base 64*jp within the block; dword t: low run 4t, high run 32 + 4t
    __device__ static int base(int lane) { return 256 * (lane >> 2) + 64 * (lane & 3); }
};
template <> struct XRuns<DT_Q5_K> {
    // Q4_K's value order: lane base 64*jp; dword t: low run 4t, high run 32 + 4t
    __device__ static int base(int lane) { return 256 * (lane >> 2) + 64 * (lane & 3); }
};
template <> struct XRuns<DT_Q6_K> {
    __device__ static int base(int lane) {
        const int jp = lane & 3;
        return 256 * (lane >> 2) + 128 * (jp >> 1) + 16 * (jp & 1);
    }
};
template <> struct XRuns<DT_Q2_K> : XRuns<DT_Q6_K> {};
template <> struct XRuns<DT_Q3_K> : XRuns<DT_Q6_K> {};
template <> struct XRuns<DT_Q4_0> {
    __device__ static int base(int lane) { return 64 * lane; }
};
template <> struct XRuns<DT_IQ4_NL> {
    __device__ static int base(int lane) { return 64 * lane; }
};
template <> struct XRuns<DT_IQ4_XS> {
    __device__ static int base(int lane) { return 64 * lane; }   // 256 (lane / 4) + 64 (lane % 4)
};
template <> struct XRuns<DT_Q4_1> : XRuns<DT_Q4_0> {};
template <> struct XRuns<DT_F16> : XRuns<DT_Q4_0> {};
template <> struct XRuns<DT_BF16> : XRuns<DT_Q4_0> {};
template <> struct XRuns<DT_Q5_0> : XRuns<DT_Q4_0> {};
template <> struct XRuns<DT_Q5_1> : XRuns<DT_Q4_0> {};
template <> struct XRuns<DT_MXFP4> {
    __device__ static int base(int lane) { return 64 * lane; }
};
template <> struct XRuns<DT_Q8_0> {
    __device__ static int base(int lane) { return 64 * lane; }
};

template <int DT, int RB> struct LdsDot;

template <int RB> struct LdsDot<DT_Q4_K, RB> {
    using F = WaveFmt<DT_Q4_K>;
    static constexpr int NS = 2;  // x sums per lane
    __device__ static void sums(const float *xl, int b0, float (&xs)[NS]) {
        float a = 0.0f, c = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            const floatx4 u = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + i));
            const floatx4 w = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 + i));
            a += (u.x + u.y) + (u.z + u.w);
            c += (w.x + w.y) + (w.z + w.w);
        }
        xs[0] = a; xs[1] = c;
    }
    __device__ static void run(const uint32_t (&raw)[RB][F::NRAW], int jp, const float *xl, int b0,
                               const float (&xs)[NS], float (&v)[RB]) {
        float acc[RB][4];
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int q = 0; q < 4; q++) acc[r][q] = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const floatx4 lo = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 4 * t));
            const floatx4 hi = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 + 4 * t));
            const float xl4[4] = {lo.x, lo.y, lo.z, lo.w}, xh4[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
            for (int r = 0; r < RB; r++) nib8(raw[r][4 + t], xl4, xh4, acc[r][t & 1], acc[r][2 + (t & 1)]);
        }
#pragma unroll
        for (int r = 0; r < RB; r++) v[r] = F::finish(raw[r], jp, acc[r], xs);
    }
};

template <int RB> struct LdsDot<DT_Q5_K, RB> {
    using F = WaveFmt<DT_Q5_K>;
    static constexpr int NS = 2;  // x sums per lane
    __device__ static void sums(const float *xl, int b0, float (&xs)[NS]) {
        LdsDot<DT_Q4_K, RB>::sums(xl, b0, xs);
    }
    __device__ static void run(const uint32_t (&raw)[RB][F::NRAW], int jp, const float *xl, int b0,
                               const float (&xs)[NS], float (&v)[RB]) {
        float acc[RB][4];
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int q = 0; q < 4; q++) acc[r][q] = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const floatx4 lo = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 4 * t));
            const floatx4 hi = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 + 4 * t));
            const float xl4[4] = {lo.x, lo.y, lo.z, lo.w}, xh4[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
            for (int r = 0; r < RB; r++) F::accum(raw[r], t, jp, xl4, xh4, acc[r]);
        }
#pragma unroll
        for (int r = 0; r < RB; r++) v[r] = F::finish(raw[r], jp, acc[r], xs);
    }
};

template <int RB> struct LdsDot<DT_Q6_K, RB> {
    using F = WaveFmt<DT_Q6_K>;
    static constexpr int NS = 4;
    __device__ static void sums(const float *xl, int b0, float (&xs)[NS]) {
#pragma unroll
        for (int qd = 0; qd < 4; qd++) {
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const floatx4 u = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * qd + i));
                a += (u.x + u.y) + (u.z + u.w);
            }
            xs[qd] = a;
        }
    }
    __device__ static void run(const uint32_t (&raw)[RB][F::NRAW], int jp, const float *xl, int b0,
                               const float (&xs)[NS], float (&v)[RB]) {
        float sq[RB][4];
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int q = 0; q < 4; q++) sq[r][q] = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            float xq[4][4];
#pragma unroll
            for (int qd = 0; qd < 4; qd++) {
                const floatx4 u = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * qd + 4 * t));
                xq[qd][0] = u.x; xq[qd][1] = u.y; xq[qd][2] = u.z; xq[qd][3] = u.w;
            }
#pragma unroll
            for (int r = 0; r < RB; r++) {
                const uint32_t A = raw[r][t], B = raw[r][4 + t], H = raw[r][8 + t];
                const uint32_t q[4] = {(A & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u),
                                       (B & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u),
                                       ((A >> 4) & 0x0F0F0F0Fu) | (H & 0x30303030u),
                                       ((B >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u)};
#pragma unroll
                for (int qd = 0; qd < 4; qd++) {
                    sq[r][qd] = mix2(q[qd] & 0x003F003Fu, xq[qd][0], xq[qd][2], sq[r][qd]);
                    sq[r][qd] = mix2((q[qd] >> 8) & 0x003F003Fu, xq[qd][1], xq[qd][3], sq[r][qd]);
                }
            }
        }
        const uint32_t sel = 8u * static_cast<uint32_t>(jp & 1);
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const float d = h2f(raw[r][14] & 0xFFFF);
            const uint32_t w0 = raw[r][12] >> sel, w1 = raw[r][13] >> sel;
            const int sc[4] = {static_cast<int8_t>(w0 & 0xFF), static_cast<int8_t>((w0 >> 16) & 0xFF),
                               static_cast<int8_t>(w1 & 0xFF), static_cast<int8_t>((w1 >> 16) & 0xFF)};
            float a = 0.0f;
#pragma unroll
            for (int qd = 0; qd < 4; qd++) {
                const float ds = d * static_cast<float>(sc[qd]);
                a = __builtin_fmaf(ds * kTwo24, sq[r][qd], a);
                a = __builtin_fmaf(-32.0f * ds, xs[qd], a);
            }
            v[r] = a;
        }
    }
};

// Q2_K / Q3_K: Q6_K's x runs and plane sums, their own codes and fold
template <int DT, int RB> struct LdsDotPlanes {
    using F = WaveFmt<DT>;
    static constexpr int NS = 4;
    __device__ static void sums(const float *xl, int b0, float (&xs)[NS]) {
        LdsDot<DT_Q6_K, RB>::sums(xl, b0, xs);
    }
    __device__ static void run(const uint32_t (&raw)[RB][F::NRAW], int jp, const float *xl, int b0,
                               const float (&xs)[NS], float (&v)[RB]) {
        float sq[RB][4];
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int q = 0; q < 4; q++) sq[r][q] = 0.0f;
        const int h = jp >> 1;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            float xq[4][4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const floatx4 u = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * j + 4 * t));
                xq[j][0] = u.x; xq[j][1] = u.y; xq[j][2] = u.z; xq[j][3] = u.w;
            }
#pragma unroll
            for (int r = 0; r < RB; r++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    uint32_t q, m;
                    if constexpr (DT == DT_Q2_K) {
                        q = plane2(raw[r][t], j);
                        m = 0x00030003u;
                    } else {
                        q = plane3(raw[r][t] >> (2 * j), raw[r][4 + t], 4 * h + j);
                        m = 0x00070007u;
                    }
                    sq[r][j] = mix2(q & m, xq[j][0], xq[j][2], sq[r][j]);
                    sq[r][j] = mix2((q >> 8) & m, xq[j][1], xq[j][3], sq[r][j]);
                }
        }
#pragma unroll
        for (int r = 0; r < RB; r++) v[r] = F::fold(raw[r], jp, sq[r], xs);
    }
};
template <int RB> struct LdsDot<DT_Q2_K, RB> : LdsDotPlanes<DT_Q2_K, RB> {};
template <int RB> struct LdsDot<DT_Q3_K, RB> : LdsDotPlanes<DT_Q3_K, RB> {};

template <int RB> struct LdsDot<DT_Q4_0, RB> {
    using F = WaveFmt<DT_Q4_0>;
    static constexpr int NS = 2;
    __device__ static void sums(const float *xl, int b0, float (&xs)[NS]) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                const floatx4 w = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * u + i));
                a += (w.x + w.y) + (w.z + w.w);
            }
            xs[u] = a;
        }
    }
    __device__ static void run(const uint32_t (&raw)[RB][F::NRAW], int, const float *xl, int b0,
                               const float (&xs)[NS], float (&v)[RB]) {
        float acc[RB][2][2];
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int u = 0; u < 2; u++) acc[r][u][0] = acc[r][u][1] = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const floatx4 lo = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * u + 4 * t));
                const floatx4 hi = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * u + 16 + 4 * t));
                const float xl4[4] = {lo.x, lo.y, lo.z, lo.w}, xh4[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
                for (int r = 0; r < RB; r++) nib8(raw[r][5 * u + t], xl4, xh4, acc[r][u][0], acc[r][u][1]);
            }
#pragma unroll
        for (int r = 0; r < RB; r++) {
            float a = 0.0f;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float d = h2f(raw[r][5 * u + 4] & 0xFFFF);
                a = __builtin_fmaf(d * kTwo24, acc[r][u][0], a);
                a = __builtin_fmaf(d * kTwo20, acc[r][u][1], a);
                a = __builtin_fmaf(-8.0f * d, xs[u], a);
            }
            v[r] = a;
        }
    }
};

template <int RB> struct LdsDot<DT_IQ4_NL, RB> {
    using F = WaveFmt<DT_IQ4_NL>;
    static constexpr int NS = 2;
    __device__ static void sums(const float *xl, int b0, float (&xs)[NS]) {
        LdsDot<DT_Q4_0, RB>::sums(xl, b0, xs);
    }
    __device__ static void run(const uint32_t (&raw)[RB][F::NRAW], int, const float *xl, int b0,
                               const float (&xs)[NS], float (&v)[RB]) {
        float acc[RB][2];
#pragma unroll
        for (int r = 0; r < RB; r++) acc[r][0] = acc[r][1] = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const floatx4 lo = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * u + 4 * t));
                const floatx4 hi = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * u + 16 + 4 * t));
                const float xl4[4] = {lo.x, lo.y, lo.z, lo.w}, xh4[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
                for (int r = 0; r < RB; r++) acc[r][u] = iq4x8(raw[r][5 * u + t], xl4, xh4, acc[r][u]);
            }
#pragma unroll
        for (int r = 0; r < RB; r++) {
            float a = 0.0f;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float d = h2f(raw[r][5 * u + 4] & 0xFFFF);
                a = __builtin_fmaf(d * kTwo24, acc[r][u], a);
                a = __builtin_fmaf(-128.0f * d, xs[u], a);
            }
            v[r] = a;
        }
    }
};

template <int RB> struct LdsDot<DT_MXFP4, RB> {
    using F = WaveFmt<DT_MXFP4>;
    static constexpr int NS = 2;
    __device__ static void sums(const float *xl, int b0, float (&xs)[NS]) {
        LdsDot<DT_Q4_0, RB>::sums(xl, b0, xs);
    }
    __device__ static void run(const uint32_t (&raw)[RB][F::NRAW], int, const float *xl, int b0,
                               const float (&xs)[NS], float (&v)[RB]) {
        float acc[RB][2];
#pragma unroll
        for (int r = 0; r < RB; r++) acc[r][0] = acc[r][1] = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const floatx4 lo = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * u + 4 * t));
                const floatx4 hi = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * u + 16 + 4 * t));
                const float xl4[4] = {lo.x, lo.y, lo.z, lo.w}, xh4[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
                for (int r = 0; r < RB; r++) acc[r][u] = iq4x8<true>(raw[r][5 * u + t], xl4, xh4, acc[r][u]);
            }
#pragma unroll
        for (int r = 0; r < RB; r++) {
            float a = 0.0f;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float d = e8m0_half(raw[r][5 * u + 4]);
                a = __builtin_fmaf(d * kTwo24, acc[r][u], a);
                a = __builtin_fmaf(-12.0f * d, xs[u], a);
            }
            v[r] = a;
        }
    }
};

template <int DT, int RB> struct LdsDotL32 {
    using F = WaveFmt<DT>;
    static constexpr int NS = 2;
    __device__ static void sums(const float *xl, int b0, float (&xs)[NS]) {
        LdsDot<DT_Q4_0, RB>::sums(xl, b0, xs);
    }
    __device__ static void run(const uint32_t (&raw)[RB][F::NRAW], int, const float *xl, int b0,
                               const float (&xs)[NS], float (&v)[RB]) {
        float acc[RB][2];
#pragma unroll
        for (int r = 0; r < RB; r++) acc[r][0] = acc[r][1] = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const floatx4 lo = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * u + 4 * t));
                const floatx4 hi = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * u + 16 + 4 * t));
#pragma unroll
                for (int r = 0; r < RB; r++) {
                    const uint32_t cl = l32_codes<DT>(&raw[r][6 * u], t, 0), ch = l32_codes<DT>(&raw[r][6 * u], t, 1);
                    float a = acc[r][u];
                    a = mix2(cl & 0x001F001Fu, lo.x, lo.z, a);
                    a = mix2((cl >> 8) & 0x001F001Fu, lo.y, lo.w, a);
                    a = mix2(ch & 0x001F001Fu, hi.x, hi.z, a);
                    acc[r][u] = mix2((ch >> 8) & 0x001F001Fu, hi.y, hi.w, a);
                }
            }
#pragma unroll
        for (int r = 0; r < RB; r++) {
            float a = 0.0f;
#pragma unroll
            for (int u = 0; u < 2; u++) a = l32_fold<DT>(&raw[r][6 * u], acc[r][u], xs[u], a);
            v[r] = a;
        }
    }
};
template <int DT, int RB> struct LdsDotFloat {
    using F = WaveFmt<DT>;
    static constexpr int NS = 1;
    __device__ static void sums(const float *, int, float (&xs)[NS]) { xs[0] = 0.0f; }
    __device__ static void run(const uint32_t (&raw)[RB][F::NRAW], int, const float *xl, int b0,
                               const float (&)[NS], float (&v)[RB]) {
        float acc[RB][2];
#pragma unroll
        for (int r = 0; r < RB; r++) acc[r][0] = acc[r][1] = 0.0f;
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const floatx4 u = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 4 * t));
#pragma unroll
            for (int r = 0; r < RB; r++) {
                acc[r][t & 1] = LaneFmtFloat<DT>::pair(raw[r][2 * t], u.x, u.y, acc[r][t & 1]);
                acc[r][t & 1] = LaneFmtFloat<DT>::pair(raw[r][2 * t + 1], u.z, u.w, acc[r][t & 1]);
            }
        }
#pragma unroll
        for (int r = 0; r < RB; r++) v[r] = acc[r][0] + acc[r][1];
    }
};
template <int RB> struct LdsDot<DT_F16, RB> : LdsDotFloat<DT_F16, RB> {};
template <int RB> struct LdsDot<DT_BF16, RB> : LdsDotFloat<DT_BF16, RB> {};
template <int RB> struct LdsDot<DT_Q4_1, RB> : LdsDotL32<DT_Q4_1, RB> {};
template <int RB> struct LdsDot<DT_Q5_0, RB> : LdsDotL32<DT_Q5_0, RB> {};
template <int RB> struct LdsDot<DT_Q5_1, RB> : LdsDotL32<DT_Q5_1, RB> {};

template <int RB> struct LdsDot<DT_IQ4_XS, RB> {
    using F = WaveFmt<DT_IQ4_XS>;
    static constexpr int NS = 2;
    __device__ static void sums(const float *xl, int b0, float (&xs)[NS]) {
        LdsDot<DT_Q4_0, RB>::sums(xl, b0, xs);
    }
    __device__ static void run(const uint32_t (&raw)[RB][F::NRAW], int jp, const float *xl, int b0,
                               const float (&xs)[NS], float (&v)[RB]) {
        float acc[RB][2];
#pragma unroll
        for (int r = 0; r < RB; r++) acc[r][0] = acc[r][1] = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const floatx4 lo = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * u + 4 * t));
                const floatx4 hi = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * u + 16 + 4 * t));
                const float xl4[4] = {lo.x, lo.y, lo.z, lo.w}, xh4[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
                for (int r = 0; r < RB; r++) acc[r][u] = iq4x8(raw[r][4 * u + t], xl4, xh4, acc[r][u]);
            }
#pragma unroll
        for (int r = 0; r < RB; r++) {
            float a = 0.0f;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float dl = iq4xs_scale(raw[r][8], raw[r][9], 2 * jp + u);
                a = __builtin_fmaf(dl * kTwo24, acc[r][u], a);
                a = __builtin_fmaf(-128.0f * dl, xs[u], a);
            }
            v[r] = a;
        }
    }
};

template <int RB> struct LdsDot<DT_Q8_0, RB> {
    using F = WaveFmt<DT_Q8_0>;
    static constexpr int NS = 2;
    __device__ static void sums(const float *xl, int b0, float (&xs)[NS]) {
        LdsDot<DT_Q4_0, RB>::sums(xl, b0, xs);
    }
    __device__ static void run(const uint32_t (&raw)[RB][F::NRAW], int, const float *xl, int b0,
                               const float (&xs)[NS], float (&v)[RB]) {
        float acc[RB][2][2];
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int u = 0; u < 2; u++) acc[r][u][0] = acc[r][u][1] = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const floatx4 xv = *reinterpret_cast<const floatx4 *>(xl + xpad(b0 + 32 * u + 4 * t));
#pragma unroll
                for (int r = 0; r < RB; r++) {
                    const uint32_t q = raw[r][9 * u + t] ^ 0x80808080u;
                    acc[r][u][0] = mix2(q & 0x00FF00FFu, xv.x, xv.z, acc[r][u][0]);
                    acc[r][u][1] = mix2((q >> 8) & 0x00FF00FFu, xv.y, xv.w, acc[r][u][1]);
                }
            }
#pragma unroll
        for (int r = 0; r < RB; r++) {
            float a = 0.0f;
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const float d = h2f(raw[r][9 * u + 8] & 0xFFFF);
                a = __builtin_fmaf(d * kTwo24, acc[r][u][0] + acc[r][u][1], a);
                a = __builtin_fmaf(-128.0f * d, xs[u], a);
            }
            v[r] = a;
        }
    }
};

template <int DT, typename XT, typename OT, int RB>
__global__ void __launch_bounds__(256) gemv_lds_kernel(SegTable t, int64_t total) {
    using F = WaveFmt<DT>;
    using D = LdsDot<DT, RB>;
    constexpr int BV = blk_vals(DT), BB = blk_bytes(DT);
    constexpr int H = RB / 2;
    extern __shared__ float xl[];
    const int lane = threadIdx.x & 63;
    const int64_t W = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t NW = static_cast<int64_t>(gridDim.x) * (blockDim.x >> 6);
    const int slot = F::slot_of(lane);
    const int nb = t.n_in / BV;
    const int nsteps = (nb + F::BPS - 1) / F::BPS;

    auto locate = [&](int64_t g, int &si, int64_t &n0) {
        si = 0;
        while (si + 1 < t.n && g >= t.seg[si + 1].blk_begin) si++;
        n0 = (g - t.seg[si].blk_begin) * (t.seg[si].kind == SEG_SILU ? H : RB);
    };
    auto fetch = [&](uint32_t (&raw)[RB][F::NRAW], int si, int64_t n0, int st) {
        const Seg &s = t.seg[si];
        const bool pair = s.kind == SEG_SILU;
        constexpr int per_lane = (blk_vals(DT) == 32) ? 2 : 1;
        int b = st * F::BPS + F::blk_of(lane);
        if (b > nb - per_lane) b = nb - per_lane;
#pragma unroll
        for (int r = 0; r < RB; r++) {
            int64_t n = n0 + (pair ? (r % H) : r);
            if (n >= s.n_out) n = s.n_out - 1;
            const uint8_t *wb = static_cast<const uint8_t *>((pair && r >= H) ? s.w2 : s.w);
            F::load(raw[r], wb + n * t.row_bytes + static_cast<int64_t>(b) * BB, slot);
        }
    };

    float xs[D::NS];
    int xs_step = -1;
    uint32_t rawA[RB][F::NRAW], rawB[RB][F::NRAW];
    int64_t g = W;
    int si = 0;
    int64_t n0 = 0;
    // the first group's weight bytes are requested before x is staged, so
    // the two HBM round trips overlap instead of following each other
    if (g < total) {
        locate(g, si, n0);
        fetch(rawA, si, n0, 0);
    }
    // stage x (all segments of a launch read the same x)
    {
        const XT *x = static_cast<const XT *>(t.seg[0].x);
        for (int k = threadIdx.x * 4; k < t.n_in; k += blockDim.x * 4) {
            floatx4 v;
            if constexpr (sizeof(XT) == 4) {
                v = *reinterpret_cast<const floatx4 *>(x + k);
            } else {
                v = floatx4{static_cast<float>(x[k]), static_cast<float>(x[k + 1]),
                             static_cast<float>(x[k + 2]), static_cast<float>(x[k + 3])};
            }
            *reinterpret_cast<floatx4 *>(xl + xpad(k)) = v;
        }
    }
    __syncthreads();

    for (; g < total; g += NW) {
        const Seg &s = t.seg[si];
        float v[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) v[r] = 0.0f;
        const int64_t gn = g + NW;
        int sn = si;
        int64_t nn = 0;
        for (int st = 0; st < nsteps; st++) {
            if (st + 1 < nsteps) {
                fetch(rawB, si, n0, st + 1);
            } else if (gn < total) {
                locate(gn, sn, nn);
                fetch(rawB, sn, nn, 0);
            }
            const bool ok = st * F::BPS + F::blk_of(lane) < nb;
            const int b0 = ok ? st * F::BPS * BV + XRuns<DT>::base(lane) : 0;
            if (xs_step != st) {
                D::sums(xl, b0, xs);
                xs_step = nsteps > 1 ? -1 : st;
            }
            float d[RB];
            D::run(rawA, slot, xl, b0, xs, d);
#pragma unroll
            for (int r = 0; r < RB; r++) v[r] += ok ? d[r] : 0.0f;
#pragma unroll
            for (int r = 0; r < RB; r++)
#pragma unroll
                for (int k = 0; k < F::NRAW; k++) rawA[r][k] = rawB[r][k];
        }
        wave_reduce_multi<RB>(v, lane);
        const int idx = reduce_owner_index<RB>(lane);
        const int kind = s.kind;
        OT *out = static_cast<OT *>(s.out);
        if (kind != SEG_SILU) {
            if (reduce_owner<RB>(lane)) {
                const int64_t n = n0 + idx;
                const float inv = (kind == SEG_ACC && t.rexp) ? exp2f(-static_cast<float>(t.rexp[0])) : 1.0f;
                if (n < s.n_out) store_out<OT>(out + n, v[0], kind, inv);
            }
        } else {
            constexpr int SH = 64 / RB;
            const float u = __shfl(v[0], (lane + H * SH) & 63, 64);
            if (reduce_owner<RB>(lane) && idx < H) {
                const int64_t n = n0 + idx;
                if (n < s.n_out) {
                    const float gs = v[0];
                    if constexpr (sizeof(OT) == 2) {
                        const float hg = static_cast<float>(static_cast<_Float16>(gs));
                        const float hu = static_cast<float>(static_cast<_Float16>(u));
                        out[n] = sat_f16(silu_f(hg) * hu);
                    } else {
                        out[n] = (gs / (1.0f + expf(-gs))) * u;
                    }
                }
            }
        }
        si = sn;
        n0 = nn;
    }
}

// --------------------------------------------- LDS-DMA streamed decode GEMV --
// Measured on MI355X: the vector-memory path delivers ~5.2 TB/s of LANE
// bytes whether they come from HBM or L2, so a decode GEMV is bound by the
// bytes its lanes receive, not by the bytes HBM sends.  Per-lane loads of a
// block's header (8 or 4 lanes re-reading the same 16 B) and per-wave x
// reloads cost as much as the weights themselves.  This kernel therefore
// receives every weight byte exactly once: a wave copies its group of RB
// consecutive rows (one contiguous region) into a private LDS slot with
// global_load_lds_dwordx4 -- 64 lanes x 16 B = 1 KB per instruction, fully
// coalesced, no VGPR round trip -- and lanes then read their pieces from
// LDS.  Three slots per wave keep two groups in flight while one is decoded;
// x is staged once per workgroup.  The compiler does not track the LDS-DMA
// dependency, so the waits are explicit (vmcnt counts this wave's
// outstanding loads in issue order).
typedef __attribute__((address_space(3))) void lds_void_t;

template <int N> __device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    // s_waitcnt simm16: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// A unit of work is RB rows x one wave step (4096 values of K); its bytes
// are RB pieces of P = BPS * BB contiguous bytes that the DMA gathers into a
// slot back to back.  XREG: the whole row is one step (K <= 4096), so each
// lane keeps its 64 activations and their group sums in registers for the
// kernel's lifetime; otherwise x is staged in LDS and read per unit.
template <int DT, typename XT, typename OT, int RB, int NSLOT, bool XREG>
__global__ void __launch_bounds__(512) gemv_valu_kernel(SegTable t, int64_t total, int xfloats) {
    using F = WaveFmt<DT>;
    using D = LdsDot<DT, RB>;
    constexpr int BV = blk_vals(DT), BB = blk_bytes(DT);
    constexpr int P = F::BPS * BB;               // one row's bytes of one step
    constexpr int U = RB * P;                    // one unit's bytes
    constexpr int CH = (U + 1023) / 1024;        // DMA instructions per unit
    constexpr int SLOT = CH * 1024;
    constexpr int per_lane = (blk_vals(DT) == 32) ? 2 : 1;
    static_assert(P % 16 == 0, "pieces must be whole 16-byte chunks");
    static_assert((NSLOT - 1) * CH < 64, "vmcnt is 6 bits");
    extern __shared__ float smem[];
    __shared__ Seg segl[kMaxSegs];
    float *xl = smem;
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t *slots = reinterpret_cast<uint8_t *>(smem + (XREG ? 0 : xfloats)) + wv * (NSLOT * SLOT);
    const int64_t W = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + wv;
    const int64_t NW = static_cast<int64_t>(gridDim.x) * (blockDim.x >> 6);
    const int slot_lane = F::slot_of(lane);
    const int nb = t.n_in / BV;
    const int nsteps = XREG ? 1 : (nb + F::BPS - 1) / F::BPS;
    const int64_t rb = t.row_bytes;
    const int64_t my_groups = W < total ? (total - 1 - W) / NW + 1 : 0;
    const int64_t my_units = my_groups * nsteps;

    // The segment table is copied to LDS: indexed in the kernel arguments it
    // would be read through vector memory, and the waits for those reads
    // would also drain the weight DMA.
    const int nseg = t.n;
    if (threadIdx.x < nseg) segl[threadIdx.x] = t.seg[threadIdx.x];
    const float inv_acc = t.rexp ? exp2f(-static_cast<float>(t.rexp[0])) : 1.0f;
    __syncthreads();
    auto seg_of = [&](int64_t g) {
        int i = 0;
        while (i + 1 < nseg && g >= segl[i + 1].blk_begin) i++;
        return i;
    };

    // Chunk c of a unit: lane bytes [1024c + 16 lane, +16) of the RB pieces,
    // i.e. row r = o / P at offset o % P of the step.  Lanes past U re-read
    // the unit's first chunk into the slot's unused tail.
    int32_t dl[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int o = c * 1024 + 16 * lane;
        const int r = o / P;
        dl[c] = o < U ? static_cast<int32_t>(r * rb + (o - r * P)) : 16 * lane;
    }
    auto issue = [&](int64_t j) {
        const int64_t g = W + (j / nsteps) * NW;
        const int st = static_cast<int>(j % nsteps);
        const int si = seg_of(g);
        const uint8_t *w = static_cast<const uint8_t *>(segl[si].w);
        const int64_t n_out = segl[si].n_out;
        const int64_t n0 = (g - segl[si].blk_begin) * RB;
        const uint8_t *base = w + n0 * rb + static_cast<int64_t>(st) * P;
        uint8_t *dst = slots + static_cast<int>(j % NSLOT) * SLOT;
        if ((n0 + RB - 1) * rb + static_cast<int64_t>(st) * P + P <= n_out * rb) {
#pragma unroll
            for (int c = 0; c < CH; c++)
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(base + dl[c]),
                                                 (lds_void_t *)(dst + c * 1024), 16, 0, 0);
        } else {
            // the matrix's last rows: clamp rows and row ends to stay inside
            const int64_t lim = rb - 16;
#pragma unroll
            for (int c = 0; c < CH; c++) {
                const int o = c * 1024 + 16 * lane;
                const int r = o < U ? o / P : 0;
                int64_t n = n0 + r;
                if (n >= n_out) n = n_out - 1;
                int64_t off = static_cast<int64_t>(st) * P + (o < U ? o - r * P : 0);
                if (off > lim) off = lim;
                __builtin_amdgcn_global_load_lds(static_cast<const void *>(w + n * rb + off),
                                                 (lds_void_t *)(dst + c * 1024), 16, 0, 0);
            }
        }
    };

#pragma unroll
    for (int k = 0; k < NSLOT - 1; k++)
        if (k < my_units) issue(k);

    // activations: registers (XREG) or LDS, fetched while the DMA is in flight
    float xv[XREG ? 64 : 1], xg[XREG ? F::NG : 1];
    const XT *xsrc = static_cast<const XT *>(t.seg[0].x);
    if constexpr (XREG) {
        const int b = F::blk_of(lane);
        const bool okx = b < nb;
        const XT *xb = xsrc + static_cast<int64_t>(okx ? b : 0) * BV;
#pragma unroll
        for (int r = 0; r < F::NRUN; r++) load_run<F::RUN>(xb + F::run_start(slot_lane, r), &xv[r * F::RUN]);
#pragma unroll
        for (int q = 0; q < F::NG; q++) xg[q] = 0.0f;
#pragma unroll
        for (int i = 0; i < 64; i++) {
            if (!okx) xv[i] = 0.0f;
            xg[F::group_of(i)] += xv[i];
        }
    } else {
        for (int k = threadIdx.x * 4; k < t.n_in; k += blockDim.x * 4) {
            floatx4 v;
            if constexpr (sizeof(XT) == 4) {
                v = *reinterpret_cast<const floatx4 *>(xsrc + k);
            } else {
                v = floatx4{static_cast<float>(xsrc[k]), static_cast<float>(xsrc[k + 1]),
                             static_cast<float>(xsrc[k + 2]), static_cast<float>(xsrc[k + 3])};
            }
            *reinterpret_cast<floatx4 *>(xl + xpad(k)) = v;
        }
        __syncthreads();
    }

    float xs[D::NS];
    int xs_step = -1;
    float v[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) v[r] = 0.0f;
    for (int64_t j = 0; j < my_units; j++) {
        // slot (j + NSLOT - 1) % NSLOT held unit j - 1, whose bytes are consumed
        if (j + NSLOT - 1 < my_units) issue(j + NSLOT - 1);
        const int64_t ahead = my_units - 1 - j;
        if (ahead >= NSLOT - 1) wait_vmcnt<(NSLOT - 1) * CH>();
        else if (NSLOT > 2 && ahead == 1) wait_vmcnt<CH>();
        else wait_vmcnt<0>();
        const int st = XREG ? 0 : static_cast<int>(j % nsteps);
        const uint8_t *slot = slots + static_cast<int>(j % NSLOT) * SLOT;
        int b = st * F::BPS + F::blk_of(lane);
        const bool ok = b < nb;
        if (b > nb - per_lane) b = nb - per_lane;
        const int lb = b - st * F::BPS;
        uint32_t raw[RB][F::NRAW];
#pragma unroll
        for (int r = 0; r < RB; r++) F::load(raw[r], slot + r * P + lb * BB, slot_lane);
        float d[RB];
        if constexpr (XREG) {
#pragma unroll
            for (int r = 0; r < RB; r++) d[r] = F::dot(raw[r], slot_lane, xv, xg);
        } else {
            const int b0 = ok ? st * F::BPS * BV + XRuns<DT>::base(lane) : 0;
            if (xs_step != st) {
                D::sums(xl, b0, xs);
                xs_step = nsteps > 1 ? -1 : st;
            }
            D::run(raw, slot_lane, xl, b0, xs, d);
        }
#pragma unroll
        for (int r = 0; r < RB; r++) v[r] += ok ? d[r] : 0.0f;
        if (XREG || st == nsteps - 1) {
            const int64_t g = W + (j / nsteps) * NW;
            const int si = seg_of(g);
            const int64_t n0 = (g - segl[si].blk_begin) * RB;
            wave_reduce_multi<RB>(v, lane);
            if (reduce_owner<RB>(lane)) {
                const int64_t n = n0 + reduce_owner_index<RB>(lane);
                const int kind = segl[si].kind;
                if (n < segl[si].n_out)
                    store_out<OT>(static_cast<OT *>(segl[si].out) + n, v[0], kind,
                                  kind == SEG_ACC ? inv_acc : 1.0f);
            }
#pragma unroll
            for (int r = 0; r < RB; r++) v[r] = 0.0f;
        }
    }
}

template <int DT, typename XT, typename OT, int RB, int NSLOT, bool XREG>
static hipError_t launch_stream(SegTable t, hipStream_t st) {
    constexpr int SLOT = ((RB * WaveFmt<DT>::BPS * blk_bytes(DT) + 1023) / 1024) * 1024;
    int64_t total = 0;
    for (int i = 0; i < t.n; i++) {
        t.seg[i].blk_begin = total;
        total += (t.seg[i].n_out + RB - 1) / RB;
    }
    const int xfloats = XREG ? 0 : (t.n_in + 4 * (t.n_in / 64) + 4 + 3) & ~3;
    const size_t xbytes = static_cast<size_t>(xfloats) * sizeof(float);
    const size_t per_wave = static_cast<size_t>(NSLOT) * SLOT;
    // waves per workgroup: the most resident waves per CU, ties to the
    // larger workgroup (fewer x stagings); occupancy per shape is cached
    struct Pick { int n_in, nw, per_cu; };
    static thread_local Pick cache[8] = {};
    int nw = 0, per_cu = 0;
    for (const Pick &c : cache)
        if (c.nw && c.n_in == (XREG ? 0 : t.n_in)) { nw = c.nw; per_cu = c.per_cu; break; }
    if (!nw) {
        int best = 0;
        for (int cand = 1; cand <= 8; cand++) {
            const size_t lds = xbytes + cand * per_wave;
            if (lds + sizeof(Seg) * kMaxSegs > 160u * 1024u) break;
            int blocks = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                    &blocks, gemv_valu_kernel<DT, XT, OT, RB, NSLOT, XREG>, 64 * cand, lds) != hipSuccess)
                blocks = 0;
            if (blocks * cand >= best && blocks > 0) { best = blocks * cand; nw = cand; per_cu = blocks; }
        }
        if (!nw) return hipErrorInvalidValue;
        for (Pick &c : cache)
            if (!c.nw) { c = Pick{XREG ? 0 : t.n_in, nw, per_cu}; break; }
    }
    static thread_local int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cus = 256;
    }
    int64_t grid = static_cast<int64_t>(cus) * per_cu;
    if (grid * nw > total) grid = (total + nw - 1) / nw;
    hipLaunchKernelGGL((gemv_valu_kernel<DT, XT, OT, RB, NSLOT, XREG>), dim3(static_cast<unsigned>(grid)),
                       dim3(64 * nw), xbytes + nw * per_wave, st, t, total, xfloats);
    return hipGetLastError();
}

// two rows per unit, two slots: measured best over RB in {1, 2, 4} and
// two or three slots on MI355X for Q4_K / Q6_K / Q8_0 at K = 4096
template <int DT, typename XT, typename OT, bool XREG>
static hipError_t launch_stream_x(const SegTable &t, hipStream_t st) {
    return launch_stream<DT, XT, OT, 2, 2, XREG>(t, st);
}

template <int DT, typename XT, typename OT>
static hipError_t launch_stream(const SegTable &t, hipStream_t st) {
    return t.n_in <= WaveFmt<DT>::BPS * blk_vals(DT) ? launch_stream_x<DT, XT, OT, true>(t, st)
                                                     : launch_stream_x<DT, XT, OT, false>(t, st);
}

template <int DT, typename XT, typename OT>
static bool try_stream(const SegTable &t, hipStream_t st, hipError_t &err) {
    if (t.rows != 1 || t.n_in > 16384) return false;
    for (int i = 0; i < t.n; i++) {
        if (t.seg[i].kind == SEG_SILU || t.seg[i].x != t.seg[0].x) return false;
        if (reinterpret_cast<uintptr_t>(t.seg[i].w) & 15) return false;
    }
    if ((blk_vals(DT) == 32) && t.n_in % 64) return false;
    if (t.row_bytes % 16) return false;
    err = launch_stream<DT, XT, OT>(t, st);
    return true;
}

constexpr int kLdsGemvMaxK = 16384;  // f32 x plus padding must fit in LDS

template <int DT, typename XT, typename OT, int RB>
static hipError_t launch_lds(SegTable t, hipStream_t st) {
    int64_t total = 0;
    for (int i = 0; i < t.n; i++) {
        t.seg[i].blk_begin = total;
        const int64_t per = t.seg[i].kind == SEG_SILU ? RB / 2 : RB;
        total += (t.seg[i].n_out + per - 1) / per;
    }
    const size_t lds = static_cast<size_t>(t.n_in + 4 * (t.n_in / 64) + 4) * sizeof(float);
    static thread_local int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cus = 256;
    }
    // resident workgroups per CU, queried once per distinct LDS size
    static thread_local size_t cached_lds[8] = {};
    static thread_local int cached_occ[8] = {};
    int per_cu = 0;
    for (int i = 0; i < 8 && cached_lds[i]; i++)
        if (cached_lds[i] == lds) { per_cu = cached_occ[i]; break; }
    if (!per_cu) {
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_lds_kernel<DT, XT, OT, RB>, 256,
                                                         lds) != hipSuccess || per_cu < 1)
            per_cu = 1;
        for (int i = 0; i < 8; i++)
            if (!cached_lds[i]) { cached_lds[i] = lds; cached_occ[i] = per_cu; break; }
    }
    int64_t grid = static_cast<int64_t>(cus) * per_cu;
    if (grid * 4 > total) grid = (total + 3) / 4;
    hipLaunchKernelGGL((gemv_lds_kernel<DT, XT, OT, RB>), dim3(static_cast<unsigned>(grid)), dim3(256),
                       lds, st, t, total);
    return hipGetLastError();
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

template <int DT, typename XT, typename OT, int RB>
static hipError_t launch_persist(SegTable t, hipStream_t st) {
    int64_t total = 0;
    for (int i = 0; i < t.n; i++) {
        t.seg[i].blk_begin = total;
        const int64_t per = t.seg[i].kind == SEG_SILU ? RB / 2 : RB;
        total += (t.seg[i].n_out + per - 1) / per;
    }
    const int nsteps = (t.n_in / blk_vals(DT) + kWave / LaneFmt<DT>::LPB - 1) / (kWave / LaneFmt<DT>::LPB);
    const int threads = 64 * nsteps;
    // resident workgroups per CU for this instantiation and block size
    static thread_local int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cus = 256;
    }
    static thread_local int per_cu = 0;
    if (!per_cu && (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_persist_kernel<DT, XT, OT, RB>,
                                                                 threads, 0) != hipSuccess || per_cu < 1))
        per_cu = 1;
    int64_t grid = static_cast<int64_t>(cus) * per_cu;
    if (grid > total) grid = total;
    hipLaunchKernelGGL((gemv_persist_kernel<DT, XT, OT, RB>), dim3(static_cast<unsigned>(grid)),
                       dim3(threads), 0, st, t, total);
    return hipGetLastError();
}

// rows == 1 picks, in order: the LDS-DMA streamed kernel (one x for all
// segments, aligned rows); the x-in-LDS kernel (one x, e.g. fused gate+up
// with SiLU); the independent-wave kernel (one x per segment); the
// persistent kernel.  rows > 1 takes the multi-row segment kernel.
template <int DT, typename XT, typename OT>
static hipError_t dispatch_mr(SegTable t, hipStream_t st) {
    if (t.rows == 1) {
        const bool two_blocks = blk_vals(DT) == 32;
        hipError_t err = hipSuccess;
        if (try_stream<DT, XT, OT>(t, st, err)) return err;
        bool same_x = true;
        for (int i = 1; i < t.n; i++) same_x = same_x && t.seg[i].x == t.seg[0].x;
        if (same_x && t.n_in <= kLdsGemvMaxK && (!two_blocks || t.n_in % 64 == 0))
            return launch_lds<DT, XT, OT, 4>(t, st);
        if (!two_blocks || t.n_in % 64 == 0) return launch_wave<DT, XT, OT, 4>(t, st);
        const int nsteps = (t.n_in / blk_vals(DT) + kWave / LaneFmt<DT>::LPB - 1) /
                           (kWave / LaneFmt<DT>::LPB);
        if (nsteps <= 8) return launch_persist<DT, XT, OT, 4>(t, st);
    }
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

// Generic-chunk formats: the multi-row segment kernel over the chunk lane
// view, for every row count (no format-specific streaming kernels).
template <int DT, typename XT, typename OT>
static hipError_t dispatch_chunk(SegTable t, hipStream_t st) {
    const int mr = t.rows <= 1 ? 1 : t.rows == 2 ? 2 : 4;
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
#define KRK_CHUNK_CASE(D) \
    case D: return dispatch_chunk<D, XT, OT>(t, st);
        KRK_CHUNK_FORMATS(KRK_CHUNK_CASE)
#undef KRK_CHUNK_CASE
        case DT_Q4_K: return dispatch_mr<DT_Q4_K, XT, OT>(t, st);
        case DT_Q5_K: return dispatch_mr<DT_Q5_K, XT, OT>(t, st);
        case DT_Q6_K: return dispatch_mr<DT_Q6_K, XT, OT>(t, st);
        case DT_Q4_0: return dispatch_mr<DT_Q4_0, XT, OT>(t, st);
        case DT_IQ4_NL: return dispatch_mr<DT_IQ4_NL, XT, OT>(t, st);
        case DT_IQ4_XS: return dispatch_mr<DT_IQ4_XS, XT, OT>(t, st);
        case DT_Q2_K: return dispatch_mr<DT_Q2_K, XT, OT>(t, st);
        case DT_Q3_K: return dispatch_mr<DT_Q3_K, XT, OT>(t, st);
        case DT_MXFP4: return dispatch_mr<DT_MXFP4, XT, OT>(t, st);
        case DT_Q4_1: return dispatch_mr<DT_Q4_1, XT, OT>(t, st);
        case DT_Q5_0: return dispatch_mr<DT_Q5_0, XT, OT>(t, st);
        case DT_Q5_1: return dispatch_mr<DT_Q5_1, XT, OT>(t, st);
        case DT_F16: return dispatch_mr<DT_F16, XT, OT>(t, st);
        case DT_BF16: return dispatch_mr<DT_BF16, XT, OT>(t, st);
        case DT_Q8_0: return dispatch_mr<DT_Q8_0, XT, OT>(t, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t gemv_segments(int dt, bool act_f16, const SegTable &t, hipStream_t st) {
    if (gemv_stream_ok(dt, t)) return gemv_stream(dt, act_f16, t, st);
    if (gemv_digits_ok(dt, t)) return gemv_digits(dt, act_f16, t, st);
    if (act_f16) return dispatch_dt<_Float16, _Float16>(dt, t, st);
    return dispatch_dt<float, float>(dt, t, st);
}

}  // namespace krk
