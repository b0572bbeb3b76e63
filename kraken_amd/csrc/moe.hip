// moe.hip -- the routed-expert FFN of one layer from device ids, through the
// device pointer table (Backend::moe_dispatch, backend.hpp:1001-1009; the
// reference's moe_table_* kernels, src/hip/kernels/moe_table.hpp:38-551).
//
// Q4_K banks with f32 activations run on the int8 matrix cores (digit-plane
// activations): one token takes two launches of the register-streaming
// GEMV (gate/up per slot, down over the concatenated slots); more tokens
// take the plan, then expert-major runs of the same kernel -- one grid row
// per active expert, whose banks are loaded once and applied to each of its
// tokens in turn -- for gate/up and for down, then the ordered reduce (step 4
// below).  Other f32 cases: one token takes two VALU launches; more tokens
// take the plan path, none of its launches per expert and none waiting on
// the host:
//   1. plan      one workgroup: expert-major plan of the (token, slot) pairs,
//                the active-expert list in ascending id (with each expert's
//                banks and plan range), and each pair's plan position;
//   2. gate/up   ONE launch over all active experts: workgroup = (expert,
//                group of ff rows); its pairs' activation rows are gathered
//                through the plan and share every weight byte read;
//                mid = silu(gate . x) * (up . x) in f32;
//   3. down      ONE launch over all active experts, part = down . mid;
//   4. reduce    out[t] = sum over t's pairs in ascending expert id of
//                fma(w, part, acc) -- the order and the fused add of the host
//                loop (engine.cpp:12360-12700, scatter_axpy_rows
//                backend_cpu.cpp:3193-3217).
// f16 activations (the reference GPU backend's act_type) take the plan path
// at every token count with the reference GPU's rounding points
// (moe_table.hpp:250-305, 418-441, 536-551): gate/up dots rounded to f16
// before silu, a row-scale pass (power of two keeping the row within f16,
// midf = f16(mid / scale)), down on midf, and a reduce that adds
// w * (f16(v) * scale) per slot in slot order with an f16 rounding after
// every add.
// The weight types and strides are read from the table on the device, per
// expert and matrix.  Layers whose types vary from expert to expert, or whose
// gate and up types differ, take the VALU kernels, whose row GEMV switches on
// each expert's types.
#include "gemv_core.hpp"
#include "krk_mi355x.h"

// every weight type an expert bank may hold (the backend validates the table
// before any launch; an unknown type never reaches these switches)
#define KRK_MOE_TYPES(X, T, A)                                                                  \
    X(DT_Q4_K, T, A) X(DT_Q6_K, T, A) X(DT_Q4_0, T, A) X(DT_Q8_0, T, A) X(DT_Q5_K, T, A)      \
    X(DT_Q2_K, T, A) X(DT_Q3_K, T, A) X(DT_IQ4_NL, T, A) X(DT_IQ4_XS, T, A) X(DT_MXFP4, T, A) \
    X(DT_Q4_1, T, A) X(DT_Q5_0, T, A) X(DT_Q5_1, T, A) X(DT_F16, T, A) X(DT_BF16, T, A)        \
    X(DT_Q8_1, T, A) X(DT_Q8_K, T, A) X(DT_TQ1_0, T, A) X(DT_TQ2_0, T, A) X(DT_NVFP4, T, A)    \
    X(DT_ROCMFP4, T, A) X(DT_ROCMFP4_FAST, T, A) X(DT_Q6_0_ROCMFPX, T, A)                     \
    X(DT_Q3_0_ROCMFPX, T, A) X(DT_Q2_0_ROCMFPX, T, A) X(DT_Q1_0, T, A) X(DT_Q2_0, T, A)      \
    X(DT_Q2_0_64, T, A) X(DT_PQ2_0, T, A) X(DT_PTQ1_0, T, A)
#define KRK_MOE_UNPAREN(...) __VA_ARGS__
#define KRK_MOE_ROWS(D, T, A) \
    case D: gemv_rows<D, KRK_MOE_UNPAREN T>(KRK_MOE_UNPAREN A); break;

namespace krk {

struct MoeWs {
    int32_t *off;       // [n_expert + 1]
    int32_t *act;       // [n_expert]     active experts, ascending
    int32_t *n_act;     // [1]
    int32_t *plan_tok;  // [P]            token of plan position
    int32_t *plan_pos;  // [P]            plan position of pair t*k+s (-1: dropped)
    float *mid;         // [P, n_ff]
    float *part;        // [P, n_embd]
    int32_t *items;     // [P][4]         {expert, first plan position, rows <= kItemRows, 0}
    int32_t *n_items;   // [1]
    _Float16 *midf;     // [P, n_ff]      f16 activations: the row-scaled mid rows
    float *rscale;      // [P]            f16 activations: each mid row's power-of-two scale
    EmRun *runs;        // [n_expert]     active experts' banks and plan ranges
    _Float16 *xg;       // [P, n_embd]    grouped GEMM: the tokens' activation rows, f16
};

static size_t al(size_t v) { return (v + 255) & ~size_t(255); }

static MoeWs carve(void *ws, int64_t P, int ne, int64_t n_embd, int64_t n_ff) {
    uint8_t *p = static_cast<uint8_t *>(ws);
    MoeWs w;
    w.off = reinterpret_cast<int32_t *>(p); p += al((ne + 1) * 4);
    w.act = reinterpret_cast<int32_t *>(p); p += al(ne * 4);
    w.n_act = reinterpret_cast<int32_t *>(p); p += al(4);
    w.plan_tok = reinterpret_cast<int32_t *>(p); p += al(P * 4);
    w.plan_pos = reinterpret_cast<int32_t *>(p); p += al(P * 4);
    w.mid = reinterpret_cast<float *>(p); p += al(P * n_ff * 4);
    w.part = reinterpret_cast<float *>(p); p += al(P * n_embd * 4);
    w.items = reinterpret_cast<int32_t *>(p); p += al(P * 16);
    w.n_items = reinterpret_cast<int32_t *>(p); p += al(4);
    w.midf = reinterpret_cast<_Float16 *>(p); p += al(P * n_ff * 2);
    w.rscale = reinterpret_cast<float *>(p); p += al(P * 4);
    w.runs = reinterpret_cast<EmRun *>(p); p += al(ne * sizeof(EmRun));
    w.xg = reinterpret_cast<_Float16 *>(p);
    return w;
}

size_t moe_workspace(int64_t n_tok, int k, int n_expert, int64_t n_embd, int64_t n_ff) {
    const int64_t P = n_tok * k;
    return al((n_expert + 1) * 4) + al(n_expert * 4) + al(4) + 2 * al(P * 4) +
           al(P * n_ff * 4) + al(P * n_embd * 4) + al(P * 16) + al(4) + al(P * n_ff * 2) + al(P * 4) +
           al(n_expert * sizeof(EmRun)) + al(P * n_embd * 2);
}

// ------------------------------------------------------------------ plan ----
// Pairs of one expert are computed independently of one another, so their
// order inside the expert's range does not change any result; placement
// takes a per-expert atomic cursor.  The expert offsets and the active list
// come from a block-wide exclusive scan (4 experts per thread).
constexpr int kPlanLds = 4096;  // (token, slot) pairs whose ids the plan keeps in LDS
constexpr int kItemRows = 2;    // plan item rows of the VALU expert kernels
__global__ void __launch_bounds__(256) moe_plan_kernel(const int32_t *__restrict__ ids, int64_t P,
                                                        int k, int ne, MoeWs w,
                                                        const krk_moe_entry *__restrict__ tab,
                                                        int item_rows) {
    __shared__ int32_t cnt[1024];
    __shared__ int32_t cur[1024];
    __shared__ int32_t sid[kPlanLds];   // the ids, when they fit
    __shared__ int32_t wsum[3][4];      // per-wave totals: pairs, active experts, items
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const bool in_lds = P <= kPlanLds;
    for (int e = tid; e < ne; e += blockDim.x) cnt[e] = 0;
    if (in_lds)
        for (int64_t i = tid; i < P; i += blockDim.x) sid[i] = ids[i];
    __syncthreads();
    auto id_at = [&](int64_t i) { return in_lds ? sid[i] : ids[i]; };
    for (int64_t i = tid; i < P; i += blockDim.x) {
        const int e = id_at(i);
        if (e >= 0 && e < ne) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // exclusive scan over experts 4 tid .. 4 tid + 3 (ne <= 1024)
    // items: each active expert's pairs in runs of up to item_rows (the rows
    // one pass of the digit kernel or the grouped GEMM takes)
    int c[4], run = 0, act = 0, its = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = 4 * tid + j;
        c[j] = e < ne ? cnt[e] : 0;
        run += c[j];
        act += c[j] > 0;
        its += (c[j] + item_rows - 1) / item_rows;
    }
    int ir = run, ia = act, ii = its;   // inclusive wave scans
    for (int d = 1; d < 64; d <<= 1) {
        const int orr = __shfl_up(ir, d, 64), oa = __shfl_up(ia, d, 64), oi = __shfl_up(ii, d, 64);
        if (lane >= d) { ir += orr; ia += oa; ii += oi; }
    }
    if (lane == 63) { wsum[0][wv] = ir; wsum[1][wv] = ia; wsum[2][wv] = ii; }
    __syncthreads();
    int base = ir - run, abase = ia - act, ibase = ii - its;
    for (int v = 0; v < wv; v++) { base += wsum[0][v]; abase += wsum[1][v]; ibase += wsum[2][v]; }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e = 4 * tid + j;
        if (e < ne) {
            w.off[e] = base;
            cur[e] = base;
            if (c[j]) {
                // the run record: the expert's banks and plan range in one place
                EmRun &r = w.runs[abase];
                r.w[0] = tab[e].p[KRK_MOE_GATE];
                r.w[1] = tab[e].p[KRK_MOE_UP];
                r.w[2] = tab[e].p[KRK_MOE_DOWN];
                r.pb = base;
                r.pe = base + c[j];
                w.act[abase++] = e;
            }
            for (int r = 0; r < c[j]; r += item_rows) {
                int32_t *it = w.items + 4 * ibase++;
                it[0] = e;
                it[1] = base + r;
                it[2] = c[j] - r < item_rows ? c[j] - r : item_rows;
                it[3] = 0;
            }
        }
        base += c[j];
    }
    if (tid == blockDim.x - 1) {
        w.off[ne] = base;   // the last thread's running total is the grand total
        w.n_act[0] = abase;
        w.n_items[0] = ibase;
    }
    __syncthreads();
    for (int64_t i = tid; i < P; i += blockDim.x) {
        const int e = id_at(i);
        if (e < 0 || e >= ne) {
            w.plan_pos[i] = -1;
            continue;
        }
        const int pos = atomicAdd(&cur[e], 1);
        w.plan_tok[pos] = static_cast<int32_t>(i / k);
        w.plan_pos[i] = pos;
    }
}

// The expert's activation row.  f32 activations (the CPU oracle's
// act_type): silu_mul, backend_cpu.cpp:2401-2406.  f16 activations (the
// reference GPU backend's): both dots rounded to f16 first and silu with the
// device exponential (moe_table.hpp:250-253, krk_hip.hpp:130).
template <typename XT>
__device__ __forceinline__ float gate_act(float g, float u) {
    if constexpr (sizeof(XT) == 2) {
        const float gf = static_cast<float>(static_cast<_Float16>(g));
        const float uf = static_cast<float>(static_cast<_Float16>(u));
        return silu_f(gf) * uf;
    } else {
        return (g / (1.0f + expf(-g))) * u;
    }
}

// Gate rows n0 .. n0 + RB/2 - 1 of an expert into acc[.][0, RB/2) and the
// same up rows into acc[.][RB/2, RB): one pass when gate and up share a type
// (each weight unit's activations loaded once for both), two otherwise.
template <typename XT, int MR, int RB>
__device__ __forceinline__ void gate_up_rows(const krk_moe_entry &en, int64_t n_ff, int n_embd,
                                             const XT *const (&xr)[MR], int64_t n0, float (&acc)[MR][RB]) {
    const uint8_t *wg = static_cast<const uint8_t *>(en.p[KRK_MOE_GATE]);
    const uint8_t *wu = static_cast<const uint8_t *>(en.p[KRK_MOE_UP]);
    if (en.type[KRK_MOE_GATE] == en.type[KRK_MOE_UP]) {
        switch (en.type[KRK_MOE_GATE]) {
            KRK_MOE_TYPES(KRK_MOE_ROWS, (XT, MR, RB), (wg, en.row_bytes[0], n_ff, n_embd, xr, n0, wu, acc))
            default: break;
        }
        return;
    }
    constexpr int H = RB / 2;
    float h[MR][H];
    switch (en.type[KRK_MOE_GATE]) {
        KRK_MOE_TYPES(KRK_MOE_ROWS, (XT, MR, H), (wg, en.row_bytes[0], n_ff, n_embd, xr, n0, nullptr, h))
        default: break;
    }
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int r = 0; r < H; r++) acc[m][r] = h[m][r];
    switch (en.type[KRK_MOE_UP]) {
        KRK_MOE_TYPES(KRK_MOE_ROWS, (XT, MR, H), (wu, en.row_bytes[1], n_ff, n_embd, xr, n0, nullptr, h))
        default: break;
    }
#pragma unroll
    for (int m = 0; m < MR; m++)
#pragma unroll
        for (int r = 0; r < H; r++) acc[m][H + r] = h[m][r];
}

// -------------------------------------------------------------- gate/up ----
template <typename XT, int MR, int RB>
__global__ void __launch_bounds__(512) moe_gu_kernel(const krk_moe_entry *__restrict__ tab,
                                                      const XT *__restrict__ xn, int64_t n_embd,
                                                      int64_t n_ff, int64_t groups, MoeWs w) {
    __shared__ float red[8][MR * RB];
    constexpr int H = RB / 2;
    // persistent: items (active expert, row group) in expert-major order; the
    // first item past the active experts ends the walk
    const int64_t items = static_cast<int64_t>(w.n_act[0]) * groups;
    for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
    const int64_t a = item / groups, g = item % groups;
    const int e = w.act[a];
    const krk_moe_entry &en = tab[e];
    const int64_t n0 = g * H;
    const int p0 = w.off[e], np = w.off[e + 1] - p0;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int pass = 0; pass < np; pass += MR) {
        const XT *xr[MR];
#pragma unroll
        for (int m = 0; m < MR; m++)
            xr[m] = pass + m < np ? xn + static_cast<int64_t>(w.plan_tok[p0 + pass + m]) * n_embd
                                  : nullptr;
        float acc[MR][RB];
        gate_up_rows<XT, MR, RB>(en, n_ff, static_cast<int>(n_embd), xr, n0, acc);
        float v[MR * RB];
#pragma unroll
        for (int m = 0; m < MR; m++)
#pragma unroll
            for (int r = 0; r < RB; r++) v[m * RB + r] = acc[m][r];
        wave_reduce_multi<MR * RB>(v, lane);
        if (reduce_owner<MR * RB>(lane)) red[wv][reduce_owner_index<MR * RB>(lane)] = v[0];
        __syncthreads();
        const int tid = threadIdx.x;
        if (tid < MR * H) {
            const int m = tid / H, r = tid % H;
            float gs = 0.0f, us = 0.0f;
            for (int kk = 0; kk < nw; kk++) {
                gs += red[kk][m * RB + r];
                us += red[kk][m * RB + H + r];
            }
            const int64_t n = n0 + r;
            if (pass + m < np && n < n_ff)
                w.mid[static_cast<int64_t>(p0 + pass + m) * n_ff + n] = gate_act<XT>(gs, us);
        }
        __syncthreads();
    }
    }
}

// ----------------------------------------------------------------- down ----
template <typename MT, int MR, int RB>
__global__ void __launch_bounds__(512) moe_down_kernel(const krk_moe_entry *__restrict__ tab,
                                                        int64_t n_embd, int64_t n_ff,
                                                        int64_t groups, MoeWs w) {
    // MT: the activation rows' type -- float mid, or the f16 row-scaled midf
    __shared__ float red[8][MR * RB];
    const int64_t items = static_cast<int64_t>(w.n_act[0]) * groups;
    for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
    const int64_t a = item / groups, g = item % groups;
    const int e = w.act[a];
    const krk_moe_entry &en = tab[e];
    const int64_t n0 = g * RB;
    const int p0 = w.off[e], np = w.off[e + 1] - p0;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const uint8_t *wd = static_cast<const uint8_t *>(en.p[KRK_MOE_DOWN]);
    for (int pass = 0; pass < np; pass += MR) {
        const MT *rows = sizeof(MT) == 2 ? reinterpret_cast<const MT *>(w.midf) : reinterpret_cast<const MT *>(w.mid);
        const MT *xr[MR];
#pragma unroll
        for (int m = 0; m < MR; m++)
            xr[m] = pass + m < np ? rows + static_cast<int64_t>(p0 + pass + m) * n_ff : nullptr;
        float acc[MR][RB];
        switch (en.type[KRK_MOE_DOWN]) {
            KRK_MOE_TYPES(KRK_MOE_ROWS, (MT, MR, RB), (wd, en.row_bytes[2], n_embd, (int)n_ff, xr, n0, nullptr, acc))
            default: break;
        }
        float v[MR * RB];
#pragma unroll
        for (int m = 0; m < MR; m++)
#pragma unroll
            for (int r = 0; r < RB; r++) v[m * RB + r] = acc[m][r];
        wave_reduce_multi<MR * RB>(v, lane);
        if (reduce_owner<MR * RB>(lane)) red[wv][reduce_owner_index<MR * RB>(lane)] = v[0];
        __syncthreads();
        const int tid = threadIdx.x;
        if (tid < MR * RB) {
            const int m = tid / RB, r = tid % RB;
            float sum = 0.0f;
            for (int kk = 0; kk < nw; kk++) sum += red[kk][tid];
            const int64_t n = n0 + r;
            if (pass + m < np && n < n_embd)
                w.part[static_cast<int64_t>(p0 + pass + m) * n_embd + n] = sum;
        }
        __syncthreads();
    }
    }
}

// ---------------------------------------------------- f16 row scale ----
// f16 activations: each live mid row's power-of-two scale and the f16 row
// the down dot reads (moe_table_scale_kernel, moe_table.hpp:256-305): the
// smallest scale >= 1 (at most 2^24) with max |mid| <= 65504 * scale, and
// midf = f16(mid * (1 / scale)), the reciprocal exact.  One workgroup per
// plan position; positions past the live pairs leave at once.
__global__ void __launch_bounds__(256) moe_scale_kernel(int64_t n_ff, int ne, MoeWs w) {
    __shared__ float red[4];
    const int64_t p = blockIdx.x;
    if (p >= w.off[ne]) return;
    const float *row = w.mid + p * n_ff;
    float mx = 0.0f;
    for (int64_t j = threadIdx.x; j < n_ff; j += blockDim.x) mx = fmaxf(mx, fabsf(row[j]));
    for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float mul = 1.0f;
    while (m > 65504.0f * mul && mul < 16777216.0f) mul *= 2.0f;
    if (threadIdx.x == 0) w.rscale[p] = mul;
    const float inv = 1.0f / mul;
    for (int64_t j = threadIdx.x; j < n_ff; j += blockDim.x)
        w.midf[p * n_ff + j] = static_cast<_Float16>(__fmul_rn(row[j], inv));
}

// f16 activations: the reference GPU's slot-order accumulation
// (moe_table_reduce_kernel, moe_table.hpp:536-551, with the partial of
// table_down_batch, 418-441): per slot s in order, part = w * (f16(v) *
// scale), two round-to-nearest products, and a = f16(a + part); a dropped
// slot adds nothing (a is already an f16 value).
__global__ void __launch_bounds__(256) moe_reduce_f16_kernel(const float *__restrict__ wts, int k,
                                                             int64_t n_embd, MoeWs w,
                                                             _Float16 *__restrict__ out) {
    const int64_t t = blockIdx.y;
    const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (j >= n_embd) return;
    float a = 0.0f;
    for (int s = 0; s < k; s++) {
        const int pos = w.plan_pos[t * k + s];
        if (pos < 0) continue;
        const float vf = static_cast<float>(static_cast<_Float16>(w.part[static_cast<int64_t>(pos) * n_embd + j]));
        const float part = __fmul_rn(wts[t * k + s], __fmul_rn(vf, w.rscale[pos]));
        a = static_cast<float>(static_cast<_Float16>(__fadd_rn(a, part)));
    }
    out[t * n_embd + j] = static_cast<_Float16>(a);
}

// --------------------------------------------------------------- reduce ----
template <typename OT>
__global__ void __launch_bounds__(256) moe_reduce_kernel(const int32_t *__restrict__ ids,
                                                         const float *__restrict__ wts, int k,
                                                         int64_t n_embd, MoeWs w,
                                                         OT *__restrict__ out) {
    // this token's live pairs in ascending expert id (ties, which the router
    // never makes, in slot order; k <= 64), then every thread adds its
    // column in that order
    __shared__ int32_t ord_pos[64];
    __shared__ float ord_w[64];
    __shared__ int32_t s_pos[64], s_id[64];
    __shared__ float s_w[64];
    __shared__ int nlive;
    const int64_t t = blockIdx.y;
    if (threadIdx.x < k) {   // the token's pairs, one load round
        s_pos[threadIdx.x] = w.plan_pos[t * k + threadIdx.x];
        s_id[threadIdx.x] = ids[t * k + threadIdx.x];
        s_w[threadIdx.x] = wts[t * k + threadIdx.x];
    }
    __syncthreads();
    // rank of each live pair among the token's live pairs by (expert id,
    // slot): one thread per slot, no private arrays
    if (threadIdx.x < k && s_pos[threadIdx.x] >= 0) {
        const int me = threadIdx.x, e = s_id[me];
        int q = 0;
        for (int s = 0; s < k; s++)
            q += s_pos[s] >= 0 && (s_id[s] < e || (s_id[s] == e && s < me));
        ord_pos[q] = s_pos[me];
        ord_w[q] = s_w[me];
    }
    if (threadIdx.x == 0) {
        int n = 0;
        for (int s = 0; s < k; s++) n += s_pos[s] >= 0;
        nlive = n;
    }
    __syncthreads();
    const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (j >= n_embd) return;
    const int n = nlive;
    float acc = 0.0f;
    for (int q = 0; q < n; q++)
        acc = __builtin_fmaf(ord_w[q], w.part[static_cast<int64_t>(ord_pos[q]) * n_embd + j], acc);
    out[t * n_embd + j] = static_cast<OT>(acc);
}

// ------------------------------------------------------- one token ----
// Decode (n_tok == 1) needs no plan: the token's experts are ids[0..k-1].
// Two launches: gate/up per (slot, row group) into mid[slot], then the down
// projections fused with the reduction -- a workgroup owns RB output rows
// and walks the token's experts in ascending id, adding fma(w, part, acc)
// in that order (the host loop's order), so no per-slot partials are stored
// and no reduce launch follows.
template <typename XT, int RB>
__global__ void __launch_bounds__(512) moe_gu1_kernel(const krk_moe_entry *__restrict__ tab,
                                                       const int32_t *__restrict__ ids, int k, int ne,
                                                       const XT *__restrict__ xn, int64_t n_embd,
                                                       int64_t n_ff, int64_t groups, float *__restrict__ mid) {
    __shared__ float red[8][RB];
    constexpr int H = RB / 2;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int64_t items = static_cast<int64_t>(k) * groups;
    for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
        const int s = static_cast<int>(item / groups);
        const int64_t n0 = (item % groups) * H;
        const int e = ids[s];
        if (e < 0 || e >= ne) continue;   // a dropped slot (uniform per workgroup)
        const krk_moe_entry &en = tab[e];
        const XT *xr[1] = {xn};
        float acc[1][RB];
        gate_up_rows<XT, 1, RB>(en, n_ff, static_cast<int>(n_embd), xr, n0, acc);
        float v[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) v[r] = acc[0][r];
        wave_reduce_multi<RB>(v, lane);
        if (reduce_owner<RB>(lane)) red[wv][reduce_owner_index<RB>(lane)] = v[0];
        __syncthreads();
        if (threadIdx.x < H) {
            const int r = threadIdx.x;
            float gs = 0.0f, us = 0.0f;
            for (int kk = 0; kk < nw; kk++) {
                gs += red[kk][r];
                us += red[kk][H + r];
            }
            const int64_t n = n0 + r;
            if (n < n_ff) mid[static_cast<int64_t>(s) * n_ff + n] = gate_act<XT>(gs, us);
        }
        __syncthreads();
    }
}

template <typename OT, int RB>
__global__ void __launch_bounds__(512) moe_down1_kernel(const krk_moe_entry *__restrict__ tab,
                                                         const int32_t *__restrict__ ids,
                                                         const float *__restrict__ wts, int k, int ne,
                                                         int64_t n_embd, int64_t n_ff, int64_t groups,
                                                         const float *__restrict__ mid, OT *__restrict__ out) {
    // wave q computes the RB rows for the token's q-th expert in ascending
    // id; the partials meet in LDS and one thread per row adds them in q order
    __shared__ float part[64][RB];
    __shared__ int ord[64];
    __shared__ int nlive;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (threadIdx.x == 0) {
        // the token's live slots in ascending expert id (insertion sort, k <= 64)
        int n = 0;
        for (int s = 0; s < k; s++) {
            const int e = ids[s];
            if (e < 0 || e >= ne) continue;
            int q = n++;
            while (q > 0 && ids[ord[q - 1]] > e) { ord[q] = ord[q - 1]; q--; }
            ord[q] = s;
        }
        nlive = n;
    }
    __syncthreads();
    const int nq = nlive;
    for (int64_t g = blockIdx.x; g < groups; g += gridDim.x) {
        const int64_t n0 = g * RB;
        for (int q = wv; q < nq; q += nw) {
            const int s = ord[q];
            const krk_moe_entry &en = tab[ids[s]];
            const float *xr[1] = {mid + static_cast<int64_t>(s) * n_ff};
            float a2[1][RB];
            const uint8_t *wd = static_cast<const uint8_t *>(en.p[KRK_MOE_DOWN]);
            switch (en.type[KRK_MOE_DOWN]) {
                KRK_MOE_TYPES(KRK_MOE_ROWS, (float, 1, RB), (wd, en.row_bytes[2], n_embd, (int)n_ff, xr, n0, nullptr, a2, 0, 1))
                default: break;
            }
            float v[RB];
#pragma unroll
            for (int r = 0; r < RB; r++) v[r] = a2[0][r];
            wave_reduce_multi<RB>(v, lane);
            if (reduce_owner<RB>(lane)) part[q][reduce_owner_index<RB>(lane)] = v[0];
        }
        __syncthreads();
        if (threadIdx.x < RB && n0 + threadIdx.x < n_embd) {
            float acc = 0.0f;
            for (int q = 0; q < nq; q++) acc = __builtin_fmaf(wts[ord[q]], part[q][threadIdx.x], acc);
            out[n0 + threadIdx.x] = static_cast<OT>(acc);
        }
        __syncthreads();
    }
}

constexpr int64_t kMoeTokenGroups = 64;
// f32 batches from this many tokens take the grouped expert GEMM when the
// gemm path allows f16 products
constexpr int64_t kMoeGemmTokens = 32;

hipError_t moe_dispatch(const MoeArgs &a, void *ws, size_t ws_bytes, hipStream_t st) {
    const int64_t P = a.n_tok * a.k;
    if (ws_bytes < moe_workspace(a.n_tok, a.k, a.n_expert, a.n_embd, a.n_ff)) return hipErrorInvalidValue;
    if (a.n_expert > 1024 || a.k > 64) return hipErrorInvalidValue;
    MoeWs w = carve(ws, P, a.n_expert, a.n_embd, a.n_ff);
    const krk_moe_entry *tab = static_cast<const krk_moe_entry *>(a.table) +
                               static_cast<int64_t>(a.layer) * a.n_expert;
    auto waves = [](int64_t K) {
        int64_t steps = (K / 32 + 63) / 64;  // 2048 values per wave step
        return static_cast<int>(steps < 1 ? 1 : steps > 8 ? 8 : steps);
    };
    const int wgu = waves(a.n_embd), wdn = waves(a.n_ff);
    // the active-expert count is known on the device only: launch a grid
    // the chip keeps resident and let the workgroups walk the items
    auto cap = [](int64_t want, int waves_per_wg) {
        const int64_t resident = 256LL * (32 / waves_per_wg);
        return dim3(static_cast<unsigned>(want < resident ? want : resident));
    };
    // The per-token tables (one token on the streaming kernel; token groups
    // on the digit kernel where the expert-major runs below do not apply),
    // the routed banks resolved on the device, one group of workgroups per
    // token:
    //   gate/up: one segment per slot, mid[t * k + s] = silu(g) * u;
    //   down:    one GEMV per token over its k slots concatenated, the
    //            routing weights folded into the activation scales, written
    //            straight to out[t].
    SegTable gu{};
    gu.n = a.k;
    gu.n_in = static_cast<int>(a.n_embd);
    gu.row_bytes = a.rb_gate;
    gu.rows = 1;
    gu.x_stride = a.n_embd;
    gu.out_stride = a.n_ff;
    gu.moe_tab = tab;
    gu.moe_ids = a.ids;
    gu.moe_ne = a.n_expert;
    gu.moe_tokens = static_cast<int>(a.n_tok);
    gu.moe_xtok = a.n_embd;
    gu.moe_otok = a.k * a.n_ff;
    for (int i = 0; i < a.k && i < kMaxSegs; i++) {
        gu.seg[i].x = a.xn;
        gu.seg[i].out = w.mid;
        gu.seg[i].n_out = a.n_ff;
        gu.seg[i].kind = SEG_SILU;
    }
    SegTable d{};
    d.n = 1;
    d.n_in = static_cast<int>(a.k * a.n_ff);
    d.row_bytes = a.rb_down;
    d.rows = 1;
    d.x_stride = d.n_in;
    d.out_stride = a.n_embd;
    d.seg[0].x = w.mid;
    d.seg[0].out = a.out;
    d.seg[0].n_out = a.n_embd;
    d.seg[0].kind = SEG_PLAIN;
    d.moe_tab = tab;
    d.moe_ids = a.ids;
    d.moe_wts = a.wts;
    d.moe_ne = a.n_expert;
    d.moe_down = 1;
    d.moe_k = a.k;
    d.moe_kslot = a.n_ff;
    d.moe_tokens = static_cast<int>(a.n_tok);
    d.moe_xtok = a.k * a.n_ff;
    d.moe_otok = a.n_embd;
    // Several tokens take expert-major runs of the streaming kernel (each
    // active expert's banks read once; measured 280 -> 256 us at 16 tokens and
    // about twice as fast as the digit kernel's items from 65 tokens up).
    // Where the streaming kernel cannot take the shapes, token groups of the
    // digit kernel serve up to kMoeTokenGroups tokens (each token reads its
    // experts for itself), and the plan path whatever the digit kernel
    // cannot take.  (The digit kernel's expert-major items, once the path
    // above 64 tokens, took exactly the shapes the streaming kernel takes
    // and were removed.)
    // Q4_K gate/up; the streaming kernel also takes a Q6_K down bank (Q4_K_M
    // layers), the digit kernel only Q4_K
    const bool q4k_gu = !a.act_f16 && a.wt == DT_Q4_K && a.aligned16 && a.rb_gate == a.rb_up &&
                        a.k <= kMaxSegs && a.k * a.n_ff <= (1 << 30);
    const bool on_digits = q4k_gu && a.wt_down == DT_Q4_K;
    const bool on_stream = q4k_gu && (a.wt_down == DT_Q4_K || a.wt_down == DT_Q6_K);
    const bool groups = on_digits && a.n_tok <= kMoeTokenGroups;
    const bool gu_ok = groups && gemv_digits_ok(DT_Q4_K, gu);
    const bool dn_ok = groups && gemv_digits_ok(DT_Q4_K, d);
    // Prefill-sized batches under a gemm path that allows f16 products: the
    // grouped expert GEMM (gemm.hip) over plan items of up to 32 mi pairs,
    // mi (1 or 2) from the mean pairs per active expert, then the ordered
    // reduce.
    // f16 operands and f32 accumulation, as the dense GEMM above 8 rows.
    if (a.mfma && !a.act_f16 && a.n_tok >= kMoeGemmTokens && a.aligned16 && a.wt >= 0 &&
        a.rb_gate == a.rb_up && moe_gemm_ok(a.wt) && moe_gemm_ok(a.wt_down) && P <= (1 << 24)) {
        const int64_t act = P < a.n_expert ? P : a.n_expert;
        const int64_t per = (P + act - 1) / act;
        const int mi = per <= 21 ? 1 : 2;
        hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(256), 0, st, a.ids, P, a.k, a.n_expert, w, tab,
                           32 * mi);
        MoeGemmArgs g{};
        g.tab = tab;
        g.items = w.items;
        g.n_items = w.n_items;
        const int64_t bound = act + P / (32 * mi);
        g.max_items = static_cast<int>(bound < P ? bound : P);
        g.mi = mi;
        // the tokens' rows as f16 once; gate/up reads each plan position's
        // row through plan_tok
        hipError_t e = moe_gather_f16(static_cast<const float *>(a.xn), a.n_embd, nullptr, nullptr, a.n_tok,
                                      w.xg, st);
        if (e != hipSuccess) return e;
        g.x = w.xg;
        g.xtok = w.plan_tok;
        g.out = w.midf;
        g.row_bytes = a.rb_gate;
        g.K = static_cast<int>(a.n_embd);
        g.N = static_cast<int>(a.n_ff);
        g.gate_up = true;
        e = moe_gemm(a.wt, g, st);
        if (e != hipSuccess) return e;
        g.x = w.midf;
        g.xtok = nullptr;
        g.out = w.part;
        g.row_bytes = a.rb_down;
        g.K = static_cast<int>(a.n_ff);
        g.N = static_cast<int>(a.n_embd);
        g.gate_up = false;
        e = moe_gemm(a.wt_down, g, st);
        if (e != hipSuccess) return e;
        const dim3 rgrid(static_cast<unsigned>((a.n_embd + 255) / 256), static_cast<unsigned>(a.n_tok));
        hipLaunchKernelGGL((moe_reduce_kernel<float>), rgrid, dim3(256), 0, st, a.ids, a.wts, a.k,
                           a.n_embd, w, static_cast<float *>(a.out));
        return hipGetLastError();
    }
    if (on_stream && a.n_tok >= 2) {
        // expert-major runs on the register-streaming kernel: one grid row
        // per active expert, whose weights are loaded once and applied to
        // each of its tokens in turn; then the ordered per-token reduce
        SegTable eg{};
        eg.n = 1;
        eg.n_in = static_cast<int>(a.n_embd);
        eg.row_bytes = a.rb_gate;
        eg.rows = 1;
        eg.seg[0].x = a.xn;
        eg.seg[0].out = w.mid;
        eg.seg[0].n_out = a.n_ff;
        eg.seg[0].kind = SEG_SILU;
        eg.moe_tab = tab;
        eg.moe_ne = a.n_expert;
        eg.em_runs = w.runs;
        eg.em_n_act = w.n_act;
        eg.em_tok = w.plan_tok;
        eg.em_max_items = static_cast<int>(P < a.n_expert ? P : a.n_expert);
        eg.em_xrow = a.n_embd;
        eg.em_orow = a.n_ff;
        SegTable ed = eg;
        ed.n_in = static_cast<int>(a.n_ff);
        ed.row_bytes = a.rb_down;
        ed.seg[0].x = w.mid;
        ed.seg[0].out = w.part;
        ed.seg[0].n_out = a.n_embd;
        ed.seg[0].kind = SEG_PLAIN;
        ed.em_tok = nullptr;
        ed.em_xrow = a.n_ff;
        ed.em_orow = a.n_embd;
        if (gemv_stream_ok(DT_Q4_K, eg) && gemv_stream_ok(a.wt_down, ed)) {
            hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(256), 0, st, a.ids, P, a.k, a.n_expert, w, tab,
                           kItemRows);
            hipError_t e = gemv_stream(DT_Q4_K, false, eg, st);
            if (e == hipSuccess) e = gemv_stream(a.wt_down, false, ed, st);
            if (e != hipSuccess) return e;
            const dim3 rgrid(static_cast<unsigned>((a.n_embd + 255) / 256), static_cast<unsigned>(a.n_tok));
            hipLaunchKernelGGL((moe_reduce_kernel<float>), rgrid, dim3(256), 0, st, a.ids, a.wts, a.k,
                               a.n_embd, w, static_cast<float *>(a.out));
            return hipGetLastError();
        }
    }
    if (on_stream && !on_digits && a.n_tok == 1 && gemv_stream_ok(DT_Q4_K, gu) && gemv_stream_ok(a.wt_down, d)) {
        // one token of a Q4_K_M layer: both launches on the streaming kernel
        const hipError_t e = gemv_stream(DT_Q4_K, false, gu, st);
        if (e != hipSuccess) return e;
        return gemv_stream(a.wt_down, false, d, st);
    }
    if (gu_ok && (dn_ok || a.n_tok == 1)) {
        // one token: the register-streaming kernel where it takes the shapes
        const bool gu_s = a.n_tok == 1 && gemv_stream_ok(DT_Q4_K, gu);
        const bool dn_s = a.n_tok == 1 && dn_ok && gemv_stream_ok(DT_Q4_K, d);
        const hipError_t e = gu_s ? gemv_stream(DT_Q4_K, false, gu, st) : gemv_digits(DT_Q4_K, false, gu, st);
        if (e != hipSuccess) return e;
        if (dn_ok) return dn_s ? gemv_stream(DT_Q4_K, false, d, st) : gemv_digits(DT_Q4_K, false, d, st);
    }
    if (a.n_tok == 1 && !a.act_f16) {
        const int64_t ggu = (a.n_ff + 3) / 4, gdn = (a.n_embd + 7) / 8;
        if (!gu_ok)
            hipLaunchKernelGGL((moe_gu1_kernel<float, 8>), cap(a.k * ggu, wgu), dim3(64 * wgu), 0, st, tab,
                               a.ids, a.k, a.n_expert, static_cast<const float *>(a.xn), a.n_embd, a.n_ff,
                               ggu, w.mid);
        hipLaunchKernelGGL((moe_down1_kernel<float, 8>), cap(gdn, 8), dim3(64 * 8), 0, st, tab, a.ids,
                           a.wts, a.k, a.n_expert, a.n_embd, a.n_ff, gdn, w.mid, static_cast<float *>(a.out));
        return hipGetLastError();
    }
    // the plan path: every f16 dispatch (the reference GPU's rounding points
    // need each (token, slot) row whole before its scale), and f32 token
    // batches the digit kernels do not take
    hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(256), 0, st, a.ids, P, a.k, a.n_expert, w, tab,
                           kItemRows);
    const int64_t amax = P < a.n_expert ? P : a.n_expert;
    const int64_t ggu = (a.n_ff + 1) / 2, gdn = (a.n_embd + 3) / 4;
    const dim3 rgrid(static_cast<unsigned>((a.n_embd + 255) / 256), static_cast<unsigned>(a.n_tok));
    if (a.act_f16) {
        hipLaunchKernelGGL((moe_gu_kernel<_Float16, 2, 4>), cap(amax * ggu, wgu), dim3(64 * wgu), 0, st,
                           tab, static_cast<const _Float16 *>(a.xn), a.n_embd, a.n_ff, ggu, w);
        hipLaunchKernelGGL(moe_scale_kernel, dim3(static_cast<unsigned>(P)), dim3(256), 0, st, a.n_ff,
                           a.n_expert, w);
        hipLaunchKernelGGL((moe_down_kernel<_Float16, 2, 4>), cap(amax * gdn, wdn), dim3(64 * wdn), 0, st, tab,
                           a.n_embd, a.n_ff, gdn, w);
        hipLaunchKernelGGL(moe_reduce_f16_kernel, rgrid, dim3(256), 0, st, a.wts, a.k, a.n_embd, w,
                           static_cast<_Float16 *>(a.out));
        return hipGetLastError();
    }
    hipLaunchKernelGGL((moe_gu_kernel<float, 2, 4>), cap(amax * ggu, wgu), dim3(64 * wgu), 0, st,
                       tab, static_cast<const float *>(a.xn), a.n_embd, a.n_ff, ggu, w);
    hipLaunchKernelGGL((moe_down_kernel<float, 2, 4>), cap(amax * gdn, wdn), dim3(64 * wdn), 0, st, tab,
                       a.n_embd, a.n_ff, gdn, w);
    hipLaunchKernelGGL((moe_reduce_kernel<float>), rgrid, dim3(256), 0, st, a.ids, a.wts, a.k,
                       a.n_embd, w, static_cast<float *>(a.out));
    return hipGetLastError();
}

}  // namespace krk
