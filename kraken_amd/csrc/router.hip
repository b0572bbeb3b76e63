// router.hip -- the MoE router's input stage on the device: softmax over the
// expert logits and top-k selection with sum-normalised weights
// (Backend::router_softmax / router_topk, backend.hpp:933-955; host rule
// engine.cpp:11704-11918), one wave per token row.  The selection and the
// weight arithmetic follow the host's order exactly; only expf differs
// (device ocml vs the host libm), which the parity tests bound.
#include "krk_dev.hpp"
#include "krk_kernels.hpp"

#include <type_traits>

// wave-wide reductions of the device library (DPP/permlane based)
extern "C" __device__ __attribute__((const)) float __ockl_wfred_max_f32(float);
extern "C" __device__ __attribute__((const)) int __ockl_wfred_min_i32(int);

namespace krk {

constexpr int kMaxExpertsPerLane = 16;   // n_expert <= 1024 over 64 lanes

// f(std::integral_constant<int, EPL>) with the fewest experts per lane, of
// 1, 2, 4, 8 and 16, that covers n_expert
template <typename F> void with_epl(int ne, F &&f) {
    if (ne <= 64) f(std::integral_constant<int, 1>{});
    else if (ne <= 128) f(std::integral_constant<int, 2>{});
    else if (ne <= 256) f(std::integral_constant<int, 4>{});
    else if (ne <= 512) f(std::integral_constant<int, 8>{});
    else f(std::integral_constant<int, kMaxExpertsPerLane>{});
}

// One wave per token row.  The exponentials are computed in parallel (the
// same expf per element as a serial loop); the sum runs serially in
// ascending expert id in lane 0, as the host does, so only expf itself can
// differ from the host.
// EPL: experts per lane (64 EPL >= ne), so a 128-expert router unrolls two
// slots instead of walking the sixteen a 1024-expert one needs
template <typename T, int EPL>
__global__ void __launch_bounds__(64) router_softmax_kernel(const T *__restrict__ logits,
                                                           float *__restrict__ probs,
                                                           int64_t n_rows, int ne) {
    __shared__ __align__(16) float ex[kMaxExpertsPerLane * 64];
    __shared__ float inv_s;
    const int64_t r = blockIdx.x;
    const int lane = threadIdx.x;
    const T *l = logits + r * ne;
    float *p = probs + r * ne;
    float v[EPL];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane + 64 * i;
        v[i] = e < ne ? static_cast<float>(l[e]) : -INFINITY;
        mx = fmaxf(mx, v[i]);
    }
    // the host's running max keeps l[0] first; max is order-free except for
    // NaN, which fmax (and the wave reduction) skip as the host's > does
    mx = __ockl_wfred_max_f32(mx);
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane + 64 * i;
        if (e < ne) ex[e] = expf(v[i] - mx);
    }
    __syncthreads();
    if (lane == 0) {
        // ascending id; the reads are batched 16 at a time so only the adds
        // form the serial chain
        float sum = 0.0f;
        int e = 0;
        for (; e + 16 <= ne; e += 16) {
            floatx4 q[4];
#pragma unroll
            for (int j = 0; j < 4; j++) q[j] = *reinterpret_cast<const floatx4 *>(&ex[e + 4 * j]);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sum += q[j].x;
                sum += q[j].y;
                sum += q[j].z;
                sum += q[j].w;
            }
        }
        for (; e < ne; e++) sum += ex[e];
        inv_s = sum > 0.0f ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    const float inv = inv_s;
    for (int e = lane; e < ne; e += 64) p[e] = ex[e] * inv;
}

hipError_t router_softmax(const void *logits, bool act_f16, float *probs, int64_t n_rows,
                          int n_expert, hipStream_t st) {
    if (n_expert > 64 * kMaxExpertsPerLane) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(n_rows));
    auto go = [&](auto epl) {
        constexpr int E = decltype(epl)::value;
        if (act_f16)
            hipLaunchKernelGGL((router_softmax_kernel<_Float16, E>), grid, dim3(64), 0, st,
                               static_cast<const _Float16 *>(logits), probs, n_rows, n_expert);
        else
            hipLaunchKernelGGL((router_softmax_kernel<float, E>), grid, dim3(64), 0, st,
                               static_cast<const float *>(logits), probs, n_rows, n_expert);
    };
    with_epl(n_expert, go);
    return hipGetLastError();
}

// One wave per token row: k rounds of a wave argmax over the experts not yet
// taken.  The winner of a round is the largest probability and, among equal
// ones, the lowest id -- what the host's ascending strict-> scan picks.  The
// normalisation sum runs serially over the k picks in pick order.
template <int EPL>
__global__ void __launch_bounds__(64) router_topk_kernel(const float *__restrict__ probs,
                                                        int64_t n_rows, int ne, int k,
                                                        int32_t *__restrict__ ids,
                                                        float *__restrict__ wts, int normalize,
                                                        float scale) {
    __shared__ float wsel[64];
    __shared__ int32_t isel[64];
    const int64_t r = blockIdx.x;
    const int lane = threadIdx.x;
    const float *p = probs + r * ne;
    float v[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane + 64 * i;
        v[i] = e < ne ? p[e] : -INFINITY;
    }
    uint32_t taken = 0;   // bit i: expert lane + 64 i taken
    for (int s = 0; s < k; s++) {
        // lane-local best: ascending id inside the lane, strict >
        float bp = -1.0f;
        int be = -1;
#pragma unroll
        for (int i = 0; i < EPL; i++) {
            const int e = lane + 64 * i;
            if (e < ne && !(taken & (1u << i)) && v[i] > bp) { bp = v[i]; be = e; }
        }
        // wave argmax: the largest p, and among lanes holding it the lowest id
        // (a lane without a candidate keeps -1 and id -1, which never win)
        const float gp = __ockl_wfred_max_f32(bp);
        be = __ockl_wfred_min_i32(be >= 0 && bp == gp ? be : 0x7fffffff);
        if (be == 0x7fffffff) be = -1;
        // the weight is p[be] from its own lane (the wave maximum may carry
        // the other zero's sign when +0 and -0 tie)
        const float pw = __shfl(bp, be & 63);
        if (be >= 0 && (be & 63) == lane) taken |= 1u << (be >> 6);
        if (lane == 0) {
            isel[s] = be;
            wsel[s] = be >= 0 ? pw : 0.0f;
        }
    }
    __syncthreads();
    if (lane == 0) {
        if (normalize) {
            float ksum = 0.0f;
            for (int s = 0; s < k; s++) ksum += wsel[s];
            const float kinv = ksum > 0.0f ? 1.0f / ksum : 0.0f;
            for (int s = 0; s < k; s++) wsel[s] *= kinv;
        }
    }
    __syncthreads();
    const bool sc = scale != 0.0f && scale != 1.0f;
    if (lane < k) {
        ids[r * k + lane] = isel[lane];
        wts[r * k + lane] = sc ? wsel[lane] * scale : wsel[lane];
    }
}

// Up to 256 experts: one thread per expert, each computing its own rank in
// one pass instead of k dependent rounds of wave reductions.  Expert e's key
// is (the order-preserving bits of p[e], ~e) as one 64-bit integer -- larger
// p first, and among equal p (-0 taken as +0, as == does) the lower id -- and
// its rank is the number of larger keys.  Candidates are what the rounds
// above can pick: p > -1 and not NaN; the others hold key 0 and count for
// nothing.  A candidate of rank < k writes itself to pick slot rank; slots
// no candidate fills stay id -1, weight 0, as above.
template <int NW>
__global__ void __launch_bounds__(64 * NW) router_topk_rank_kernel(const float *__restrict__ probs,
                                                                  int64_t n_rows, int ne, int k,
                                                                  int32_t *__restrict__ ids,
                                                                  float *__restrict__ wts, int normalize,
                                                                  float scale) {
    __shared__ __align__(16) uint64_t key[64 * NW];
    __shared__ float wsel[64];
    __shared__ int32_t isel[64];
    const int64_t r = blockIdx.x;
    const int t = threadIdx.x;
    const float v = t < ne ? probs[r * ne + t] : -INFINITY;
    const bool cand = v > -1.0f;
    const uint32_t b = __float_as_uint(v + 0.0f);
    const uint32_t ob = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    const uint64_t my = cand ? (static_cast<uint64_t>(ob) << 32) | static_cast<uint32_t>(~t) : 0;
    key[t] = my;
    if (t < k) {
        isel[t] = -1;
        wsel[t] = 0.0f;
    }
    __syncthreads();
    if (cand) {
        int rank = 0;
#pragma unroll 16
        for (int j = 0; j < 64 * NW; j++) rank += key[j] > my;
        if (rank < k) {
            isel[rank] = t;
            wsel[rank] = v;
        }
    }
    __syncthreads();
    if (t == 0 && normalize) {
        float ksum = 0.0f;
        for (int s = 0; s < k; s++) ksum += wsel[s];
        const float kinv = ksum > 0.0f ? 1.0f / ksum : 0.0f;
        for (int s = 0; s < k; s++) wsel[s] *= kinv;
    }
    __syncthreads();
    const bool sc = scale != 0.0f && scale != 1.0f;
    if (t < k) {
        ids[r * k + t] = isel[t];
        wts[r * k + t] = sc ? wsel[t] * scale : wsel[t];
    }
}

hipError_t router_topk(const float *probs, int64_t n_rows, int n_expert, int k, int32_t *ids,
                       float *wts, int normalize, float scale, hipStream_t st) {
    if (n_expert > 64 * kMaxExpertsPerLane || k > 64) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(n_rows));
    if (n_expert <= 256) {
        const int nw = (n_expert + 63) / 64;
        if (nw <= 1)
            hipLaunchKernelGGL(router_topk_rank_kernel<1>, grid, dim3(64), 0, st, probs, n_rows, n_expert, k, ids,
                               wts, normalize, scale);
        else if (nw == 2)
            hipLaunchKernelGGL(router_topk_rank_kernel<2>, grid, dim3(128), 0, st, probs, n_rows, n_expert, k, ids,
                               wts, normalize, scale);
        else
            hipLaunchKernelGGL(router_topk_rank_kernel<4>, grid, dim3(256), 0, st, probs, n_rows, n_expert, k, ids,
                               wts, normalize, scale);
        return hipGetLastError();
    }
    with_epl(n_expert, [&](auto epl) {
        hipLaunchKernelGGL((router_topk_kernel<decltype(epl)::value>), grid, dim3(64), 0, st, probs, n_rows,
                           n_expert, k, ids, wts, normalize, scale);
    });
    return hipGetLastError();
}

// ------------------------------------------------------------ plan ----
// Backend::moe_plan_build (backend.hpp:976-980; backend_hip.hip:2473-2485,
// router.hpp:241-275): off[n_expert + 1] prefix offsets of the routed pairs
// per expert; rows / wt [n_rows * k] in expert-major order, each expert's
// pairs in (token, slot) order -- rows[at] = the pair's token, wt[at] its
// weight (0 without wts).  The order is prescribed, so the fill is stable:
// chunks of 256 pairs in order, a pair's place = its expert's cursor + the
// number of earlier pairs of the chunk with the same expert.  One workgroup.
__global__ void __launch_bounds__(256) plan_build_kernel(const int32_t *__restrict__ ids, int64_t P, int k,
                                                          int ne, int32_t *__restrict__ off,
                                                          int32_t *__restrict__ rows, float *__restrict__ wt,
                                                          const float *__restrict__ wts) {
    __shared__ int32_t cur[1024];
    __shared__ int32_t ce[256];
    const int tid = threadIdx.x;
    for (int e = tid; e < ne; e += 256) cur[e] = 0;
    __syncthreads();
    for (int64_t i = tid; i < P; i += 256) {
        const int e = ids[i];
        if (e >= 0 && e < ne) atomicAdd(&cur[e], 1);
    }
    __syncthreads();
    if (tid == 0) {   // exclusive scan: off, and each expert's cursor
        int run = 0;
        for (int e = 0; e < ne; e++) {
            const int c = cur[e];
            off[e] = run;
            cur[e] = run;
            run += c;
        }
        off[ne] = run;
    }
    __syncthreads();
    for (int64_t c0 = 0; c0 < P; c0 += 256) {
        const int64_t i = c0 + tid;
        const int e = i < P ? ids[i] : -1;
        const bool live = e >= 0 && e < ne;
        ce[tid] = live ? e : -1;
        __syncthreads();
        if (live) {
            int rank = 0;
            for (int j = 0; j < tid; j++) rank += ce[j] == e;
            const int at = cur[e] + rank;
            rows[at] = static_cast<int32_t>(i / k);
            wt[at] = wts ? wts[i] : 0.0f;
        }
        __syncthreads();
        if (live) atomicAdd(&cur[e], 1);
        __syncthreads();
    }
}

hipError_t moe_plan_build(const int32_t *ids, int64_t n_rows, int k, int n_expert, int32_t *off,
                          int32_t *rows, float *wt, const float *wts, hipStream_t st) {
    if (n_expert > 1024) return hipErrorInvalidValue;
    hipLaunchKernelGGL(plan_build_kernel, dim3(1), dim3(256), 0, st, ids, n_rows * k, k, n_expert, off, rows,
                       wt, wts);
    return hipGetLastError();
}

// ------------------------------------------------------ routing scan ----
// Backend::scan_accum (backend.hpp:955-972; router.hpp:222-239): fold one
// layer's routing into the caller's cumulative histograms, hits[layer *
// n_expert + id] += 1 per routed pair and mass[layer * n_expert + e] += the
// expert's probability summed over the rows (in row order, then one atomic
// add per expert and call).  One thread per expert; the pairs are counted
// by a grid-stride loop.
__global__ void __launch_bounds__(256) scan_accum_kernel(const float *__restrict__ probs,
                                                          const int32_t *__restrict__ ids, int64_t n, int ne,
                                                          int k, int64_t base, unsigned *__restrict__ hits,
                                                          float *__restrict__ mass) {
    const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (g < ne) {
        float s = 0.0f;
        for (int64_t t = 0; t < n; t++) s += probs[t * ne + g];
        if (s != 0.0f) atomicAdd(&mass[base + g], s);
    }
    const int64_t pairs = n * k, stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = g; i < pairs; i += stride) {
        const int id = ids[i];
        if (id >= 0 && id < ne) atomicAdd(&hits[base + id], 1u);
    }
}

hipError_t scan_accum(const float *probs, const int32_t *ids, int64_t n_rows, int n_expert, int k, int layer,
                      unsigned *hits, float *mass, hipStream_t st) {
    const int64_t blocks = (n_expert + 255) / 256;
    hipLaunchKernelGGL(scan_accum_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, probs, ids,
                       n_rows, n_expert, k, static_cast<int64_t>(layer) * n_expert, hits, mass);
    return hipGetLastError();
}

}  // namespace krk
