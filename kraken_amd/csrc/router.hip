// router.hip -- the MoE router's input stage on the device: softmax over the
// expert logits and top-k selection with sum-normalised weights
// (Backend::router_softmax / router_topk, backend.hpp:933-955; host rule
// engine.cpp:11704-11918), one wave per token row.  The selection and the
// weight arithmetic follow the host's order exactly; only expf differs
// (device ocml vs the host libm), which the parity tests bound.
#include "krk_dev.hpp"
#include "krk_kernels.hpp"

namespace krk {

constexpr int kMaxExpertsPerLane = 16;   // n_expert <= 1024 over 64 lanes

// One wave per token row.  The exponentials are computed in parallel (the
// same expf per element as a serial loop); the sum runs serially in
// ascending expert id in lane 0, as the host does, so only expf itself can
// differ from the host.
template <typename T>
__global__ void __launch_bounds__(64) router_softmax_kernel(const T *__restrict__ logits,
                                                           float *__restrict__ probs,
                                                           int64_t n_rows, int ne) {
    __shared__ float ex[kMaxExpertsPerLane * 64];
    __shared__ float inv_s;
    const int64_t r = blockIdx.x;
    const int lane = threadIdx.x;
    const T *l = logits + r * ne;
    float *p = probs + r * ne;
    float v[kMaxExpertsPerLane];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; i++) {
        const int e = lane + 64 * i;
        v[i] = e < ne ? static_cast<float>(l[e]) : -INFINITY;
        mx = fmaxf(mx, v[i]);
    }
    // the host's running max keeps l[0] first; max is order-free except for NaN
    for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 64));
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; i++) {
        const int e = lane + 64 * i;
        if (e < ne) ex[e] = expf(v[i] - mx);
    }
    __syncthreads();
    if (lane == 0) {
        float sum = 0.0f;
        for (int e = 0; e < ne; e++) sum += ex[e];
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
    if (act_f16)
        hipLaunchKernelGGL((router_softmax_kernel<_Float16>), grid, dim3(64), 0, st,
                           static_cast<const _Float16 *>(logits), probs, n_rows, n_expert);
    else
        hipLaunchKernelGGL((router_softmax_kernel<float>), grid, dim3(64), 0, st,
                           static_cast<const float *>(logits), probs, n_rows, n_expert);
    return hipGetLastError();
}

// One wave per token row: k rounds of a wave argmax over the experts not yet
// taken.  The winner of a round is the largest probability and, among equal
// ones, the lowest id -- what the host's ascending strict-> scan picks.  The
// normalisation sum runs serially over the k picks in pick order.
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
    float v[kMaxExpertsPerLane];
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; i++) {
        const int e = lane + 64 * i;
        v[i] = e < ne ? p[e] : -INFINITY;
    }
    uint32_t taken = 0;   // bit i: expert lane + 64 i taken
    for (int s = 0; s < k; s++) {
        // lane-local best: ascending id inside the lane, strict >
        float bp = -1.0f;
        int be = -1;
#pragma unroll
        for (int i = 0; i < kMaxExpertsPerLane; i++) {
            const int e = lane + 64 * i;
            if (e < ne && !(taken & (1u << i)) && v[i] > bp) { bp = v[i]; be = e; }
        }
        // wave argmax: larger p wins, equal p -> lower id (an invalid -1 loses)
        for (int m = 32; m >= 1; m >>= 1) {
            const float op = __shfl_xor(bp, m, 64);
            const int oe = __shfl_xor(be, m, 64);
            const bool take = (oe >= 0) && (be < 0 || op > bp || (op == bp && oe < be));
            bp = take ? op : bp;
            be = take ? oe : be;
        }
        if (be >= 0 && (be & 63) == lane) taken |= 1u << (be >> 6);
        if (lane == 0) {
            isel[s] = be;
            wsel[s] = be >= 0 ? p[be] : 0.0f;
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

hipError_t router_topk(const float *probs, int64_t n_rows, int n_expert, int k, int32_t *ids,
                       float *wts, int normalize, float scale, hipStream_t st) {
    if (n_expert > 64 * kMaxExpertsPerLane || k > 64) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(n_rows));
    hipLaunchKernelGGL(router_topk_kernel, grid, dim3(64), 0, st, probs, n_rows, n_expert, k, ids,
                       wts, normalize, scale);
    return hipGetLastError();
}

}  // namespace krk
