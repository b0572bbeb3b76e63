// router.hip -- the MoE router's input stage on the device: softmax over the
// expert logits and top-k selection with sum-normalised weights
// (Backend::router_softmax / router_topk, backend.hpp:933-955; host rule
// engine.cpp:11704-11918).  One thread per token row, walking the experts in
// ascending id exactly as the host loop does, so the selection and the weight
// arithmetic follow the host's order; only expf differs (device ocml vs the
// host libm), which the parity tests bound.
#include "krk_dev.hpp"
#include "krk_kernels.hpp"

namespace krk {

template <typename T>
__global__ void __launch_bounds__(64) router_softmax_kernel(const T *__restrict__ logits,
                                                           float *__restrict__ probs,
                                                           int64_t n_rows, int ne) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= n_rows) return;
    const T *l = logits + r * ne;
    float *p = probs + r * ne;
    float mx = static_cast<float>(l[0]);
    for (int e = 1; e < ne; e++) mx = fmaxf(mx, static_cast<float>(l[e]));
    float sum = 0.0f;
    for (int e = 0; e < ne; e++) {
        const float v = expf(static_cast<float>(l[e]) - mx);
        p[e] = v;
        sum += v;
    }
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (int e = 0; e < ne; e++) p[e] *= inv;
}

hipError_t router_softmax(const void *logits, bool act_f16, float *probs, int64_t n_rows,
                          int n_expert, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>((n_rows + 63) / 64));
    if (act_f16)
        hipLaunchKernelGGL((router_softmax_kernel<_Float16>), grid, dim3(64), 0, st,
                           static_cast<const _Float16 *>(logits), probs, n_rows, n_expert);
    else
        hipLaunchKernelGGL((router_softmax_kernel<float>), grid, dim3(64), 0, st,
                           static_cast<const float *>(logits), probs, n_rows, n_expert);
    return hipGetLastError();
}

// k rounds of argmax over the experts not yet taken; strict > in ascending
// id keeps the lower id on a tie.  The taken set is a 1024-bit mask.
__global__ void __launch_bounds__(64) router_topk_kernel(const float *__restrict__ probs,
                                                        int64_t n_rows, int ne, int k,
                                                        int32_t *__restrict__ ids,
                                                        float *__restrict__ wts, int normalize,
                                                        float scale) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (r >= n_rows) return;
    const float *p = probs + r * ne;
    uint32_t taken[32];
    for (int i = 0; i < 32; i++) taken[i] = 0u;
    float wsel[64];
    for (int s = 0; s < k; s++) {
        int best = -1;
        float bestp = -1.0f;
        for (int e = 0; e < ne; e++) {
            if (taken[e >> 5] & (1u << (e & 31))) continue;
            const float v = p[e];
            if (v > bestp) { bestp = v; best = e; }
        }
        ids[r * k + s] = best;
        wsel[s] = best >= 0 ? p[best] : 0.0f;
        if (best >= 0) taken[best >> 5] |= 1u << (best & 31);
    }
    if (normalize) {
        float ksum = 0.0f;
        for (int s = 0; s < k; s++) ksum += wsel[s];
        const float kinv = ksum > 0.0f ? 1.0f / ksum : 0.0f;
        for (int s = 0; s < k; s++) wsel[s] *= kinv;
    }
    const bool sc = scale != 0.0f && scale != 1.0f;
    for (int s = 0; s < k; s++) wts[r * k + s] = sc ? wsel[s] * scale : wsel[s];
}

hipError_t router_topk(const float *probs, int64_t n_rows, int n_expert, int k, int32_t *ids,
                       float *wts, int normalize, float scale, hipStream_t st) {
    const dim3 grid(static_cast<unsigned>((n_rows + 63) / 64));
    hipLaunchKernelGGL(router_topk_kernel, grid, dim3(64), 0, st, probs, n_rows, n_expert, k, ids,
                       wts, normalize, scale);
    return hipGetLastError();
}

}  // namespace krk
