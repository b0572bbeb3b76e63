// probe.hip -- a plain read-bandwidth probe: the ceiling a single launch of
// a pure HBM stream reaches on this part, measured beside the decode GEMV
// it bounds (the GEMV reads each weight byte once, so a kernel that only
// reads the same bytes and does nothing else is its floor).  Measurement
// only; no reference counterpart.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "krk_kernels.hpp"

namespace krk {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// each workgroup reads a contiguous share, four 16-byte loads per thread in
// flight per step; the xor of everything is written only if it matches a
// value no input of the probe produces, so the loads cannot be dropped
__global__ void __launch_bounds__(256) probe_read_kernel(const u32x4 *__restrict__ p, int64_t per_block,
                                                         int64_t n, uint32_t *__restrict__ sink) {
    const int64_t b0 = static_cast<int64_t>(blockIdx.x) * per_block;
    const int64_t b1 = b0 + per_block < n ? b0 + per_block : n;
    uint32_t acc = 0;
    for (int64_t i = b0 + threadIdx.x; i < b1; i += 4 * 256) {
        u32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int64_t j = i + u * 256;
            v[u] = j < b1 ? p[j] : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 4; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x & 1023] = acc;
}

}  // namespace

hipError_t probe_read(const void *src, int64_t bytes, int blocks, void *sink, hipStream_t st) {
    if (bytes < 16 || bytes % 16 || blocks < 1 || (reinterpret_cast<uintptr_t>(src) & 15))
        return hipErrorInvalidValue;
    const int64_t n = bytes / 16;
    const int64_t per = (n + blocks - 1) / blocks;
    hipLaunchKernelGGL(probe_read_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st,
                       static_cast<const u32x4 *>(src), per, n, static_cast<uint32_t *>(sink));
    return hipGetLastError();
}

}  // namespace krk
