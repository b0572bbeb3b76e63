// probe.hip -- measurement probes, no reference counterpart:
//   * a plain read-bandwidth probe: the ceiling a single launch of a pure HBM
//     stream reaches on this part, measured beside the decode GEMV it bounds
//     (the GEMV reads each weight byte once, so a kernel that only reads the
//     same bytes and does nothing else is its floor);
//   * a plain f16 x f16 GEMM (no dequantization) and its matrix-core
//     skeleton without global loads: what dense f16 MFMA work reaches on
//     this part with the operands it is given, measured beside the prefill
//     GEMM it bounds.
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

// ---- f16 GEMM probe: out[M, N] = x[M, K] . w[N, K]^T, f16 in and out.
// Tile 256 x 256, K step 32; 4 waves (one per SIMD) in 2 x 2, each 128 x 128
// on v_mfma_f32_32x32x16_f16 (256 accumulators per lane).  Both operands go
// global -> LDS by global_load_lds_dwordx4 into four stages of 256 + 256
// rows x 64 bytes; a row's 16-byte chunk c sits at slot c ^ ((r >> 2) & 3),
// so the 16 lanes of a fragment read sharing a chunk hit distinct bank
// groups.  One barrier per K step; fragment reads of the next sub-step are
// interleaved with the current sub-step's MFMAs.  LOADS = false: the first
// stage is loaded once and the K loop re-reads it (the skeleton's MFMA and
// LDS work with no global traffic).
constexpr int PB_K = 32, PB_ST = 4, PB_ROWB = 64, PB_STAGE = 512 * PB_ROWB;
typedef __attribute__((address_space(3))) void probe_lds_t;
typedef _Float16 ph8 __attribute__((ext_vector_type(8)));
typedef float pf16 __attribute__((ext_vector_type(16)));

template <int N> __device__ __forceinline__ void probe_wait_vm() {
    // s_waitcnt simm16: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <bool LOADS>
__global__ void __launch_bounds__(256, 1)
    probe_gemm_kernel(const _Float16 *__restrict__ x, const _Float16 *__restrict__ w, _Float16 *__restrict__ out,
                      int M, int N, int K, int tiles_m) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[PB_ST * PB_STAGE];
    // XCD-aware order, M fastest within an XCD's run of tiles
    const int G = gridDim.x, b = blockIdx.x, per = G / 8;
    const int g = b >= per * 8 ? b : (b & 7) * per + (b >> 3);
    const int m0 = (g % tiles_m) * 256, n0 = (g / tiles_m) * 256;
    const int nk = K / PB_K;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, wm = wave >> 1, wn = wave & 1;
    const _Float16 *asrc[4], *bsrc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int r = 64 * wave + 16 * j + (lane >> 2);
        const int c = (lane & 3) ^ ((r >> 2) & 3);
        asrc[j] = x + static_cast<int64_t>(min(m0 + r, M - 1)) * K + 8 * c;
        bsrc[j] = w + static_cast<int64_t>(min(n0 + r, N - 1)) * K + 8 * c;
    }
    auto issue = [&](int step, int st) {
        uint8_t *base = lds + st * PB_STAGE + 64 * wave * PB_ROWB;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            __builtin_amdgcn_global_load_lds(static_cast<const void *>(asrc[j] + step * PB_K),
                                             (probe_lds_t *)(base + 16 * j * PB_ROWB), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(static_cast<const void *>(bsrc[j] + step * PB_K),
                                             (probe_lds_t *)(base + 256 * PB_ROWB + 16 * j * PB_ROWB), 16, 0, 0);
        }
    };
    const int fr = lane & 31, sw = (fr >> 2) & 3;
    const int aoff = (wm * 128 + fr) * PB_ROWB, boff = 256 * PB_ROWB + (wn * 128 + fr) * PB_ROWB;
    pf16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    ph8 fa0[4], fb0[4], fa1[4], fb1[4];
    auto rd = [&](const uint8_t *sb, int ks, ph8 (&fa)[4], ph8 (&fb)[4]) {
        const int sl = ((2 * ks + (lane >> 5)) ^ sw) * 16;
#pragma unroll
        for (int i = 0; i < 4; i++) fa[i] = *reinterpret_cast<const ph8 *>(sb + aoff + i * 32 * PB_ROWB + sl);
#pragma unroll
        for (int j = 0; j < 4; j++) fb[j] = *reinterpret_cast<const ph8 *>(sb + boff + j * 32 * PB_ROWB + sl);
    };
    auto mm = [&](const ph8 (&fa)[4], const ph8 (&fb)[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        // the other set's 8 reads spread over the first 8 of the 16 MFMAs
#pragma unroll
        for (int r = 0; r < 8; r++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    };
    // this wave's DMAs of `step` have landed once at most the later steps'
    // (8 instructions each) are outstanding; then a bare barrier (not
    // __syncthreads, which would drain every outstanding DMA)
    auto publish = [&](int step) {
        const int later = LOADS ? max(0, min(nk - 1, step + PB_ST - 2) - step) : 0;
        if (later >= 2) probe_wait_vm<16>();
        else if (later == 1) probe_wait_vm<8>();
        else probe_wait_vm<0>();
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    for (int s = 0; s < (LOADS ? PB_ST - 1 : 1); s++)
        if (s < nk) issue(s, s);
    publish(0);
    rd(lds, 0, fa0, fb0);
    for (int t = 0; t < nk; t++) {
        if (LOADS && t + PB_ST - 1 < nk) issue(t + PB_ST - 1, (t + PB_ST - 1) % PB_ST);
        const uint8_t *sb = lds + (LOADS ? (t % PB_ST) * PB_STAGE : 0);
        rd(sb, 1, fa1, fb1);
        mm(fa0, fb0);
        publish(t + 1);
        rd(lds + (LOADS ? ((t + 1) % PB_ST) * PB_STAGE : 0), 0, fa0, fb0);
        mm(fa1, fb1);
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            __builtin_amdgcn_sched_barrier(0);
            const int n = n0 + wn * 128 + j * 32 + (lane & 31);
            if (n >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < M) out[static_cast<int64_t>(m) * N + n] = static_cast<_Float16>(acc[i][j][r]);
            }
        }
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

hipError_t probe_gemm(const void *x, const void *w, void *out, int64_t M, int64_t N, int64_t K, bool loads,
                      hipStream_t st) {
    if (M < 1 || N < 1 || K < PB_K || K % PB_K || M > (1 << 30) || N > (1 << 30) || K > (1 << 30) ||
        ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15))
        return hipErrorInvalidValue;
    const int tm = static_cast<int>((M + 255) / 256), tn = static_cast<int>((N + 255) / 256);
    const dim3 grid(static_cast<unsigned>(tm * tn));
    if (loads)
        hipLaunchKernelGGL(probe_gemm_kernel<true>, grid, dim3(256), 0, st, static_cast<const _Float16 *>(x),
                           static_cast<const _Float16 *>(w), static_cast<_Float16 *>(out), static_cast<int>(M),
                           static_cast<int>(N), static_cast<int>(K), tm);
    else
        hipLaunchKernelGGL(probe_gemm_kernel<false>, grid, dim3(256), 0, st, static_cast<const _Float16 *>(x),
                           static_cast<const _Float16 *>(w), static_cast<_Float16 *>(out), static_cast<int>(M),
                           static_cast<int>(N), static_cast<int>(K), tm);
    return hipGetLastError();
}

}  // namespace krk
