// dequant.hip -- the exactness surface: whole rows through the 32-value chunk
// contract (bit-identical to the host decoders, src/quant.cpp:331-512 and
// dequant_row 1911-1960), and the Q8 activation quantizer
// (quantize_q8_32_d, src/quant.cpp:2167-2197) that the int8 rung feeds on.
#include "krk_formats.hpp"
#include "krk_kernels.hpp"

namespace krk {

// One thread per 32-value chunk.  Row r, chunk c -> out[r, 32c .. 32c+31].
template <int DT, bool F16>
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t *__restrict__ w,
                                                      int64_t row_bytes, int64_t n_rows,
                                                      int64_t n_in, void *__restrict__ out) {
    constexpr int BV = blk_vals(DT), BB = blk_bytes(DT), CPB = BV / 32;
    const int64_t chunks_per_row = n_in / 32;
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (gid >= n_rows * chunks_per_row) return;
    const int64_t r = gid / chunks_per_row, c = gid % chunks_per_row;
    const uint8_t *blk = w + r * row_bytes + (c / CPB) * BB;
    float y[32];
    dequant_chunk<DT>(blk, static_cast<int>(c % CPB), y);
    const int64_t o = r * n_in + c * 32;
    if constexpr (F16) {
        // IEEE RNE to f16, with the sign of a zero kept: gfx950's packed
        // f32->f16 conversion returns +0 for -0, and the f32 values here are
        // the host decoder's bits, signed zeros included.
        uint16_t *oh = static_cast<uint16_t *>(out) + o;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const _Float16 h = static_cast<_Float16>(y[i]);
            uint16_t hb;
            __builtin_memcpy(&hb, &h, 2);
            oh[i] = static_cast<uint16_t>(hb | ((__float_as_uint(y[i]) >> 16) & 0x8000u));
        }
    } else {
        float *of = static_cast<float *>(out) + o;
#pragma unroll
        for (int i = 0; i < 32; i += 4)
            *reinterpret_cast<floatx4 *>(of + i) = floatx4{y[i], y[i + 1], y[i + 2], y[i + 3]};
    }
}

template <bool F16>
static hipError_t dq(int dt, const void *w, int64_t rb, int64_t n_rows, int64_t n_in, void *out,
                     hipStream_t st) {
    const int64_t total = n_rows * (n_in / 32);
    const dim3 grid(static_cast<unsigned>((total + 255) / 256));
    const uint8_t *wb = static_cast<const uint8_t *>(w);
    switch (dt) {
        case DT_Q4_0: hipLaunchKernelGGL((dequant_kernel<DT_Q4_0, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_IQ4_NL: hipLaunchKernelGGL((dequant_kernel<DT_IQ4_NL, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_IQ4_XS: hipLaunchKernelGGL((dequant_kernel<DT_IQ4_XS, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_Q2_K: hipLaunchKernelGGL((dequant_kernel<DT_Q2_K, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_Q3_K: hipLaunchKernelGGL((dequant_kernel<DT_Q3_K, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_MXFP4: hipLaunchKernelGGL((dequant_kernel<DT_MXFP4, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_Q4_1: hipLaunchKernelGGL((dequant_kernel<DT_Q4_1, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_Q5_0: hipLaunchKernelGGL((dequant_kernel<DT_Q5_0, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_Q5_1: hipLaunchKernelGGL((dequant_kernel<DT_Q5_1, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_F16: hipLaunchKernelGGL((dequant_kernel<DT_F16, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
#define KRK_CHUNK_CASE(D) \
    case D: hipLaunchKernelGGL((dequant_kernel<D, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        KRK_CHUNK_FORMATS(KRK_CHUNK_CASE)
#undef KRK_CHUNK_CASE
        case DT_BF16: hipLaunchKernelGGL((dequant_kernel<DT_BF16, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_Q8_0: hipLaunchKernelGGL((dequant_kernel<DT_Q8_0, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_Q4_K: hipLaunchKernelGGL((dequant_kernel<DT_Q4_K, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_Q5_K: hipLaunchKernelGGL((dequant_kernel<DT_Q5_K, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        case DT_Q6_K: hipLaunchKernelGGL((dequant_kernel<DT_Q6_K, F16>), grid, dim3(256), 0, st, wb, rb, n_rows, n_in, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t dequant_rows(int dt, const void *w, int64_t row_bytes, int64_t n_rows, int64_t n_in,
                        void *out, bool to_f16, hipStream_t st) {
    return to_f16 ? dq<true>(dt, w, row_bytes, n_rows, n_in, out, st)
                  : dq<false>(dt, w, row_bytes, n_rows, n_in, out, st);
}

// quantize_q8_32_d: amax over the 32 values, d = amax / 127 (0 for an
// all-zero block), codes = round-to-nearest-even(x * (1/d)) clamped to
// [-127, 127]; a NaN product lands on -127 as the host's cvtps + clamp does.
// CT int8_t writes the packed codes; CT _Float16 writes the same codes as
// exact f16 values (the int8 rung's MFMA operand).
template <typename XT, typename CT>
__global__ void __launch_bounds__(256) quantize_q8_kernel(const XT *__restrict__ x, int64_t nblk,
                                                          CT *__restrict__ xq,
                                                          float *__restrict__ dx,
                                                          float *__restrict__ sx16 = nullptr) {
    const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblk) return;
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] = static_cast<float>(x[b * 32 + i]);
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    dx[b] = d;
    uint32_t packed[8];
    if (d == 0.0f) {
#pragma unroll
        for (int k = 0; k < 8; k++) packed[k] = 0u;
    } else {
        const float inv = 1.0f / d;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            uint32_t word = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float pr = v[4 * k + j] * inv;
                int q = (pr != pr) ? -127 : static_cast<int>(fminf(fmaxf(__builtin_rintf(pr), -127.0f), 127.0f));
                word |= (static_cast<uint32_t>(q) & 0xFFu) << (8 * j);
            }
            packed[k] = word;
        }
    }
    if (sx16) {  // code sums of the two 16-value halves (the affine int8 fold)
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int c = static_cast<int8_t>(packed[k] >> (8 * j));
                if (k < 4) s0 += c; else s1 += c;
            }
        sx16[2 * b] = static_cast<float>(s0);
        sx16[2 * b + 1] = static_cast<float>(s1);
    }
    if constexpr (sizeof(CT) == 1) {
        uint32_t *o = reinterpret_cast<uint32_t *>(xq + b * 32);
#pragma unroll
        for (int k = 0; k < 8; k++) o[k] = packed[k];
    } else {
        half8 *o = reinterpret_cast<half8 *>(xq + b * 32);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            half8 h;
#pragma unroll
            for (int j = 0; j < 8; j++)
                h[j] = static_cast<_Float16>(static_cast<int8_t>(packed[2 * k + j / 4] >> (8 * (j % 4))));
            o[k] = h;
        }
    }
}

hipError_t quantize_q8_rows(const void *x, bool x_f16, int64_t rows, int64_t n, int8_t *xq,
                            float *dx, hipStream_t st) {
    const int64_t nblk = rows * (n / 32);
    const dim3 grid(static_cast<unsigned>((nblk + 255) / 256));
    if (x_f16)
        hipLaunchKernelGGL((quantize_q8_kernel<_Float16, int8_t>), grid, dim3(256), 0, st,
                           static_cast<const _Float16 *>(x), nblk, xq, dx);
    else
        hipLaunchKernelGGL((quantize_q8_kernel<float, int8_t>), grid, dim3(256), 0, st,
                           static_cast<const float *>(x), nblk, xq, dx);
    return hipGetLastError();
}

hipError_t quantize_q8_rows_f16codes(const void *x, bool x_f16, int64_t rows, int64_t n,
                                     _Float16 *xq, float *dx, float *sx16, hipStream_t st) {
    const int64_t nblk = rows * (n / 32);
    const dim3 grid(static_cast<unsigned>((nblk + 255) / 256));
    if (x_f16)
        hipLaunchKernelGGL((quantize_q8_kernel<_Float16, _Float16>), grid, dim3(256), 0, st,
                           static_cast<const _Float16 *>(x), nblk, xq, dx, sx16);
    else
        hipLaunchKernelGGL((quantize_q8_kernel<float, _Float16>), grid, dim3(256), 0, st,
                           static_cast<const float *>(x), nblk, xq, dx, sx16);
    return hipGetLastError();
}

}  // namespace krk
