// krk_dev.hpp -- device-side building blocks shared by the gfx950 kernels:
// block geometry, aligned raw loads of 2-byte-aligned GGUF blocks, f16
// helpers and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace krk {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int intx4 __attribute__((ext_vector_type(4)));
typedef int intx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// Q4_K 144 B / 256, Q5_K 176 B / 256, Q6_K 210 B / 256, Q4_0 and IQ4_NL 18 B / 32,
// Q8_0 34 B / 32, IQ4_XS 136 B / 256
// (include/krk/quant.hpp geometry; src/quant.cpp:1805-1900).
enum : int { DT_F32 = 0, DT_F16 = 1, DT_Q4_0 = 2, DT_Q8_0 = 8, DT_Q4_K = 12, DT_Q5_K = 13, DT_Q6_K = 14,
             DT_IQ4_NL = 20, DT_IQ4_XS = 23, DT_Q2_K = 10, DT_Q3_K = 11, DT_MXFP4 = 39,
             DT_Q4_1 = 3, DT_Q5_0 = 6, DT_Q5_1 = 7, DT_BF16 = 30,
             // served through the generic chunk path (include/krk/quant.hpp:25-31, 67-68, 105,
             // 128-129, 166-168)
             DT_Q8_1 = 9, DT_Q8_K = 15, DT_TQ1_0 = 34, DT_TQ2_0 = 35, DT_NVFP4 = 40, DT_ROCMFP4 = 100,
             DT_ROCMFP4_FAST = 101, DT_Q6_0_ROCMFPX = 102, DT_Q3_0_ROCMFPX = 104, DT_Q2_0_ROCMFPX = 107,
             DT_Q1_0 = 41, DT_Q2_0 = 42, DT_Q2_0_64 = 48, DT_PQ2_0 = 142, DT_PTQ1_0 = 143 };

__device__ __forceinline__ float h2f(uint32_t h16) {
    _Float16 h;
    uint16_t v = static_cast<uint16_t>(h16);
    __builtin_memcpy(&h, &v, 2);
    return static_cast<float>(h);
}

// One dword from a 4-byte aligned address (global memory, vector load).
__device__ __forceinline__ uint32_t ld32(const uint8_t *p) {
    return *reinterpret_cast<const uint32_t *>(p);
}
// The bytes from p to the end of the 4-aligned dword that holds p, in the
// low bits (zeros above).  The aligned address comes from pointer
// arithmetic, which keeps p's address space (an integer round trip would
// make the load a FLAT one).
__device__ __forceinline__ uint32_t ld32_at(const uint8_t *p) {
    const uint32_t o = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3);
    return ld32(p - o) >> (8 * o);
}
__device__ __forceinline__ u32x4 ld128(const uint8_t *p) {
    return *reinterpret_cast<const u32x4 *>(p);
}
__device__ __forceinline__ u32x2 ld64(const uint8_t *p) {
    return *reinterpret_cast<const u32x2 *>(p);
}
// Device (global) memory through a pointer the compiler cannot place: one
// read from memory (a table entry, a run record) is generic to it, and loads
// through a generic pointer are FLAT instructions, which also count against
// lgkmcnt, so every wait for an LDS read would wait for them too and
// prefetched weights would stop being in flight across LDS work.  gbyte
// pointers load with global instructions.
typedef const __attribute__((address_space(1))) uint8_t gbyte;
__device__ __forceinline__ gbyte *to_global(const uint8_t *p) { return (gbyte *)p; }
__device__ __forceinline__ u32x4 ld128(gbyte *p) {
    return *(const __attribute__((address_space(1))) u32x4 *)p;
}
__device__ __forceinline__ u32x4 ldg128(const uint8_t *p) { return ld128(to_global(p)); }
// A weight read whose whole cache line is consumed by the same instruction
// (lane-contiguous pieces) and never again: the nontemporal policy ("nt")
// streams it.  (Reads that use half a line, the other half coming from
// another instruction, must not take it: the second half is then fetched
// again.)
__device__ __forceinline__ u32x4 ld128_nt(gbyte *p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4 *)p);
}
// 2-byte aligned reads (Q6_K's 210-byte blocks): the part runs its global
// memory with unaligned access allowed, which hipcc's gfx950 target assumes
// (one dwordx4 / dword / ushort load each)
typedef u32x4 u32x4_a2 __attribute__((aligned(2)));
typedef uint32_t u32_a2 __attribute__((aligned(2)));
__device__ __forceinline__ u32x4 ld128_a2(gbyte *p) {
    return *(const __attribute__((address_space(1))) u32x4_a2 *)p;
}
__device__ __forceinline__ uint32_t ld32_a2(gbyte *p) {
    return *(const __attribute__((address_space(1))) u32_a2 *)p;
}
__device__ __forceinline__ uint32_t ld16g(gbyte *p) {
    return *(const __attribute__((address_space(1))) uint16_t *)p;
}

// ({hi,lo} >> 8*s)[31:0], s in 0..3 (v_alignbyte_b32).
__device__ __forceinline__ uint32_t align_bytes(uint32_t hi, uint32_t lo, uint32_t s) {
    return __builtin_amdgcn_alignbyte(hi, lo, s);
}

// Byte k (0..3) of a dword as f32; the backend selects v_cvt_f32_ubyteN.
template <int K>
__device__ __forceinline__ float ubyte_f(uint32_t v) {
    return static_cast<float>((v >> (8 * K)) & 0xFFu);
}

// Signed byte k of a dword as f32.
template <int K>
__device__ __forceinline__ float sbyte_f(uint32_t v) {
    return static_cast<float>(static_cast<int32_t>(v << (24 - 8 * K)) >> 24);
}

__device__ __forceinline__ float shfl_xor(float v, int m) {
    return __shfl_xor(v, m, kWave);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
    return v;
}

// Reduce V values per lane (V a power of two, 1..64) across the 64 lanes of a
// wave.  Afterwards lane l holds the total of value (l >> (6 - log2 V)) in
// v[0]; a lane whose low 6-log2(V) bits are zero is that value's owner.
// Each halving step exchanges the half of the array the partner keeps, so the
// whole reduction costs V-1 + 6-log2(V) shuffles instead of 6*V.
template <int V>
__device__ __forceinline__ void wave_reduce_multi(float (&v)[V], int lane) {
    constexpr int LOGV = (V >= 64) ? 6 : (V >= 32) ? 5 : (V >= 16) ? 4 : (V >= 8) ? 3
                       : (V >= 4) ? 2 : (V >= 2) ? 1 : 0;
#pragma unroll
    for (int s = 0; s < LOGV; s++) {
        const int m = 32 >> s;
        const int half = V >> (s + 1);
        const bool upper = (lane & m) != 0;
#pragma unroll
        for (int i = 0; i < half; i++) {
            // keep [half, 2*half) when upper else [0, half)
            const float keep = upper ? v[i + half] : v[i];
            const float give = upper ? v[i] : v[i + half];
            v[i] = keep + shfl_xor(give, m);
        }
    }
#pragma unroll
    for (int m = (32 >> LOGV); m >= 1; m >>= 1) v[0] += shfl_xor(v[0], m);
}

// Index of the value a lane owns after wave_reduce_multi<V>.
template <int V>
__device__ __forceinline__ int reduce_owner_index(int lane) {
    constexpr int LOGV = (V >= 64) ? 6 : (V >= 32) ? 5 : (V >= 16) ? 4 : (V >= 8) ? 3
                       : (V >= 4) ? 2 : (V >= 2) ? 1 : 0;
    // Bit s of the index is the lane bit tested at step s (mask 32 >> s),
    // with upper halves keeping the high indices: index bit (LOGV-1-s).
    int idx = 0;
#pragma unroll
    for (int s = 0; s < LOGV; s++)
        if (lane & (32 >> s)) idx |= (V >> (s + 1));
    return idx;
}

template <int V>
__device__ __forceinline__ bool reduce_owner(int lane) {
    constexpr int LOGV = (V >= 64) ? 6 : (V >= 32) ? 5 : (V >= 16) ? 4 : (V >= 8) ? 3
                       : (V >= 4) ? 2 : (V >= 2) ? 1 : 0;
    return (lane & ((64 >> LOGV) - 1)) == 0;
}

__device__ __forceinline__ _Float16 sat_f16(float v) {
    if (v != v) return static_cast<_Float16>(0.0f);
    v = fminf(fmaxf(v, -65504.0f), 65504.0f);
    return static_cast<_Float16>(v);
}

}  // namespace krk
