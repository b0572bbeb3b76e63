// gemv_stream.hip -- decode GEMV (one activation row; dense Q4_K also two to
// four) for Q4_K, Q6_K, Q4_0 and Q8_0 weights with every byte of a
// workgroup's tile requested in its first instructions, and the routed
// expert modes of the MoE dispatch built on it.
//
// The products run on the int8 matrix cores exactly as in gemv_digits.hip:
// the weight codes are the B operand, the activations enter as three exact
// int8 digit planes per 32-value sub-block, and the block formula (Q4_K:
// src/quant.cpp:427-447; Q6_K: 491-512, the code offset 32 applied through
// the exact integer sums of x; Q4_0: 331-339; Q8_0: 381-387) is applied once
// per (row, sub-block or scale group) to the exact plane sums.  What differs
// is the data movement, which sets the time of a decode GEMV far more than
// the arithmetic does:
//
//   * A workgroup owns one tile of up to 32 rows over all of K; its waves
//     split K into contiguous slices of NBW blocks.  A wave loads its x slice
//     and then every weight byte of its slice of the tile straight into
//     registers (three 16-byte loads per 16 rows x 1 block), before any
//     arithmetic.  With two workgroups per CU the whole matrix of a 33 MB
//     decode GEMV is in flight from the start of the launch.
//   * The digit table of a wave covers only its own K slice, so a wave builds
//     it alone: no barrier and no LDS-shared table stands between the data
//     arriving and the first MFMA.  Each (16 rows, block) group is decoded
//     as soon as its three loads have landed (the loads return in order).
//   * The waves' partial sums meet once, in LDS, at the end of the tile, and
//     are added in wave order, so the result does not depend on timing.
//
// Tiles: plain and residual (SEG_ACC) segments take tiles of TR rows (16 to
// 32, chosen per launch so that the tiles fill the chip in as few rounds as
// possible); gate/up (SEG_SILU) segments take 16 gate rows and the same 16
// up rows and write silu(gate) * up.  The grid is tiles x segments.
#include <algorithm>
#include <cstdint>

#include "gemv_core.hpp"
#include "krk_formats.hpp"
#include "krk_kernels.hpp"
#include "krk_mi355x.h"

namespace krk {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kTab = 768;   // digit bytes per 256-value block: 8 sub-blocks x 3 planes x 32
// Several rows: the tables are built once per call (stream_xtab_kernel) and
// each block's entry is 848 bytes: the 768 digit bytes, a 16-byte zero pad
// (which the lanes whose A rows are zero read instead of selecting zeros)
// and the eight sub-blocks' {2^-e, sum x}; a wave copies its slice whole.
constexpr int kTabPad = 768, kTabEx = 784, kTabRows = 848;
__host__ __device__ constexpr int tab_stride(int xr) { return xr > 1 ? kTabRows : kTab; }

constexpr int kMaxWaves = 16;
constexpr int kStreamRows = 8;   // dense Q4_K launches of up to this many activation rows
constexpr int kStreamRowsWide = 4;   // ... of slices wider than two blocks
constexpr size_t kLdsMax = 163840;   // LDS per workgroup on gfx950 (160 KB)

__device__ __forceinline__ v4i lds_v4i(const uint8_t *p) { return *reinterpret_cast<const v4i *>(p); }

// Load-transpose geometry of a tile of TR rows and a wave slice of NBW
// blocks of PB 16-byte pieces each (Q4_K: 9 pieces = its 144 bytes; Q6_K:
// 14 pieces over its 210 bytes, the last one its bytes 194..209) on LDS
// strides of 16 PB bytes: P pieces per row, NJ load instructions per lane,
// and a ring of SR row slots (rows 16.. of a two-group tile reuse the slots
// of rows 0.. once the first group is consumed; the rows that reuse them
// arrive only in instructions after the last one the first group needs)
template <int NBW, int TR, int PB = 9> struct LtGeom {
    static constexpr int P = PB * NBW, SLB = 16 * PB * NBW;
    static constexpr int NJ = (TR * P + 63) / 64;
    static constexpr int J0 = (16 * P + 63) / 64 - 1;
    static constexpr int SR0 = (64 * (J0 + 1) + P - 1) / P;
    static constexpr int SR = TR <= 16 ? TR : (SR0 < 16 ? 16 : SR0);
    static_assert(TR <= 32 && (TR <= 16 || SR + 16 >= TR), "two row groups at most");
};

// Q4_0 sub-block s (of the eight in 256 values) -> its digit-table slot:
// 0 1 4 5 2 3 6 7, so that MFMA m of lane pair p meets block 4 p + m
__host__ __device__ constexpr int q40_slot(int s) { return s ^ ((((s >> 1) ^ (s >> 2)) & 1) * 6); }

// quad-lane exchanges (lanes l ^ 1 and l ^ 2) through DPP
__device__ __forceinline__ float quad_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}

// eight consecutive activations (16-byte aligned) as f32
__device__ __forceinline__ void load_x8(const float *p, float (&v)[8]) {
    const floatx4 a = *reinterpret_cast<const floatx4 *>(p);
    const floatx4 b = *reinterpret_cast<const floatx4 *>(p + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void load_x8(const _Float16 *p, float (&v)[8]) {
    const half8 h = *reinterpret_cast<const half8 *>(p);
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = static_cast<float>(h[k]);
}

// The digit planes of eight activations, values 8 (lane & 3) .. + 7 of one
// 32-value sub-block (the quad of lanes 4j .. 4j + 3 holds the sub-block):
// the three planes' bytes for these values into the sub-block's 96 table
// bytes (natural value order) and, from lane 4j, {2^-e, sum x}.  The same
// arithmetic as the one-row kernel's in-place build.
__device__ __forceinline__ void q4k_sub_digits(const float (&v)[8], int lane, uint8_t *sub, float2 *exs) {
    float amax = 0.0f, sum = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        amax = fmaxf(amax, fabsf(v[k]));
        sum += v[k];
    }
    amax = fmaxf(amax, quad_xor1(amax));
    amax = fmaxf(amax, quad_xor2(amax));
    sum += quad_xor1(sum);
    sum += quad_xor2(sum);
    const uint32_t Eb = (__float_as_uint(amax) >> 23) & 255u;
    const bool live = amax > 0.0f && Eb < 255u;
    int e = live ? 148 - static_cast<int>(Eb) : 0;
    e = e > 126 ? 126 : e;
    const float up = __uint_as_float(static_cast<uint32_t>(127 + e) << 23);
    const float dn = __uint_as_float(static_cast<uint32_t>(127 - e) << 23);
    uint32_t Y[8];
#pragma unroll
    for (int k = 0; k < 8; k++)
        Y[k] = __float_as_uint(__builtin_fmaf(v[k], up, 12582912.0f)) + (0x808080u - 0x4B400000u);
    uint32_t p0[2], p1[2], p2[2];
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        const uint32_t *y = Y + 4 * hh;
        const uint32_t A01 = __builtin_amdgcn_perm(y[1], y[0], 0x05010400u);
        const uint32_t A23 = __builtin_amdgcn_perm(y[3], y[2], 0x05010400u);
        const uint32_t B01 = __builtin_amdgcn_perm(y[1], y[0], 0x06020602u);
        const uint32_t B23 = __builtin_amdgcn_perm(y[3], y[2], 0x06020602u);
        p0[hh] = live ? __builtin_amdgcn_perm(A23, A01, 0x05040100u) ^ 0x80808080u : 0u;
        p1[hh] = live ? __builtin_amdgcn_perm(A23, A01, 0x07060302u) ^ 0x80808080u : 0u;
        p2[hh] = live ? __builtin_amdgcn_perm(B23, B01, 0x05040100u) ^ 0x80808080u : 0u;
    }
    uint8_t *o = sub + 8 * (lane & 3);
    *reinterpret_cast<u32x2 *>(o) = u32x2{p0[0], p0[1]};
    *reinterpret_cast<u32x2 *>(o + 32) = u32x2{p1[0], p1[1]};
    *reinterpret_cast<u32x2 *>(o + 64) = u32x2{p2[0], p2[1]};
    if ((lane & 3) == 0) *exs = float2{live ? dn : 1.0f, sum};
}

// The activation rows' digit tables of a several-row launch, once per call:
// row r's blocks 0 .. nbp - 1 at out + (r nbp + b) 848 (blocks from nb on,
// a ragged last slice's, as zero activations: no digits, {1, 0}).  One wave
// per (two blocks, row).
template <typename XT>
__global__ void __launch_bounds__(64) stream_xtab_kernel(const XT *__restrict__ x, int64_t x_stride, int nb, int nbp,
                                                         uint8_t *__restrict__ out) {
    const int lane = threadIdx.x;
    const int sbw = lane >> 2, blk = 2 * static_cast<int>(blockIdx.x) + (sbw >> 3), s = sbw & 7;
    const bool in = blk < nb;
    float v[8];
    load_x8(x + static_cast<int64_t>(blockIdx.y) * x_stride + (in ? static_cast<int64_t>(blk) * 256 + s * 32 + 8 * (lane & 3) : 0),
            v);
    if (!in) {
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = 0.0f;
    }
    uint8_t *base = out + (static_cast<int64_t>(blockIdx.y) * nbp + (blk < nbp ? blk : nbp - 1)) * kTabRows;
    if (blk < nbp) {
        q4k_sub_digits(v, lane, base + s * 96, reinterpret_cast<float2 *>(base + kTabEx) + s);
        if (s == 0 && (lane & 3) == 0) *reinterpret_cast<u32x4 *>(base + kTabPad) = u32x4{0u, 0u, 0u, 0u};
    }
}

// MOE: 0 plain segments; 1 routed gate/up pairs of one token (grid row s =
// slot s, its banks read from moe_tab[moe_ids[s]], its output at seg[0].out
// + s n_out); 2 the routed down projection of one token (K = the k slots'
// activation rows concatenated; a wave's slice lies in one slot, whose bank
// it reads and whose routing weight scales its activations); 3 and 4
// expert-major runs (gate/up pairs, down): grid row a = active expert
// em_runs[a], its weights loaded once and applied to each of its rows in turn
template <int DT, typename XT, typename OT, int NBW, int TR, int NWMAX, bool NWEXACT, int MOE = 0, int LA = 8,
          int XR = 1, bool LT = false>
// (the second bound is waves per SIMD: four for the expert-major runs and
// for six to eight rows, whose registers would otherwise leave one
// workgroup per CU)
__global__ void __launch_bounds__(64 * NWMAX, MOE >= 3 || (XR > 4 && NWMAX == 8) ? 4 : 1)
    gemv_stream_kernel(SegTable t) {
    // XR: activation rows (dense Q4_K launches of 2..4 rows): every row's
    // activations load before the weights, one digit table per row, each
    // weight group decoded once and multiplied against every row
    static_assert(XR == 1 || (MOE == 0 && DT == DT_Q4_K), "several rows: dense Q4_K");
    // LT: the weights move as lane-contiguous 16-byte pieces (full cache
    // lines, nontemporal) and are transposed through the wave's LDS
    static_assert(!LT || ((DT == DT_Q4_K || DT == DT_Q6_K || DT == DT_Q4_0 || DT == DT_Q8_0) && MOE < 3),
                  "load-transpose: Q4_K, Q6_K, Q4_0 or Q8_0, dense or routed");
    using LTG = LtGeom<NBW, TR, DT == DT_Q6_K ? 14 : DT == DT_Q8_0 ? 17 : 9>;
    constexpr bool Q6 = DT == DT_Q6_K;
    constexpr bool Q40 = DT == DT_Q4_0;
    constexpr bool Q80 = DT == DT_Q8_0;
    constexpr bool QS = Q40 || Q80;        // 32-value blocks, eight per 256 values
    constexpr int BB = Q6 ? 210 : Q80 ? 272 : 144;   // bytes per 256 values
    constexpr int RG = (TR + 15) / 16;     // 16-row groups of a plain tile
    constexpr int NL = RG * NBW;           // (16 rows, block) groups of a wave
    constexpr int NPASS = (NBW + 1) / 2;   // x passes: 16 sub-blocks of 8 x 4 lanes each
    constexpr bool PAD = XR > 1;           // zero-padded tables, A operands read without selects
    constexpr int KT = tab_stride(XR);
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // NWEXACT: the launch has exactly NWMAX waves (the common widths 8 and
    // 16), which lets the LDS offsets and the final sums fold to constants
    const int nw = NWEXACT ? NWMAX : static_cast<int>(blockDim.x) >> 6;
    const int c16 = lane & 15, gq = lane >> 4;
    const int kb0 = wv * NBW;

    // the tile: segment blockIdx.y, tile blockIdx.x of it.  Indexing the
    // segment by the grid, and reading all of its fields before any test,
    // keeps them one round of scalar loads away from the first weight
    // request.  A segment with fewer tiles than the grid's width gives its
    // extra workgroups the last rows to re-read, and they store nothing.
    const Seg &sg = t.seg[MOE ? 0 : blockIdx.y];
    const int kind = sg.kind;
    const int64_t n_out = sg.n_out;
    const uint8_t *w = static_cast<const uint8_t *>(sg.w);
    const uint8_t *w2s = static_cast<const uint8_t *>(sg.w2);
    OT *outp = static_cast<OT *>(sg.out);
    const XT *x = static_cast<const XT *>(sg.x);
    const int64_t rb = t.row_bytes;
    const int nb = t.n_in >> 8;
    const bool pair = kind == SEG_SILU;
    const int rows_t = pair ? 16 : TR;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * rows_t;
    // routed banks: one dependent read of the slot's id and table entry
    // (a dropped slot reads expert 0's bank; its output is never used, or
    // its routing weight is 0)
    float wslot = 1.0f;
    int kblk = kb0;   // first block of this wave's slice within its bank row
    if constexpr (MOE == 1) {
        const int e = t.moe_ids[blockIdx.y];
        const bool live = e >= 0 && e < t.moe_ne;
        const krk_moe_entry &en = static_cast<const krk_moe_entry *>(t.moe_tab)[live ? e : 0];
        w = static_cast<const uint8_t *>(en.p[KRK_MOE_GATE]);
        w2s = static_cast<const uint8_t *>(en.p[KRK_MOE_UP]);
        outp += static_cast<int64_t>(blockIdx.y) * n_out;
    } else if constexpr (MOE == 2) {
        const int bps = static_cast<int>(t.moe_kslot >> 8);   // blocks per slot
        const int sl = kb0 / bps < t.moe_k ? kb0 / bps : t.moe_k - 1;
        const int e = t.moe_ids[sl];
        const bool live = e >= 0 && e < t.moe_ne;
        w = static_cast<const uint8_t *>(static_cast<const krk_moe_entry *>(t.moe_tab)[live ? e : 0].p[KRK_MOE_DOWN]);
        wslot = live ? t.moe_wts[sl] : 0.0f;
        kblk = kb0 - sl * bps;
    }
    int pb = 0, pe = 1;   // the rows served: expert-major runs' plan positions
    if constexpr (MOE >= 3) {
        // the run record and the active count in one round of scalar loads
        const EmRun &run = t.em_runs[blockIdx.y];
        const int nact = *t.em_n_act;
        pb = run.pb;
        pe = run.pe;
        w = static_cast<const uint8_t *>(run.w[MOE == 3 ? 0 : 2]);
        w2s = static_cast<const uint8_t *>(run.w[1]);
        if (static_cast<int>(blockIdx.y) >= nact) return;   // beyond the active experts
    }
    auto row_x = [&](int p) {
        return MOE >= 3 ? x + static_cast<int64_t>(t.em_tok ? t.em_tok[p] : p) * t.em_xrow : x;
    };
    const uint8_t *w2 = pair ? w2s : w;

    // ---- the wave's activations first: pass p, lane l holds values
    // 8 (l & 3) .. + 7 of the slice's sub-block 16 p + l / 4
    // the loads issue at raised wave priority, so a wave that is still
    // issuing wins the vector-memory port over one that is already decoding
    // rows per pass: six to eight rows run in passes of four, their digit
    // tables rebuilt in the same (wave-private) LDS while the weights stay
    // in registers, so two workgroups still fit a CU
    constexpr int XP = XR > 5 ? 4 : XR;
    float xvr[PAD ? 1 : XP][NPASS][8];
    // (several rows: the pass's table slices, NBW 848-byte blocks per row,
    // 16 bytes a lane per piece; copied from the call's precomputed tables)
    constexpr int PQ = PAD ? (NBW * (kTabRows / 16) + 63) / 64 : 1;
    u32x4 tv[PAD ? XP : 1][PQ];
    const int nbp = PAD ? nw * NBW : 0;
    auto load_tabs = [&](int r0, int r1) {
#pragma unroll
        for (int r = 0; r < XP; r++) {
            if (r0 + r >= r1) break;
            const uint8_t *src = t.xtab + (static_cast<int64_t>(r0 + r) * nbp + kb0) * kTabRows;
#pragma unroll
            for (int j = 0; j < PQ; j++) {
                const int q = 64 * j + lane;
                tv[r][j] = q < NBW * (kTabRows / 16) ? ldg128(src + 16 * q) : u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto load_xrow_to = [&](const XT *xr, float (&xv)[NPASS][8]) {
#pragma unroll
        for (int p = 0; p < NPASS; p++) {
            const int sbw = p * 16 + (lane >> 2);
            const bool in = sbw < 8 * NBW && kb0 + (sbw >> 3) < nb;
            load_x8(xr + (in ? static_cast<int64_t>(kb0) * 256 + sbw * 32 + 8 * (lane & 3) : 0), xv[p]);
            if (!in) {
#pragma unroll
                for (int k = 0; k < 8; k++) xv[p][k] = 0.0f;
            }
        }
    };
    auto load_xrow = [&](const XT *xr) { load_xrow_to(xr, xvr[0]); };
    __builtin_amdgcn_s_setprio(3);
    if constexpr (PAD) {
        load_tabs(0, XP);
    } else {
        load_xrow(row_x(pb));
#pragma unroll
        for (int xr = 1; xr < XP; xr++) load_xrow_to(x + xr * t.x_stride, xvr[xr]);
    }
    // ---- then every weight byte of the wave's slice of the tile: group i =
    // (row group rg, block b), lane (c16, gq) takes of row rg * 16 + c16:
    //   Q4_K: the 16-byte header and code bytes 16 gq .. + 15 of each
    //         64-byte half (hd, qa, qb);
    //   Q6_K: with h = gq / 2, l = gq % 2: ql bytes 64 h + 16 l and
    //         64 h + 32 + 16 l (hd, qa), qh bytes 128 + 32 h + 16 l (qb), and
    //         16 bytes at 192 + 2 h holding the half's eight scales and, for
    //         h = 1, d (sc)
    //   Q4_0, Q8_0: blocks 2 gq and 2 gq + 1 of the eight (hd, qa, qb, qc, dd)
    u32x4 hd[NL], qa[NL], qb[NL];
    u32x4 sc[Q6 ? NL : 1];
    uint32_t dd6[Q6 && LT ? NL : 1];   // (LT) Q6_K's d, read from the LDS copy
    uint32_t dd[QS ? NL : 1];
    u32x4 qc[Q80 ? NL : 1];
    const int h6 = gq >> 1, lh6 = gq & 1;
    gbyte *src[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int rg = i / NBW, b = i - (i / NBW) * NBW;
        int64_t n;
        const uint8_t *base;
        if (pair) {
            n = n0 + c16;
            base = rg == 0 ? w : w2;
        } else {
            const int r = rg * 16 + c16 < rows_t ? rg * 16 + c16 : rows_t - 1;
            n = n0 + r;
            base = w;
        }
        if (n >= n_out) n = n_out - 1;
        // a ragged last slice re-reads the matrix's last block (discarded)
        const int blk = (kb0 + b < nb ? kb0 + b : nb - 1) - kb0 + kblk;
        src[i] = to_global(base + n * rb + static_cast<int64_t>(blk) * BB);
    }
    auto issue = [&](int i) {
        if constexpr (Q6) {
            hd[i] = ld128_a2(src[i] + 64 * h6 + 16 * lh6);
            qa[i] = ld128_a2(src[i] + 64 * h6 + 32 + 16 * lh6);
            qb[i] = ld128_a2(src[i] + 128 + 32 * h6 + 16 * lh6);
            // the sixteen scales and d: lanes of half h = 0 take bytes
            // 192..207 (their eight scales first), of h = 1 bytes 194..209
            // (their eight scales at 6..13, d at 14..15)
            sc[i] = ld128_a2(src[i] + 192 + 2 * h6);
        } else if constexpr (Q40) {
            // blocks 2 gq and 2 gq + 1 of the eight: 36 bytes at 36 gq
            hd[i] = ld128_a2(src[i] + 36 * gq);
            qa[i] = ld128_a2(src[i] + 36 * gq + 16);
            dd[i] = ld32_a2(src[i] + 36 * gq + 32);
        } else if constexpr (Q80) {
            // blocks 2 gq and 2 gq + 1 of the eight: 68 bytes at 68 gq
            hd[i] = ld128_a2(src[i] + 68 * gq);
            qa[i] = ld128_a2(src[i] + 68 * gq + 16);
            qb[i] = ld128_a2(src[i] + 68 * gq + 32);
            qc[i] = ld128_a2(src[i] + 68 * gq + 48);
            dd[i] = ld32_a2(src[i] + 68 * gq + 64);
        } else {
            hd[i] = ld128(src[i]);
            qa[i] = ld128(src[i] + 16 + 16 * gq);
            qb[i] = ld128(src[i] + 80 + 16 * gq);
        }
    };
    // LT: piece q = 64 j + lane of the tile is row q / P, bytes 16 (q % P)
    // of the wave's slice (P pieces per row), all requested at once
    u32x4 lv[LT ? LTG::NJ : 1];
    if constexpr (LT) {
        // wave-uniform bases and limits; per lane a 32-bit offset (rows are
        // shorter than 2^26 bytes): the row is clamped to the matrix's last,
        // the offset to the last 16 bytes of the slice's last block
        // (a segment shorter than the grid's width gives its extra tiles
        // n0 >= n_out: they re-read the matrix's last row, as the plain
        // path does, and store nothing; rmax is never negative, so the
        // unsigned offsets below stay inside the matrix)
        const int64_t slice = static_cast<int64_t>(kblk) * BB;
        const int64_t nbase = n0 < n_out ? n0 : n_out - 1;
        const uint8_t *wb0 = w + nbase * rb + slice;
        const uint8_t *wb1 = w2 + nbase * rb + slice;
        const int64_t left = n_out - nbase;
        const int rlim = pair ? 16 : TR;
        const int rmax = static_cast<int>(left < rlim ? left : rlim) - 1;
        const int omax = ((nb - kb0 < NBW ? nb - kb0 : NBW) * BB) - 16;
        const int bmax = (nb - kb0 < NBW ? nb - kb0 : NBW) - 1;   // the slice's last block
        const uint32_t rb32 = static_cast<uint32_t>(rb);
#pragma unroll
        for (int j = 0; j < LTG::NJ; j++) {
            const int q = 64 * j + lane;
            const int r = q / LTG::P;
            int o = (q - r * LTG::P) * 16;
            if constexpr (Q6) {
                // piece kk of block b: bytes 16 kk, the last one bytes 194..209
                const int k = q - r * LTG::P, bq = k / 14, kk = k - 14 * bq;
                o = (bq < bmax ? bq : bmax) * 210 + (kk < 13 ? 16 * kk : 194);
            } else {
                o = o < omax ? o : omax;
            }
            if (pair) {
                const int rr = (r & 15) < rmax ? (r & 15) : rmax;
                const uint8_t *bj = r >= 16 ? wb1 : wb0;
                lv[j] = ld128_nt(to_global(bj + (static_cast<uint32_t>(rr) * rb32 + static_cast<uint32_t>(o))));
            } else {
                const int rr = r < rmax ? r : rmax;
                lv[j] = ld128_nt(to_global(wb0 + (static_cast<uint32_t>(rr) * rb32 + static_cast<uint32_t>(o))));
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < (LA < NL ? LA : NL); i++) issue(i);
    }
    __builtin_amdgcn_s_setprio(0);
    // the residual scale 2^-rexp of SEG_ACC segments, read while the weights
    // are in flight rather than after the final barrier
    const float acc_inv = kind == SEG_ACC && t.rexp ? exp2f(-static_cast<float>(t.rexp[0])) : 1.0f;

    for (int pr = pb; pr < pe; pr++) {
    // (expert-major runs: every wave has read the previous row's sums)
    if (MOE >= 3 && pr > pb) __syncthreads();
    // ---- the digit table of the slice (this wave's own LDS), layout
    // [block][sub-block][plane][32 bytes], {2^-e, sum x} per sub-block, and
    // for Q6_K the exact integer sums of X over each 16-value half (int bits)
    // (several rows: the LDS holds XR times the tables, {2^-e, sum x}
    // arrays and partial sums, row by row)
    // layout: XP table slots, then the XR rows' partial sums, then (LT) the
    // slice buffers
    const int tstride = PAD ? nw * NBW * KT : nw * (NBW * KT + 2 * NBW * 8 * static_cast<int>(sizeof(float2)));
    const int rstride = XP * tstride + XR * 32 * nw * 4;
    auto tab_of = [&](int sl) { return lds + sl * tstride + wv * (NBW * KT); };
    auto ex_of = [&](int sl) {
        return reinterpret_cast<float2 *>(lds + sl * tstride + nw * (NBW * KT)) + wv * (NBW * 8);
    };
    auto red_of = [&](int xr) { return reinterpret_cast<float *>(lds + XP * tstride + xr * 32 * nw * 4); };
    // {2^-e, sum x} of block b of table slot sl
    auto ex_blk = [&](int sl, int b) -> const float2 * {
        if constexpr (PAD) return reinterpret_cast<const float2 *>(tab_of(sl) + b * KT + kTabEx);
        else return ex_of(sl) + b * 8;
    };
    uint8_t *tab = tab_of(0);
    float2 *ex = ex_of(0);
    float2 *ex16 = reinterpret_cast<float2 *>(lds + nw * (NBW * KT)) + nw * (NBW * 8) + wv * (NBW * 8);
    // ---- per-lane MFMA roles (A row c16 = 4 sub-block' + digit plane)
    const int ap = c16 & 3, as = c16 >> 2;
    const int sl = 2 * (gq >> 1);
    const bool a_lo = ap < 3 && as == sl, a_hi = ap < 3 && as == sl + 1;
    const int a_off = as * 96 + (ap < 3 ? ap : 0) * 32 + 16 * (gq & 1);
    const uint32_t M = 0x0F0F0F0Fu;
    const uint32_t bsh = 8u * static_cast<uint32_t>(gq);
    const v4i Z = {0, 0, 0, 0};
    // Q6_K: lane group gq's A rows hold sub-block 4 h + qd's half l
    const bool a6 = ap < 3 && as == gq;
    const int a6_off = 4 * h6 * 96 + (ap < 3 ? ap : 0) * 32 + 16 * lh6;
    // the lanes' A-operand offsets within a block's table: lanes whose A
    // rows are zero read the block's zero pad (no select, no branch)
    const int o_lo0 = a_lo ? a_off : kTabPad, o_lo1 = a_lo ? a_off + 384 : kTabPad;
    const int o_hi0 = a_hi ? a_off : kTabPad, o_hi1 = a_hi ? a_off + 384 : kTabPad;
    float acc[RG];
#pragma unroll
    for (int rg = 0; rg < RG; rg++) acc[rg] = 0.0f;
    float accx[XR > 1 ? XR - 1 : 1][RG];   // activation rows 1..
#pragma unroll
    for (int xr = 0; xr < (XR > 1 ? XR - 1 : 1); xr++)
#pragma unroll
        for (int rg = 0; rg < RG; rg++) accx[xr][rg] = 0.0f;
#pragma unroll
    for (int p0 = 0; p0 < XR; p0 += XP) {
    const int pend = p0 + XP < XR ? p0 + XP : XR;
    // (a later pass's activations: L2-resident rows, loaded once the
    // previous pass has released their registers)
    if (p0 > 0) {
        if constexpr (PAD) {
            load_tabs(p0, pend);
        } else {
#pragma unroll
            for (int xr = p0; xr < pend; xr++) load_xrow_to(x + xr * t.x_stride, xvr[xr - p0]);
        }
    }
    if constexpr (PAD) {
        // the pass's rows: their slices into the wave's table slots (this
        // wave's reads of the previous pass completed in order before these
        // writes)
#pragma unroll
        for (int r = 0; r < XP; r++) {
            if (p0 + r >= pend) break;
#pragma unroll
            for (int j = 0; j < PQ; j++) {
                const int q = 64 * j + lane;
                if (q < NBW * (kTabRows / 16)) *reinterpret_cast<u32x4 *>(tab_of(r) + 16 * q) = tv[r][j];
            }
        }
    } else {
#pragma unroll
    for (int xr = p0; xr < pend; xr++) {
    uint8_t *tab = tab_of(xr - p0);
    float2 *ex = ex_of(xr - p0);
#pragma unroll
    for (int p = 0; p < NPASS; p++) {
        const int sbw = p * 16 + (lane >> 2);
        const float *v = xvr[xr - p0][p];
        float amax = 0.0f, sum = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            amax = fmaxf(amax, fabsf(v[k]));
            sum += v[k];
        }
        amax = fmaxf(amax, quad_xor1(amax));
        amax = fmaxf(amax, quad_xor2(amax));
        sum += quad_xor1(sum);
        sum += quad_xor2(sum);
        // 2^e with |x| 2^e < 2^22: e = 148 - the exponent field of the
        // sub-block's largest |x|, so the top digit stays within [-64, 64];
        // zero and non-finite sub-blocks get no digits (a non-finite x makes
        // the sum, and so the row, non-finite as in the reference)
        const uint32_t Eb = (__float_as_uint(amax) >> 23) & 255u;
        const bool live = amax > 0.0f && Eb < 255u;
        int e = live ? 148 - static_cast<int>(Eb) : 0;
        e = e > 126 ? 126 : e;
        const float up = __uint_as_float(static_cast<uint32_t>(127 + e) << 23);
        const float dn = __uint_as_float(static_cast<uint32_t>(127 - e) << 23);
        // X = rint(x 2^e) by one fma with 1.5 2^23 (x 2^e is exact and
        // |x 2^e| < 2^22, so the sum rounds to the nearest integer, ties to
        // even); Y = X + 0x808080 holds the balanced digits as biased bytes:
        // d_i = byte_i(Y) ^ 0x80 with X = d0 + 2^8 d1 + 2^16 d2
        uint32_t Y[8];
#pragma unroll
        for (int k = 0; k < 8; k++)
            Y[k] = __float_as_uint(__builtin_fmaf(v[k], up, 12582912.0f)) + (0x808080u - 0x4B400000u);
        uint32_t p0[2], p1[2], p2[2];
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const uint32_t *y = Y + 4 * hh;
            // bytes 0 and 1 of a value pair, and byte 2 of it
            const uint32_t A01 = __builtin_amdgcn_perm(y[1], y[0], 0x05010400u);
            const uint32_t A23 = __builtin_amdgcn_perm(y[3], y[2], 0x05010400u);
            const uint32_t B01 = __builtin_amdgcn_perm(y[1], y[0], 0x06020602u);
            const uint32_t B23 = __builtin_amdgcn_perm(y[3], y[2], 0x06020602u);
            p0[hh] = live ? __builtin_amdgcn_perm(A23, A01, 0x05040100u) ^ 0x80808080u : 0u;
            p1[hh] = live ? __builtin_amdgcn_perm(A23, A01, 0x07060302u) ^ 0x80808080u : 0u;
            p2[hh] = live ? __builtin_amdgcn_perm(B23, B01, 0x05040100u) ^ 0x80808080u : 0u;
        }
        int xsum = 0;
        if constexpr (Q6) {
            uint32_t ys = 0u;
#pragma unroll
            for (int k = 0; k < 8; k++) ys += Y[k];
            xsum = live ? static_cast<int>(ys - 8u * 0x808080u) : 0;
        }
        if (sbw < 8 * NBW) {
            // Q4_0 and Q8_0: block s of the eight sits in table slot
            // q40_slot(s); Q4_0's values in the order 0..7, 16..23, 8..15,
            // 24..31 (the order its codes take in the B operand)
            const int sbt = QS ? q40_slot(sbw & 7) : (sbw & 7);
            const int po = Q40 ? 8 * (((lane & 1) << 1) | ((lane >> 1) & 1)) : 8 * (lane & 3);
            uint8_t *o = tab + (sbw >> 3) * KT + sbt * 96 + po;
            *reinterpret_cast<u32x2 *>(o) = u32x2{p0[0], p0[1]};
            *reinterpret_cast<u32x2 *>(o + 32) = u32x2{p1[0], p1[1]};
            *reinterpret_cast<u32x2 *>(o + 64) = u32x2{p2[0], p2[1]};
            // (routed down: the slot's weight scales the activations)
            if ((lane & 3) == 0) ex[(sbw & ~7) + sbt] = float2{(live ? dn : 1.0f) * wslot, sum * wslot};
        }
        if constexpr (Q6) {
            // lanes 4j, 4j + 1 hold values 0..15 of sub-block j, 4j + 2, 4j + 3
            // values 16..31
            xsum += __float_as_int(quad_xor1(__int_as_float(xsum)));
            const int xsum_hi = __float_as_int(quad_xor2(__int_as_float(xsum)));
            if (sbw < 8 * NBW && (lane & 3) == 0) ex16[sbw] = float2{__int_as_float(xsum), __int_as_float(xsum_hi)};
        }
    }
    }   // activation rows
    }   // tables built in place

    // (expert-major runs: the next row's activations load while this one
    // is multiplied)
    if (MOE >= 3 && pr + 1 < pe) load_xrow(row_x(pr + 1));
    // two-block slices read their A operands once, before the first group
    // lands (wider slices read them per group: registers)
    // (expert-major runs keep their weights live across rows, several
    // activation rows need the registers too)
    constexpr bool HOLD = NBW == 2 && !Q6 && MOE < 3 && XR == 1;
    v4i HA[HOLD ? NBW : 1][4];
    float2 HE[HOLD ? NBW : 1][2];
    if constexpr (HOLD) {
        // every lane reads, and the lanes whose A rows are zero mask the
        // words (no branch around the reads)
        const int mlo = a_lo ? -1 : 0, mhi = a_hi ? -1 : 0;
#pragma unroll
        for (int b = 0; b < NBW; b++) {
            const uint8_t *tb = tab + b * KT + a_off;
            const v4i r0 = lds_v4i(tb), r1 = lds_v4i(tb + 384);
            HA[b][0] = r0 & mlo;
            HA[b][1] = r1 & mlo;
            HA[b][2] = r0 & mhi;
            HA[b][3] = r1 & mhi;
            HE[b][0] = ex[b * 8 + gq];
            HE[b][1] = ex[b * 8 + 4 + gq];
        }
    }
    // group i is decoded after group i + LA is requested (LA: requests in
    // flight ahead of the decode; measured best with every request issued
    // before the first decode)
    // LT: the wave's slice buffer (rows in a ring of LTG::SR slots, so rows
    // 16.. may reuse the slots of rows 0.. once those are consumed)
    uint8_t *wbuf = lds + rstride + wv * (LTG::SR * LTG::SLB);
    auto lt_slot = [&](int r) { return r < LTG::SR ? r : r - LTG::SR; };
    int lt_put = 0;   // instructions written to the buffer so far
#pragma unroll
    for (int i = 0; i < NL; i++) {
        if (!LT && i + LA < NL && pr == pb && p0 == 0) issue(i + LA);
        __builtin_amdgcn_sched_barrier(0);
        const int rg = i / NBW, b = i - (i / NBW) * NBW;
        if constexpr (LT) {
            // the pieces of every row of row group rg into the buffer (one
            // wave's LDS operations complete in order)
            const int jend = ((16 * (rg + 1) < TR ? 16 * (rg + 1) : TR) * LTG::P + 63) / 64;
#pragma unroll
            for (int j = 0; j < LTG::NJ; j++) {
                if (j < lt_put || j >= jend) continue;
                const int q = 64 * j + lane;
                if (q < TR * LTG::P) {
                    const int r = q / LTG::P;
                    *reinterpret_cast<u32x4 *>(wbuf + lt_slot(r) * LTG::SLB + (q - r * LTG::P) * 16) = lv[j];
                }
            }
            lt_put = jend > lt_put ? jend : lt_put;
            int r = rg * 16 + c16;
            r = r < TR ? r : TR - 1;
            const uint8_t *sb = wbuf + lt_slot(r) * LTG::SLB + 16 * (LTG::P / NBW) * b;
            if constexpr (Q6) {
                // LDS block: bytes 0..207 in place, bytes 194..209 at 208..223:
                // the sixteen scales at 192 (this half's eight at 8 h), d at 222
                hd[i] = *reinterpret_cast<const u32x4 *>(sb + 64 * h6 + 16 * lh6);
                qa[i] = *reinterpret_cast<const u32x4 *>(sb + 64 * h6 + 32 + 16 * lh6);
                qb[i] = *reinterpret_cast<const u32x4 *>(sb + 128 + 32 * h6 + 16 * lh6);
                sc[i] = *reinterpret_cast<const u32x4 *>(sb + 192);
                dd6[i] = *reinterpret_cast<const uint32_t *>(sb + 220) >> 16;
                // a ragged slice's missing block: d = 0 and zero scales add
                // exactly zero
                if (kb0 + b >= nb) {
                    sc[i] = u32x4{0u, 0u, 0u, 0u};
                    dd6[i] = 0u;
                }
            } else if constexpr (Q80) {
                // lane group gq's blocks 2 gq, 2 gq + 1 at 68 gq of the
                // 272-byte group (4-byte aligned reads)
                u32x4 v0, v1, v2, v3;
                __builtin_memcpy(&v0, __builtin_assume_aligned(sb + 68 * gq, 4), 16);
                __builtin_memcpy(&v1, __builtin_assume_aligned(sb + 68 * gq + 16, 4), 16);
                __builtin_memcpy(&v2, __builtin_assume_aligned(sb + 68 * gq + 32, 4), 16);
                __builtin_memcpy(&v3, __builtin_assume_aligned(sb + 68 * gq + 48, 4), 16);
                hd[i] = v0;
                qa[i] = v1;
                qb[i] = v2;
                qc[i] = v3;
                dd[i] = *reinterpret_cast<const uint32_t *>(sb + 68 * gq + 64);
                if (kb0 + b >= nb) {
                    hd[i] = u32x4{0u, 0u, 0u, 0u};
                    qa[i] = hd[i];
                    qb[i] = hd[i];
                    qc[i] = hd[i];
                    dd[i] = 0u;
                }
            } else if constexpr (Q40) {
                // lane group gq's blocks 2 gq, 2 gq + 1 at 36 gq of the
                // 144-byte group (4-byte aligned reads)
                u32x4 a, c;
                __builtin_memcpy(&a, __builtin_assume_aligned(sb + 36 * gq, 4), 16);
                __builtin_memcpy(&c, __builtin_assume_aligned(sb + 36 * gq + 16, 4), 16);
                hd[i] = a;
                qa[i] = c;
                dd[i] = *reinterpret_cast<const uint32_t *>(sb + 36 * gq + 32);
                // a ragged slice's missing block: d = 0 (and zero codes)
                if (kb0 + b >= nb) {
                    hd[i] = u32x4{0u, 0u, 0u, 0u};
                    qa[i] = u32x4{0u, 0u, 0u, 0u};
                    dd[i] = 0u;
                }
            } else {
                hd[i] = *reinterpret_cast<const u32x4 *>(sb);
                qa[i] = *reinterpret_cast<const u32x4 *>(sb + 16 + 16 * gq);
                qb[i] = *reinterpret_cast<const u32x4 *>(sb + 80 + 16 * gq);
                // a ragged slice's missing block: d = dmin = 0 against zero
                // activations adds exactly zero (no branch between the groups)
                if (kb0 + b >= nb) hd[i] = u32x4{0u, 0u, 0u, 0u};
            }
        }
        if (!LT && kb0 + b >= nb) continue;   // wave-uniform: the ragged slice's missing blocks
        if constexpr (Q6) {
            // chunk qd of the block: in lane group gq = 2 h + l, the 16 values
            // 128 h + 32 qd + 16 l + i -- one scale group; code q = 4 low bits
            // from ql | 2 high bits from qh (dequant_q6_K, quant.cpp:491-512),
            // 0..63 as int8; the offset 32 through the 16-value sums of X:
            // S = sum (q - 32) X, |S| <= 16 * 32 * 2^22, exact in wrapping int32
            const u32x4 l0 = hd[i], l1 = qa[i], qh = qb[i];
            // d from a lane of half 1 (lane l ^ 32 or l itself)
            float d;
            uint32_t scx, scy;
            if constexpr (LT) {
                // (LDS copy: all sixteen scales from byte 192, d beside)
                d = h2f(dd6[i]);
                scx = h6 ? sc[i].z : sc[i].x;
                scy = h6 ? sc[i].w : sc[i].y;
            } else {
                d = h2f(__builtin_amdgcn_permlane32_swap(sc[i].w, sc[i].w, false, false)[1] >> 16);
                scx = h6 ? __builtin_amdgcn_alignbyte(sc[i].z, sc[i].y, 2) : sc[i].x;
                scy = h6 ? __builtin_amdgcn_alignbyte(sc[i].w, sc[i].z, 2) : sc[i].y;
            }
            float a = acc[rg];
#pragma unroll
            for (int qd = 0; qd < 4; qd++) {
                const u32x4 ql = (qd & 1) ? l1 : l0;
                const uint32_t ns = (qd >> 1) * 4u, hs = 2u * qd;
                const v4i B = {static_cast<int>(((ql.x >> ns) & M) | (((qh.x >> hs) & 0x03030303u) << 4)),
                               static_cast<int>(((ql.y >> ns) & M) | (((qh.y >> hs) & 0x03030303u) << 4)),
                               static_cast<int>(((ql.z >> ns) & M) | (((qh.z >> hs) & 0x03030303u) << 4)),
                               static_cast<int>(((ql.w >> ns) & M) | (((qh.w >> hs) & 0x03030303u) << 4))};
                // scale of group 8 h + 2 qd + l: byte 2 qd + l of the lane's eight
                const int jj = 2 * qd + lh6;
                const uint32_t sw = jj < 4 ? scx : scy;
                const float ds = d * static_cast<float>(static_cast<int8_t>(sw >> (8 * (jj & 3))));
                // A rows 4 gq + p: digit plane p of sub-block 4 h + qd, half l
                const v4i A = a6 ? lds_v4i(tab + b * KT + a6_off + qd * 96) : Z;
                const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, Z, 0, 0, 0);
                const int sbi = b * 8 + 4 * h6 + qd;
                const float2 h2 = ex16[sbi];
                const uint32_t xs = static_cast<uint32_t>(__float_as_int(lh6 ? h2.y : h2.x));
                const int S = static_cast<int>(static_cast<uint32_t>(C[0]) + (static_cast<uint32_t>(C[1]) << 8) +
                                               (static_cast<uint32_t>(C[2]) << 16) - 32u * xs);
                a = __builtin_fmaf(ds, ex[sbi].x * static_cast<float>(S), a);
            }
            acc[rg] = a;
            __builtin_amdgcn_sched_barrier(0);
            continue;
        }
        const uint8_t *tb = tab + b * KT;
        const int hb = HOLD ? b : 0;
        // A operands of one row's table at tbb: padded tables read every
        // lane's offset, plain ones select zeros for the lanes outside
        auto a_ops = [&](const uint8_t *tbb, v4i &a0l, v4i &a1l, v4i &a0h, v4i &a1h) {
            if constexpr (PAD) {
                a0l = lds_v4i(tbb + o_lo0);
                a1l = lds_v4i(tbb + o_lo1);
                a0h = lds_v4i(tbb + o_hi0);
                a1h = lds_v4i(tbb + o_hi1);
            } else {
                a0l = a_lo ? lds_v4i(tbb + a_off) : Z;
                a1l = a_lo ? lds_v4i(tbb + a_off + 384) : Z;
                a0h = a_hi ? lds_v4i(tbb + a_off) : Z;
                a1h = a_hi ? lds_v4i(tbb + a_off + 384) : Z;
            }
        };
        if constexpr (Q80) {
            // lane group gq holds blocks 2 gq, 2 gq + 1: {d, 32 int8 codes}
            // twice.  MFMA m of lane pair p = gq / 2 takes block 4 p + m, lane
            // 2 p its codes 0..15 and lane 2 p + 1 codes 16..31; the 16-lane
            // swap trades the halves and the scales between the two lanes
            const uint32_t W[17] = {hd[i].x, hd[i].y, hd[i].z, hd[i].w, qa[i].x, qa[i].y, qa[i].z, qa[i].w,
                                    qb[i].x, qb[i].y, qb[i].z, qb[i].w, qc[i].x, qc[i].y, qc[i].z, qc[i].w, dd[i]};
            uint32_t X[8], Y[8];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                X[k] = __builtin_amdgcn_alignbyte(W[k + 1], W[k], 2);
                Y[k] = __builtin_amdgcn_alignbyte(W[k + 5], W[k + 4], 2);
                X[4 + k] = W[9 + k];
                Y[4 + k] = W[13 + k];
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const auto sw = __builtin_amdgcn_permlane16_swap(X[k], Y[k], false, false);
                X[k] = sw[0];
                Y[k] = sw[1];
            }
            const auto dsw = __builtin_amdgcn_permlane16_swap(W[0] & 0xFFFFu, W[8] >> 16, false, false);
            auto codes = [&](const uint32_t *c) {
                return v4i{static_cast<int>(c[0]), static_cast<int>(c[1]), static_cast<int>(c[2]),
                           static_cast<int>(c[3])};
            };
            v4i A0l, A1l, A0h, A1h;
            if constexpr (HOLD) {
                A0l = HA[hb][0];
                A1l = HA[hb][1];
                A0h = HA[hb][2];
                A1h = HA[hb][3];
            } else {
                a_ops(tb, A0l, A1l, A0h, A1h);
            }
            const float2 ex0 = HOLD ? HE[hb][0] : ex[b * 8 + gq], ex1 = HOLD ? HE[hb][1] : ex[b * 8 + 4 + gq];
            v4i C0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0l, codes(X), Z, 0, 0, 0);
            C0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0h, codes(X + 4), C0, 0, 0, 0);
            v4i C1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1l, codes(Y), Z, 0, 0, 0);
            C1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1h, codes(Y + 4), C1, 0, 0, 0);
            // table slots gq and 4 + gq: d sum q x (dequant_q8_0,
            // src/quant.cpp:381-387); |sum q X| < 2^34, so the exact plane
            // sums are combined in f32
            const float s0 = __builtin_fmaf(65536.0f, static_cast<float>(C0[2]),
                                            __builtin_fmaf(256.0f, static_cast<float>(C0[1]), static_cast<float>(C0[0])));
            const float s1 = __builtin_fmaf(65536.0f, static_cast<float>(C1[2]),
                                            __builtin_fmaf(256.0f, static_cast<float>(C1[1]), static_cast<float>(C1[0])));
            float a = acc[rg];
            a = __builtin_fmaf(h2f(dsw[0]), ex0.x * s0, a);
            a = __builtin_fmaf(h2f(dsw[1]), ex1.x * s1, a);
            acc[rg] = a;
            __builtin_amdgcn_sched_barrier(0);
            continue;
        }
        if constexpr (Q40) {
            // lane group gq holds blocks 2 gq, 2 gq + 1: {d, 16 code bytes}
            // twice.  MFMA m of lane pair p = gq / 2 takes block 4 p + m, lane
            // 2 p its code bytes 0..7 and lane 2 p + 1 bytes 8..15 (low nibbles
            // = values j .. j + 7, high = j + 16 .. j + 23); the 16-lane swap
            // trades the halves and the scales between the two lanes
            const u32x4 L0 = hd[i], L1 = qa[i];
            const uint32_t L2 = dd[i];
            uint32_t X[4] = {__builtin_amdgcn_alignbyte(L0.y, L0.x, 2), __builtin_amdgcn_alignbyte(L0.z, L0.y, 2),
                             L1.y, L1.z};
            uint32_t Y[4] = {__builtin_amdgcn_alignbyte(L0.w, L0.z, 2), __builtin_amdgcn_alignbyte(L1.x, L0.w, 2),
                             L1.w, L2};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const auto sw = __builtin_amdgcn_permlane16_swap(X[k], Y[k], false, false);
                X[k] = sw[0];
                Y[k] = sw[1];
            }
            const auto dsw = __builtin_amdgcn_permlane16_swap(L0.x & 0xFFFFu, L1.x >> 16, false, false);
            auto codes = [&](uint32_t c0, uint32_t c1) {
                return v4i{static_cast<int>(c0 & M), static_cast<int>(c1 & M), static_cast<int>((c0 >> 4) & M),
                           static_cast<int>((c1 >> 4) & M)};
            };
            v4i A0l, A1l, A0h, A1h;
            if constexpr (HOLD) {
                A0l = HA[hb][0];
                A1l = HA[hb][1];
                A0h = HA[hb][2];
                A1h = HA[hb][3];
            } else {
                a_ops(tb, A0l, A1l, A0h, A1h);
            }
            const float2 ex0 = HOLD ? HE[hb][0] : ex[b * 8 + gq], ex1 = HOLD ? HE[hb][1] : ex[b * 8 + 4 + gq];
            v4i C0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0l, codes(X[0], X[1]), Z, 0, 0, 0);
            C0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0h, codes(X[2], X[3]), C0, 0, 0, 0);
            v4i C1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1l, codes(Y[0], Y[1]), Z, 0, 0, 0);
            C1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1h, codes(Y[2], Y[3]), C1, 0, 0, 0);
            // table slots gq and 4 + gq: the value d (q - 8) of
            // dequant_q4_0 (src/quant.cpp:331-339) as d (2^-e S - 8 sum x)
            const int S0 = C0[0] + (C0[1] << 8) + (C0[2] << 16);
            const int S1 = C1[0] + (C1[1] << 8) + (C1[2] << 16);
            float a = acc[rg];
            a = __builtin_fmaf(h2f(dsw[0]), __builtin_fmaf(ex0.x, static_cast<float>(S0), -8.0f * ex0.y), a);
            a = __builtin_fmaf(h2f(dsw[1]), __builtin_fmaf(ex1.x, static_cast<float>(S1), -8.0f * ex1.y), a);
            acc[rg] = a;
            __builtin_amdgcn_sched_barrier(0);
            continue;
        }
        v4i A0l, A1l, A0h, A1h;
        if constexpr (HOLD) {
            A0l = HA[hb][0];
            A1l = HA[hb][1];
            A0h = HA[hb][2];
            A1h = HA[hb][3];
        } else {
            a_ops(tb, A0l, A1l, A0h, A1h);
        }
        const float2 ex0 = HOLD ? HE[hb][0] : ex_blk(0, b)[gq], ex1 = HOLD ? HE[hb][1] : ex_blk(0, b)[4 + gq];
        const u32x4 h = hd[i], q0 = qa[i], q1 = qb[i];
        const v4i B0l = {static_cast<int>(q0.x & M), static_cast<int>(q0.y & M), static_cast<int>(q0.z & M),
                         static_cast<int>(q0.w & M)};
        const v4i B0h = {static_cast<int>((q0.x >> 4) & M), static_cast<int>((q0.y >> 4) & M),
                         static_cast<int>((q0.z >> 4) & M), static_cast<int>((q0.w >> 4) & M)};
        const v4i B1l = {static_cast<int>(q1.x & M), static_cast<int>(q1.y & M), static_cast<int>(q1.z & M),
                         static_cast<int>(q1.w & M)};
        const v4i B1h = {static_cast<int>((q1.x >> 4) & M), static_cast<int>((q1.y >> 4) & M),
                         static_cast<int>((q1.z >> 4) & M), static_cast<int>((q1.w >> 4) & M)};
        // scales and mins of sub-blocks gq and 4 + gq (get_scale_min_k4,
        // src/quant.cpp:427-435): byte gq of scales[0..3], [4..7], [8..11]
        const uint32_t s1 = h.y >> bsh, s2 = h.z >> bsh, s3 = h.w >> bsh;
        const float d = h2f(h.x & 0xFFFFu), dmin = h2f(h.x >> 16);
        const float sc0 = static_cast<float>(s1 & 63u), m0 = static_cast<float>(s2 & 63u);
        const float sc1 = static_cast<float>((s3 & 15u) | ((s1 >> 2) & 0x30u));
        const float m1 = static_cast<float>(((s3 >> 4) & 15u) | ((s2 >> 2) & 0x30u));
        // one activation row's digit planes against the group's codes
        auto row_dot = [&](const v4i &a0l, const v4i &a1l, const v4i &a0h, const v4i &a1h, const float2 &e0,
                           const float2 &e1, float a) {
            v4i C0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0l, B0l, Z, 0, 0, 0);
            C0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0h, B0h, C0, 0, 0, 0);
            v4i C1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1l, B1l, Z, 0, 0, 0);
            C1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1h, B1h, C1, 0, 0, 0);
            // lane (c16, gq): C rows 4 gq .. 4 gq + 2 are sub-block gq's (C0)
            // and 4 + gq's (C1) three plane sums for weight row c16
            const int S0 = C0[0] + (C0[1] << 8) + (C0[2] << 16);
            const int S1 = C1[0] + (C1[1] << 8) + (C1[2] << 16);
            a = __builtin_fmaf(d * sc0, e0.x * static_cast<float>(S0), a);
            a = __builtin_fmaf(-dmin * m0, e0.y, a);
            a = __builtin_fmaf(d * sc1, e1.x * static_cast<float>(S1), a);
            a = __builtin_fmaf(-dmin * m1, e1.y, a);
            return a;
        };
        if (p0 == 0) acc[rg] = row_dot(A0l, A1l, A0h, A1h, ex0, ex1, acc[rg]);
#pragma unroll
        for (int xr = p0 > 1 ? p0 : 1; xr < pend; xr++) {
            const float2 *ey = ex_blk(xr - p0, b);
            v4i a0l, a1l, a0h, a1h;
            a_ops(tab_of(xr - p0) + b * KT, a0l, a1l, a0h, a1h);
            accx[xr - 1][rg] = row_dot(a0l, a1l, a0h, a1h, ey[gq], ey[4 + gq], accx[xr - 1][rg]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    }   // passes of activation rows

    // ---- the waves' partial sums -> LDS [row][wave]; one thread per output
    // row adds them in wave order
#pragma unroll
    for (int xr = 0; xr < XR; xr++) {
    float *red = red_of(xr);
#pragma unroll
    for (int rg = 0; rg < RG; rg++) {
        // the sum over the four 16-lane rows by the cross-row swaps (VALU,
        // no LDS): a swap of v with itself leaves rows (0, 0, 2, 2) in one
        // result and (1, 1, 3, 3) in the other (16-lane swap), or (0, 1, 0,
        // 1) and (2, 3, 2, 3) (32-lane swap)
        float v = xr == 0 ? acc[rg] : accx[XR > 1 ? xr - 1 : 0][rg];
        const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
        const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
        if (gq == 0) red[(rg * 16 + c16) * nw + wv] = v;
    }
    }
    __syncthreads();
    for (int oi = static_cast<int>(threadIdx.x); oi < rows_t * XR; oi += 64 * nw) {
    const int xr = XR == 1 ? 0 : oi / rows_t;
    const int r = oi - xr * rows_t;
    if (n0 + r >= n_out) continue;
    const float *red = red_of(xr);
    auto row_sum = [&](int rr) {
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < NWMAX; k++)
            if (k < nw) v += red[rr * nw + k];
        return v;
    };
    OT *o = outp + (MOE >= 3 ? static_cast<int64_t>(pr) * t.em_orow : 0) + xr * t.out_stride + n0 + r;
    if (kind == SEG_SILU) {
        const float gs = row_sum(r), us = row_sum(16 + r);
        if constexpr (sizeof(OT) == 2) {
            // fused_gate_silu_kernel (fused.hpp:161-166): both dots rounded to
            // f16, activation in f32, saturated
            const float hg = static_cast<float>(static_cast<_Float16>(gs));
            const float hu = static_cast<float>(static_cast<_Float16>(us));
            *o = sat_f16(silu_f(hg) * hu);
        } else {
            *o = (gs / (1.0f + expf(-gs))) * us;   // silu_mul, backend_cpu.cpp:2401-2406
        }
    } else {
        store_out<OT>(o, row_sum(r), kind, acc_inv);
    }
    }   // output rows
    }
}


size_t stream_lds(int nw, int nbw, int xr = 1) {
    const size_t xp = xr > 5 ? 4 : xr;   // table slots: rows per pass
    const size_t per = xr > 1 ? kTabRows : kTab + 2 * 8 * sizeof(float2);
    return xp * nw * nbw * per + xr * 32 * static_cast<size_t>(nw) * sizeof(float);
}
// the load-transpose slice buffers of a launch
size_t stream_lt_lds(int nw, int nbw, int tr, int pb = 9) {
    const int p = pb * nbw, j0 = (16 * p + 63) / 64 - 1;
    const int sr0 = (64 * (j0 + 1) + p - 1) / p;
    const int sr = tr <= 16 ? tr : (sr0 < 16 ? 16 : sr0);
    return static_cast<size_t>(nw) * sr * 16 * pb * nbw;
}

template <int DT, typename XT, typename OT, int NBW, int TR, int MOE, int XR = 1>
hipError_t launch(const SegTable &t, int64_t tiles, int nw, hipStream_t st) {
    // Q4_K one-row launches of two-block slices (K <= 8192), and of
    // three-block slices in 16-row tiles (K <= 12288: the routed down
    // projection, 11008-wide rows), load their weights by load-transpose;
    // at sixteen waves the three-block buffers and tables take 156 KB of the
    // 160 KB of LDS
    // (Q6_K: two-block slices)
    // (expert-major runs keep their weights in registers across rows: the
    // gate/up pairs would spill beside the pieces in flight, and the down
    // projection measured 4% slower with it)
    // (Q4_0: its 256-value groups are 144 bytes like Q4_K's blocks; Q8_0's
    // 272-byte groups fit the LDS up to eight waves (K <= 4096), and sixteen
    // waves keep register loads)
    constexpr bool LT = XR == 1 && MOE < 3 &&
                        ((DT == DT_Q4_K && (NBW == 2 || (NBW == 3 && TR == 16))) ||
                         ((DT == DT_Q6_K || DT == DT_Q4_0 || DT == DT_Q8_0) && NBW == 2));
    constexpr bool LTW = LT && DT != DT_Q8_0;   // (over eight waves)
    const size_t l = stream_lds(nw, NBW, XR) +
                     ((nw <= 8 ? LT : LTW) ? stream_lt_lds(nw, NBW, TR, DT == DT_Q6_K ? 14 : DT == DT_Q8_0 ? 17 : 9) : 0);
    const dim3 grid(static_cast<unsigned>(tiles),
                    static_cast<unsigned>(MOE == 2 ? 1 : MOE >= 3 ? t.em_max_items : t.n));
    if (nw == 8)
        hipLaunchKernelGGL((gemv_stream_kernel<DT, XT, OT, NBW, TR, 8, true, MOE, 8, XR, LT>), grid, dim3(64 * nw), l, st,
                           t);
    else if (nw < 8)
        hipLaunchKernelGGL((gemv_stream_kernel<DT, XT, OT, NBW, TR, 8, false, MOE, 8, XR, LT>), grid, dim3(64 * nw), l, st,
                           t);
    else if (nw == kMaxWaves)
        hipLaunchKernelGGL((gemv_stream_kernel<DT, XT, OT, NBW, TR, kMaxWaves, true, MOE, 8, XR, LTW>), grid, dim3(64 * nw),
                           l, st, t);
    else
        hipLaunchKernelGGL((gemv_stream_kernel<DT, XT, OT, NBW, TR, kMaxWaves, false, MOE, 8, XR, LTW>), grid,
                           dim3(64 * nw), l, st, t);
    return hipGetLastError();
}

template <int DT, typename XT, typename OT, int NBW, int XR = 1>
hipError_t launch_tr(const SegTable &t, int tr, int64_t tiles, int nw, hipStream_t st) {
    if constexpr (NBW == 2) {
        switch (tr) {
            case 20: return launch<DT, XT, OT, NBW, 20, 0, XR>(t, tiles, nw, st);
            case 24: return launch<DT, XT, OT, NBW, 24, 0, XR>(t, tiles, nw, st);
            case 28: return launch<DT, XT, OT, NBW, 28, 0, XR>(t, tiles, nw, st);
            case 32: return launch<DT, XT, OT, NBW, 32, 0, XR>(t, tiles, nw, st);
            default: break;
        }
    }
    return launch<DT, XT, OT, NBW, 16, 0, XR>(t, tiles, nw, st);
}

template <int DT, typename XT, typename OT, int XR = 1>
hipError_t launch_nbw(int nbw, const SegTable &t, int tr, int64_t tiles, int nw, hipStream_t st) {
    switch (nbw) {
        case 2: return launch_tr<DT, XT, OT, 2, XR>(t, tr, tiles, nw, st);
        case 3: return launch_tr<DT, XT, OT, 3, XR>(t, tr, tiles, nw, st);
        default: return launch_tr<DT, XT, OT, 4, XR>(t, tr, tiles, nw, st);
    }
}

// blocks per wave: two when K has at most 32 blocks (eight waves for 4096),
// else as few as keep the waves at 16 per workgroup
int stream_nbw(int nb) { return nb <= 32 ? 2 : (nb + kMaxWaves - 1) / kMaxWaves; }

}  // namespace

int device_cus() {
    static thread_local int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cus = 256;
    }
    return cus;
}

bool gemv_stream_ok(int dt, const SegTable &t) {
    if ((dt != DT_Q4_K && dt != DT_Q6_K && dt != DT_Q4_0 && dt != DT_Q8_0) || t.rows < 1)
        return false;
    // (the load-transpose tiles address 32 rows within 32-bit offsets)
    if (t.row_bytes >= (int64_t{1} << 26)) return false;
    // several activation rows: dense Q4_K, up to kStreamRows, rows 16-byte aligned
    if (t.rows > 1 && (dt != DT_Q4_K || t.rows > kStreamRows || t.moe_tab || t.x_stride % 4)) return false;
    if (t.moe_tab) {
        // Q4_K banks; the down bank may also be Q6_K (Q4_K_M layers: its
        // 210-byte blocks need only 2-byte aligned rows)
        const bool down = t.moe_down || (t.em_runs && t.seg[0].kind == SEG_PLAIN);
        if (!(dt == DT_Q4_K || (dt == DT_Q6_K && down)) || t.n_in % 256 || t.row_bytes % (dt == DT_Q6_K ? 2 : 16))
            return false;
        const int nb = t.n_in / 256, nbw = stream_nbw(nb);
        if (t.em_runs) {
            // expert-major runs, Q4_K banks: gate/up pairs (n_in of at most
            // 32 blocks) or the down bank; 16-byte aligned activation rows
            const Seg &s0 = t.seg[0];
            return t.n == 1 && !t.moe_down && t.em_n_act && t.em_max_items > 0 &&
                   t.em_xrow % 4 == 0 && nb <= 4 * kMaxWaves && (reinterpret_cast<uintptr_t>(s0.x) & 15) == 0 &&
                   ((s0.kind == SEG_SILU && nbw == 2) || s0.kind == SEG_PLAIN);
        }
        // one routed token: gate/up pairs (one per slot, n_in of at most 32
        // blocks) or the down projection over the concatenated slots, each
        // wave's slice inside one slot
        if (t.moe_tokens > 1) return false;
        if (t.moe_down)
            return t.n == 1 && t.moe_k >= 1 && t.moe_kslot % 256 == 0 && t.n_in == t.moe_k * t.moe_kslot &&
                   (t.moe_kslot / 256) % nbw == 0 && nb <= 4 * kMaxWaves && t.seg[0].kind == SEG_PLAIN &&
                   (reinterpret_cast<uintptr_t>(t.seg[0].x) & 15) == 0;
        for (int i = 0; i < t.n; i++)
            if (t.seg[i].kind != SEG_SILU || t.seg[i].x != t.seg[0].x) return false;
        return nbw == 2 && (reinterpret_cast<uintptr_t>(t.seg[0].x) & 15) == 0;
    }
    // Q4_K rows, and Q4_0 / Q8_0 rows of whole 256-value groups, are 16-byte
    // multiples and start 16-byte aligned; Q6_K's 210-byte blocks need only
    // the 2-byte alignment of their f16 fields
    const uintptr_t wal = dt == DT_Q6_K ? 1 : 15;
    if (t.n_in % 256 || t.n_in > 256 * 4 * kMaxWaves || (t.row_bytes & static_cast<int64_t>(wal))) return false;
    const int nbw = stream_nbw(t.n_in / 256);
    // the one-shot tiles serve launches the resident workgroups cover in about
    // two rounds; a larger matrix (a vocabulary head) streams better through
    // the persistent row-split digit kernel, whose waves keep a ring of
    // units in flight from tile to tile
    int64_t rows = 0;
    for (int i = 0; i < t.n; i++) rows += t.seg[i].n_out;
    const int nw = (t.n_in / 256 + nbw - 1) / nbw;
    // (several rows: their digit tables within the 160 KB of LDS; five and
    // more rows on two-block slices)
    if (t.rows > 1 && (!t.xtab || stream_lds(nw, nbw, static_cast<int>(t.rows)) > kLdsMax ||
                       (t.rows > kStreamRowsWide && nbw != 2)))
        return false;
    // (one-row Q4_K and Q4_0 launches of two-block slices stream any
    // height: a 128256-row Q4_K head took 57.8 us here against 66.6 us on
    // the digit kernel, Q4_0 70.3 us against 82.3 on the VALU kernel; the
    // Q6_K head stays on the digit kernel (92 us against 95-110; 85.2
    // against 90.5 with 16-row tiles at two workgroups per CU), Q8_0's on
    // the VALU kernel (106 us against 113; with load-transpose 101.2 against
    // 103.7 on one box))
    if (rows > 2 * 32 * static_cast<int64_t>(device_cus()) * (nw <= 8 ? 2 : 1) &&
        !((dt == DT_Q4_K || dt == DT_Q4_0) && nbw == 2 && t.rows == 1))
        return false;
    for (int i = 0; i < t.n; i++) {
        const Seg &s = t.seg[i];
        // gate/up pairs take two row groups, which wider slices cannot afford
        if (s.kind == SEG_SILU && nbw > 2) return false;
        if (s.x != t.seg[0].x || (reinterpret_cast<uintptr_t>(s.x) & 15) ||
            (reinterpret_cast<uintptr_t>(s.w) & wal))
            return false;
        if (s.kind == SEG_SILU && (reinterpret_cast<uintptr_t>(s.w2) & wal)) return false;
    }
    return true;
}

size_t gemv_stream_xtab_bytes(int64_t rows, int64_t n_in) {
    const int nb = static_cast<int>(n_in / 256);
    if (rows < 2 || nb < 1) return 0;
    const int nbw = stream_nbw(nb);
    const int nw = (nb + nbw - 1) / nbw;
    return static_cast<size_t>(rows) * nw * nbw * kTabRows;
}

hipError_t gemv_stream(int dt, bool act_f16, const SegTable &t0, hipStream_t st) {
    SegTable t = t0;
    const int nb = t.n_in / 256;
    const int nbw = stream_nbw(nb);
    const int nw = (nb + nbw - 1) / nbw;
    if (t.moe_tab) {
        // routed experts (f32 activations, Q4_K): gate/up pairs take 32-row
        // tiles (16 + 16), the down projection 16-row tiles when its slices
        // are wider than two blocks
        if (act_f16 || !(dt == DT_Q4_K || dt == DT_Q6_K)) return hipErrorNotSupported;
        if (dt == DT_Q6_K) {   // the down bank of a Q4_K_M layer
            if (t.em_runs) {
                if (t.seg[0].kind == SEG_SILU) return hipErrorNotSupported;
                const int64_t width = (t.seg[0].n_out + 15) / 16;
                switch (nbw) {
                    case 2: return launch<DT_Q6_K, float, float, 2, 16, 4>(t, width, nw, st);
                    case 3: return launch<DT_Q6_K, float, float, 3, 16, 4>(t, width, nw, st);
                    default: return launch<DT_Q6_K, float, float, 4, 16, 4>(t, width, nw, st);
                }
            }
            if (!t.moe_down) return hipErrorNotSupported;
            const int64_t width = (t.seg[0].n_out + 15) / 16;
            switch (nbw) {
                case 2: return launch<DT_Q6_K, float, float, 2, 16, 2>(t, width, nw, st);
                case 3: return launch<DT_Q6_K, float, float, 3, 16, 2>(t, width, nw, st);
                default: return launch<DT_Q6_K, float, float, 4, 16, 2>(t, width, nw, st);
            }
        }
        if (t.em_runs) {
            if (t.seg[0].kind == SEG_SILU)
                return launch<DT_Q4_K, float, float, 2, 32, 3>(t, (t.seg[0].n_out + 15) / 16, nw, st);
            const int64_t width = (t.seg[0].n_out + 15) / 16;
            switch (nbw) {
                case 2: return launch<DT_Q4_K, float, float, 2, 16, 4>(t, width, nw, st);
                case 3: return launch<DT_Q4_K, float, float, 3, 16, 4>(t, width, nw, st);
                default: return launch<DT_Q4_K, float, float, 4, 16, 4>(t, width, nw, st);
            }
        }
        if (!t.moe_down) {
            const int64_t width = (t.seg[0].n_out + 15) / 16;
            return launch<DT_Q4_K, float, float, 2, 32, 1>(t, width, nw, st);
        }
        const int64_t cap = static_cast<int64_t>(device_cus()) * (nw <= 8 ? 2 : 1);
        int tr = 16;
        if (nbw == 2) {
            int64_t best = INT64_MAX;
            for (int c = 16; c <= 32; c += 4) {
                const int64_t cost = ((t.seg[0].n_out + c - 1) / c + cap - 1) / cap * c;
                if (cost < best) { best = cost; tr = c; }
            }
        }
        const int64_t width = (t.seg[0].n_out + tr - 1) / tr;
        switch (nbw) {
            case 2:
                switch (tr) {
                    case 20: return launch<DT_Q4_K, float, float, 2, 20, 2>(t, width, nw, st);
                    case 24: return launch<DT_Q4_K, float, float, 2, 24, 2>(t, width, nw, st);
                    case 28: return launch<DT_Q4_K, float, float, 2, 28, 2>(t, width, nw, st);
                    case 32: return launch<DT_Q4_K, float, float, 2, 32, 2>(t, width, nw, st);
                    default: return launch<DT_Q4_K, float, float, 2, 16, 2>(t, width, nw, st);
                }
            case 3: return launch<DT_Q4_K, float, float, 3, 16, 2>(t, width, nw, st);
            default: return launch<DT_Q4_K, float, float, 4, 16, 2>(t, width, nw, st);
        }
    }
    bool has_pair = false;
    for (int i = 0; i < t.n; i++) has_pair |= t.seg[i].kind == SEG_SILU;
    // tile height: among 16, 20, .., 32 (32 with gate/up pairs, which need
    // two row groups; 16 for slices of more than two blocks, whose registers
    // hold one row group), the one whose tiles fill the resident workgroups
    // (two per CU at up to eight waves) in the fewest rounds x rows
    // (workgroups per CU: two at up to eight waves, fewer when several rows'
    // tables fill the LDS)
    // (load-transpose buffers: one-row launches of two-block slices, and
    // Q4_K's three-block slices, whose tiles are 16 rows)
    const bool lt = t.rows == 1 && ((nbw == 2 && (dt != DT_Q8_0 || nw <= 8)) || (dt == DT_Q4_K && nbw == 3));
    const size_t lds1 = stream_lds(nw, nbw, static_cast<int>(t.rows)) +
                        (lt ? stream_lt_lds(nw, nbw, 32, dt == DT_Q6_K ? 14 : dt == DT_Q8_0 ? 17 : 9) : 0);
    const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(nw <= 8 ? 2 : 1, static_cast<int64_t>(kLdsMax / lds1)));
    const int64_t cap = static_cast<int64_t>(device_cus()) * per_cu;
    int tr = 16;
    int64_t best = INT64_MAX;
    // (six to eight rows: 16-row tiles; taller ones spill 25-27 registers at
    // the four waves per SIMD these rows run at, 27-40 us against 20 at 8 rows)
    for (int c = has_pair ? 32 : 16; c <= (nbw > 2 || t.rows > 5 ? 16 : 32); c += 4) {
        int64_t tiles = 0;
        for (int i = 0; i < t.n; i++) {
            const int rows_t = t.seg[i].kind == SEG_SILU ? 16 : c;
            tiles += (t.seg[i].n_out + rows_t - 1) / rows_t;
        }
        // (Q6_K's one-row load-transpose tiles above 16 rows hold 135
        // registers a lane: one workgroup per CU)
        const int64_t capc = dt == DT_Q6_K && lt && c > 16 ? static_cast<int64_t>(device_cus()) : cap;
        const int64_t cost = (tiles + capc - 1) / capc * c;
        if (cost < best) { best = cost; tr = c; }
    }
    // the grid: one row of tiles per segment, as wide as the longest
    int64_t width = 0;
    for (int i = 0; i < t.n; i++) {
        const int64_t rows_t = t.seg[i].kind == SEG_SILU ? 16 : tr;
        const int64_t n = (t.seg[i].n_out + rows_t - 1) / rows_t;
        width = n > width ? n : width;
    }
    if (width >= (int64_t{1} << 31) || t.n < 1) return hipErrorNotSupported;
    if (dt == DT_Q6_K)
        return act_f16 ? launch_nbw<DT_Q6_K, _Float16, _Float16>(nbw, t, tr, width, nw, st)
                       : launch_nbw<DT_Q6_K, float, float>(nbw, t, tr, width, nw, st);
    if (dt == DT_Q4_0)
        return act_f16 ? launch_nbw<DT_Q4_0, _Float16, _Float16>(nbw, t, tr, width, nw, st)
                       : launch_nbw<DT_Q4_0, float, float>(nbw, t, tr, width, nw, st);
    if (dt == DT_Q8_0)
        return act_f16 ? launch_nbw<DT_Q8_0, _Float16, _Float16>(nbw, t, tr, width, nw, st)
                       : launch_nbw<DT_Q8_0, float, float>(nbw, t, tr, width, nw, st);

    if (t.rows > 1) {
        // the rows' digit tables, once for every workgroup of the launch
        const int nbp = nw * nbw;
        const dim3 xg(static_cast<unsigned>((nbp + 1) / 2), static_cast<unsigned>(t.rows));
        if (act_f16)
            hipLaunchKernelGGL(stream_xtab_kernel<_Float16>, xg, dim3(64), 0, st,
                               static_cast<const _Float16 *>(t.seg[0].x), t.x_stride, nb, nbp, t.xtab);
        else
            hipLaunchKernelGGL(stream_xtab_kernel<float>, xg, dim3(64), 0, st, static_cast<const float *>(t.seg[0].x),
                               t.x_stride, nb, nbp, t.xtab);
        if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    }
    switch (t.rows) {
        case 2:
            return act_f16 ? launch_nbw<DT_Q4_K, _Float16, _Float16, 2>(nbw, t, tr, width, nw, st)
                           : launch_nbw<DT_Q4_K, float, float, 2>(nbw, t, tr, width, nw, st);
        case 3:
            return act_f16 ? launch_nbw<DT_Q4_K, _Float16, _Float16, 3>(nbw, t, tr, width, nw, st)
                           : launch_nbw<DT_Q4_K, float, float, 3>(nbw, t, tr, width, nw, st);
        case 4:
            return act_f16 ? launch_nbw<DT_Q4_K, _Float16, _Float16, 4>(nbw, t, tr, width, nw, st)
                           : launch_nbw<DT_Q4_K, float, float, 4>(nbw, t, tr, width, nw, st);
        // five to eight rows: two-block slices only (gemv_stream_ok)
        case 5:
            return act_f16 ? launch_tr<DT_Q4_K, _Float16, _Float16, 2, 5>(t, tr, width, nw, st)
                           : launch_tr<DT_Q4_K, float, float, 2, 5>(t, tr, width, nw, st);
        case 6:
            return act_f16 ? launch_tr<DT_Q4_K, _Float16, _Float16, 2, 6>(t, tr, width, nw, st)
                           : launch_tr<DT_Q4_K, float, float, 2, 6>(t, tr, width, nw, st);
        case 7:
            return act_f16 ? launch_tr<DT_Q4_K, _Float16, _Float16, 2, 7>(t, tr, width, nw, st)
                           : launch_tr<DT_Q4_K, float, float, 2, 7>(t, tr, width, nw, st);
        case 8:
            return act_f16 ? launch_tr<DT_Q4_K, _Float16, _Float16, 2, 8>(t, tr, width, nw, st)
                           : launch_tr<DT_Q4_K, float, float, 2, 8>(t, tr, width, nw, st);
        default: break;
    }
    return act_f16 ? launch_nbw<DT_Q4_K, _Float16, _Float16>(nbw, t, tr, width, nw, st)
                   : launch_nbw<DT_Q4_K, float, float>(nbw, t, tr, width, nw, st);
}

}  // namespace krk
