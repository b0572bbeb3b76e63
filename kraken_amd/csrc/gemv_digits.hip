// gemv_digits.hip -- Q4_K and Q6_K decode GEMV on the int8 matrix cores.
//
// Decode GEMV (rows == 1) is bound by HBM, but with a 4-bit format the VALU
// work of a dequantize-and-FMA loop (one v_fma_mix per weight plus the
// nibble unpacking, scales and reductions: ~2.8 VALU ops per weight) costs
// as much time as the bytes.  Here the products run on the int8 MFMA:
//
//   * B operand: the weight codes themselves.  Sixteen low (or high)
//     nibbles of a lane's four code dwords are sixteen int8 values after a
//     single AND (and a shift for the high ones): 0.375 VALU ops per weight.
//   * A operand: the activations as exact integers.  Each 32-value
//     sub-block of x is scaled by a power of two so that its largest value
//     has 22 bits, rounded to an integer X (error <= 2^-22 of the sub-block
//     maximum) and split into three balanced int8 digits,
//     X = d0 + 2^8 d1 + 2^16 d2.  Rows 4s'+p of A hold digit plane p of
//     sub-block s', zero elsewhere, so one 16x16x64 MFMA yields for every
//     weight row (column) and sub-block the three exact int32 plane sums.
//   * The Q4_K block formula (src/quant.cpp:427-447, dequant_q4_K with
//     get_scale_min_k4) is applied to the plane sums once per (row,
//     sub-block):  y += d*sc * 2^-e * (C0 + 2^8 C1 + 2^16 C2) - dmin*m * sum(x).
//
// The products are exact; the result differs from the f32 reference chain
// only by the 2^-22 activation rounding and f32 accumulation order, far
// inside the 1e-5 relative budget.
//
// Data movement: each wave streams units of ROWS rows x 256*KB values
// (ROWS row pieces of KB*144 contiguous bytes) into a private LDS slot
// with global_load_lds_dwordx4 -- every weight byte is delivered once and
// coalesced -- while the digit table of x is built once per workgroup.
// NSLOT slots keep NSLOT-1 units in flight during the decode.
#include <cstdint>

#include "gemv_core.hpp"
#include "krk_formats.hpp"
#include "krk_kernels.hpp"
#include "krk_mi355x.h"

namespace krk {

namespace {


typedef __attribute__((address_space(3))) void lds_void_t;
typedef int v4i __attribute__((ext_vector_type(4)));

template <int N> __device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    // s_waitcnt simm16: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

constexpr int kTabBlk = 768;   // digit bytes per 256-value block: 8 sub-blocks x 3 planes x 32
constexpr int kZero = 512;     // zero bytes read by lanes whose A row is empty
constexpr int kMaxK = 16384;
constexpr int kMaxDownSlots = 16;
static_assert(sizeof(Seg) * (kMaxSegs - 1) >= kMaxDownSlots * (sizeof(void *) + sizeof(float)),
              "down-mode slot table fits in the segment table");
constexpr int kXPasses = 8;    // x sub-blocks staged per thread (4 threads per sub-block)
constexpr int kRedWaves = 8;   // reduction slots per row (waves per workgroup <= 8)
// Waves that issue their first weight DMA only after building the digit
// table: a wave stalls while the memory pipeline cannot accept its DMA, and
// these keep the table build moving meanwhile (measured: 4 of 8 best).
constexpr int kLateWaves = 4;

__device__ __forceinline__ v4i ld_v4i(const uint8_t *p) { return *reinterpret_cast<const v4i *>(p); }

// LDS-DMA of N bytes per lane (the builtin needs a literal size)
template <int N> __device__ __forceinline__ void dma_lds(const void *src, uint8_t *dst);
template <> __device__ __forceinline__ void dma_lds<16>(const void *src, uint8_t *dst) {
    __builtin_amdgcn_global_load_lds(src, (lds_void_t *)dst, 16, 0, 0);
}

template <int DT, typename XT, typename OT, int ROWS, int KB, int NSLOT, bool DOWN, int NX, bool MT, bool RSPLIT>
__global__ void __launch_bounds__(512) gemv_digits_kernel(SegTable t, int64_t total, int nks, int nwc) {
    constexpr bool Q6 = DT == DT_Q6_K;
    // 32-value formats: 8 blocks per 256 values, each in an LDS slot of
    // 16-byte windows taken inside the block (Q8_0: 34 -> 48 bytes, Q4_0:
    // 18 -> 32), so the codes sit 16-byte aligned at slot offset 16
    constexpr bool QS = DT == DT_Q8_0 || DT == DT_Q4_0;
    constexpr bool Q8 = DT == DT_Q8_0;
    constexpr int bb = Q8 ? 34 : 18, sbl = Q8 ? 48 : 32;   // QS block bytes, LDS slot
    constexpr int BB = Q6 ? 210 : QS ? 8 * bb : 144;       // source bytes per 256 values
    constexpr int P = KB * BB;                   // row piece of one unit
    constexpr int RGN = (ROWS + 15) / 16;        // 16-row MFMA groups (the last may be partial)
    constexpr int RS = 16 * RGN;                 // reduction stride
    // LDS unit layout: row r at r * PL, delivered by dwordx4 LDS-DMA.  Q4_K
    // pieces are 16-byte multiples.  Q6_K blocks (210 bytes) go to a 224-byte
    // stride so every LDS read is 16-byte aligned: each lane picks its own
    // 16-byte source window inside its block (sources are 2-byte aligned),
    // so no byte outside the matrix is ever read.
    constexpr int BL = Q6 ? 224 : QS ? 8 * sbl : BB;   // LDS bytes per 256 values
    constexpr int PL = KB * BL;                  // LDS row stride
    constexpr int U = ROWS * PL;
    constexpr int DMA = 16;                      // bytes per lane per LDS-DMA instruction
    constexpr int CHB = 64 * DMA;                // bytes per instruction
    constexpr int CH = (U + CHB - 1) / CHB;
    constexpr int SLOT = ((U + 1023) / 1024) * 1024;
    static_assert(NSLOT * CH < 64, "vmcnt is 6 bits");
    static_assert(!(Q6 || QS) || (!DOWN && !MT), "Q6_K, Q8_0, Q4_0: plain segments");
    const int64_t nrows = t.rows;   // activation rows of this launch
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ Seg segl[kMaxSegs];
    // down mode uses segl[0] only; the bank and the weight of each slot live
    // in segl[1..] (the LDS budget is full: 8 waves take all but this table)
    const uint8_t **bankl = reinterpret_cast<const uint8_t **>(&segl[1]);
    float *wl = reinterpret_cast<float *>(bankl + kMaxDownSlots);
    const int nb = t.n_in / 256;
    // NX activation rows share every weight unit: one digit table per row
    const int tstride = nb * kTabBlk;                 // bytes of one row's table
    uint8_t *tab = lds;                               // [NX][nb][8][3][32] int8 digits
    uint8_t *zero = tab + NX * tstride;               // kZero zero bytes
    float2 *ex = reinterpret_cast<float2 *>(zero + kZero);  // [NX][nb * 8] {2^-e, sum x}
    // Q6_K: exact integer sums of X over each 16-value half of a sub-block
    // (for the code offset 32), stored as int bits
    float2 *ex16 = ex + NX * nb * 8;                  // [NX][nb * 8] (Q6_K only)
    uint8_t *slots0 = reinterpret_cast<uint8_t *>(ex + (Q6 || DT == DT_Q4_0 ? 2 : 1) * NX * nb * 8);
    float *red = reinterpret_cast<float *>(slots0 + nwc * (NSLOT * SLOT));  // [2][NX][RS][kRedWaves]

    // Every wave streams, multiplies and builds a share of the digit table.
    // The vector-memory counter of a wave is in order, so each wave issues
    // its x loads FIRST, then its weight DMA, and waits only until the DMA
    // instructions remain outstanding: x has then arrived, the weights keep
    // streaming while the table is built.
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t *slots = slots0 + wv * (NSLOT * SLOT);
    const int64_t rb = t.row_bytes;
    // A workgroup owns tiles of ROWS rows (tiles lb, lb + nlb, ...); its
    // waves split K: wave wv takes the units ks = wv, wv + nwc, ...  With
    // several routed tokens, workgroup group tok serves token tok.
    constexpr bool multi = MT;   // several routed tokens
    const int nlb = MT ? t.moe_wpt : static_cast<int>(gridDim.x);
    const int tok = multi ? static_cast<int>(blockIdx.x) / nlb : 0;
    const int lb = multi ? static_cast<int>(blockIdx.x) - tok * nlb : static_cast<int>(blockIdx.x);
    // Row split (chosen when there are many tiles): each wave owns whole
    // tiles (all K units), so no cross-wave reduction is needed.
    constexpr bool rsplit = RSPLIT;
    // tile and unit counts fit 31 bits (the launch checks total * nks), so
    // the per-unit index arithmetic stays in 32-bit scalar registers
    const int wid = rsplit ? lb * nwc + wv : lb;
    const int wstride = rsplit ? nlb * nwc : nlb;
    const int ntiles = static_cast<int>(total);
    const int my_tiles =
        wid < ntiles ? static_cast<int>(static_cast<uint32_t>(ntiles - 1 - wid) / static_cast<uint32_t>(wstride)) + 1
                     : 0;
    const int cnt = rsplit ? nks : (wv < nks ? (nks - 1 - wv) / nwc + 1 : 0);
    const int my_units = my_tiles * cnt;

    const int nseg = t.n;
    const int upk = DOWN ? static_cast<int>(t.moe_kslot / (KB * 256)) : 1;   // units per slot
    auto seg_w = [&](int64_t g, const Seg *tab_) {
        int i = 0;
        while (i + 1 < nseg && g >= tab_[i + 1].blk_begin) i++;
        return i;
    };

    // chunk c, lane l: slot bytes [1024c + 16l, +16) = tile row r = o / P at
    // offset o % P.  Rows 0..15 come from base 0, rows 16..31 from base 1:
    // the next 16 rows of the same matrix, or for a gate/up (SiLU) segment
    // the same 16 rows of the up matrix.
    // source offset, inside the row piece, of LDS offset rem of a row.
    // Q6_K: windows 0..12 of a block are its bytes 0..207; window 13 (LDS
    // 208..223) takes bytes 194..209, so d sits at LDS 222
    // QS: window 0 of a block is bytes 0..15 (d first), window 1 bytes
    // 2..17 (codes 0..15), Q8_0's window 2 bytes 18..33 (codes 16..31)
    auto src_off = [](int rem) {
        if constexpr (Q6) {
            const int b = rem / BL, off = rem - b * BL;
            return b * BB + (off < BB - 2 ? off : BB - 16);
        } else if constexpr (QS) {
            const int b = rem / sbl, w = (rem - b * sbl) >> 4;
            return b * bb + (w == 0 ? 0 : w == 1 ? 2 : 18);
        } else {
            return rem;
        }
    };
    int32_t dl[CH];
    uint32_t hi_rows = 0;   // bit c: this lane's chunk c lies in rows 16..31
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int o = c * CHB + DMA * lane;
        const int r = o < U ? o / PL : 0;
        dl[c] = o < U ? static_cast<int32_t>((r & 15) * rb + src_off(o - r * PL)) : 0;
        if (r >= 16) hi_rows |= 1u << c;
    }
    // the first units read the segment table from the kernel arguments (the
    // LDS copy is not ready yet); later ones from LDS
    auto issue = [&](int j, const Seg *tab_) {
        const int jt = static_cast<int>(static_cast<uint32_t>(j) / static_cast<uint32_t>(cnt)), jk = j - jt * cnt;
        const int64_t g = wid + static_cast<int64_t>(jt) * wstride;
        const int ks = rsplit ? jk : wv + jk * nwc;
        const int si = seg_w(g, tab_);
        const bool pair = tab_[si].kind == SEG_SILU;
        const int tr = pair ? 16 : ROWS;               // output rows per tile
        const uint8_t *w;
        int64_t k0;
        if constexpr (DOWN) {
            // the unit's slot and its offset inside that slot's bank row
            const int sl = ks / upk;
            w = bankl[sl];
            k0 = static_cast<int64_t>(ks - sl * upk) * P;
        } else {
            w = static_cast<const uint8_t *>(tab_[si].w);
            k0 = static_cast<int64_t>(ks) * P;
        }
        const uint8_t *w1 = pair ? static_cast<const uint8_t *>(tab_[si].w2) : w + 16 * rb;
        const int64_t n_out = tab_[si].n_out;
        const int64_t n0 = (g - tab_[si].blk_begin) * tr;
        uint8_t *dst = slots + static_cast<int>(j % NSLOT) * SLOT;
        if ((n0 + tr - 1) * rb + k0 + P <= n_out * rb) {
            const uint8_t *b0 = w + n0 * rb + k0, *b1 = w1 + n0 * rb + k0;
#pragma unroll
            for (int c = 0; c < CH; c++)
                dma_lds<DMA>(static_cast<const void *>(((hi_rows >> c) & 1 ? b1 : b0) + dl[c]), dst + c * CHB);
        } else {
            // the matrix's last rows: clamp rows and row ends to stay inside
            const int64_t lim = rb - DMA;
#pragma unroll
            for (int c = 0; c < CH; c++) {
                const int o = c * CHB + DMA * lane;
                const int r = o < U ? o / PL : 0;
                const bool up = pair && r >= 16;
                int64_t n = n0 + (pair ? (r & 15) : r);
                if (n >= n_out) n = n_out - 1;
                int64_t off = k0 + (o < U ? src_off(o - r * PL) : 0);
                if (off > lim) off = lim;
                dma_lds<DMA>(static_cast<const void *>((up ? w1 : w) + n * rb + off), dst + c * CHB);
            }
        }
    };

    // ---- x loads (four threads per 32-value sub-block, kXPasses passes over
    // the NX rows' sub-blocks; rows past nrows read as zero)
    const XT *x = static_cast<const XT *>(t.seg[0].x) + (MT ? tok * t.moe_xtok : 0);
    // activation row r of this launch
    auto xrow_off = [&](int r) -> int64_t { return static_cast<int64_t>(r) * t.x_stride; };
    const int q = threadIdx.x & 3;
    const int nsb = nb * 8;
    const int nxs = NX * nsb;
    float xv[kXPasses][8];
#pragma unroll
    for (int u = 0; u < kXPasses; u++) {
        const int f = (threadIdx.x >> 2) + u * (blockDim.x >> 2);
        const int xr = NX > 1 ? f / nsb : 0, sb = NX > 1 ? f - xr * nsb : f;
        const bool xin = f < nxs && xr < nrows;
        const XT *xp = x + (xin ? xrow_off(xr) + sb * 32 : 0) + 8 * q;
        if (u * (blockDim.x >> 2) >= nxs) break;   // uniform
        if (NX > 1 && !xin) {
#pragma unroll
            for (int k = 0; k < 8; k++) xv[u][k] = 0.0f;
        } else if constexpr (sizeof(XT) == 4) {
            const floatx4 u0 = *reinterpret_cast<const floatx4 *>(xp);
            const floatx4 u1 = *reinterpret_cast<const floatx4 *>(xp + 4);
            xv[u][0] = u0.x; xv[u][1] = u0.y; xv[u][2] = u0.z; xv[u][3] = u0.w;
            xv[u][4] = u1.x; xv[u][5] = u1.y; xv[u][6] = u1.z; xv[u][7] = u1.w;
        } else {
            const half8 h = *reinterpret_cast<const half8 *>(xp);
#pragma unroll
            for (int k = 0; k < 8; k++) xv[u][k] = static_cast<float>(h[k]);
        }
    }
    // ---- routed experts: resolve the segments on the device first (one
    // dependent read of the ids and the table entries per workgroup)
    const bool moe = t.moe_tab != nullptr;
    if (DOWN) {
        if (threadIdx.x < t.moe_k) {
            const krk_moe_entry *mt = static_cast<const krk_moe_entry *>(t.moe_tab);
            const int64_t pi = static_cast<int64_t>(tok) * t.moe_k + threadIdx.x;
            const int e = t.moe_ids[pi];
            const bool live = e >= 0 && e < t.moe_ne;
            bankl[threadIdx.x] = static_cast<const uint8_t *>(mt[live ? e : 0].p[KRK_MOE_DOWN]);
            wl[threadIdx.x] = live ? t.moe_wts[pi] : 0.0f;
        }
        if (threadIdx.x == 0) {
            Seg sg = t.seg[0];
            if (multi) sg.out = static_cast<float *>(sg.out) + tok * t.moe_otok;
            segl[0] = sg;
        }
        __syncthreads();
    } else if (moe) {
        if (threadIdx.x < nseg) {
            const int32_t *ids = t.moe_ids + static_cast<int64_t>(tok) * nseg;
            const krk_moe_entry *mt = static_cast<const krk_moe_entry *>(t.moe_tab);
            int e = ids[threadIdx.x];
            const bool live = e >= 0 && e < t.moe_ne;
            // segments in ascending expert id (dropped slots last): tokens
            // sharing an expert then stream it at about the same time
            int rank = 0;
            for (int i = 0; i < nseg; i++) {
                const int o = ids[i];
                const bool ol = o >= 0 && o < t.moe_ne;
                const bool before = live ? (ol && (o < e || (o == e && i < static_cast<int>(threadIdx.x))))
                                         : (ol || i < static_cast<int>(threadIdx.x));
                rank += before ? 1 : 0;
            }
            if (!live) e = 0;   // a dropped slot: any bank, its row is never read
            Seg sg = t.seg[threadIdx.x];
            sg.w = mt[e].p[KRK_MOE_GATE];
            sg.w2 = mt[e].p[KRK_MOE_UP];
            sg.out = static_cast<float *>(t.seg[0].out) + (multi ? tok * t.moe_otok : 0) +
                     static_cast<int64_t>(threadIdx.x) * t.seg[0].n_out;
            sg.blk_begin = t.seg[rank].blk_begin;   // equal segments: the tile ranges are the same
            segl[rank] = sg;
        }
        __syncthreads();
    }

    // ---- weight DMA of the first NSLOT units, then wait for x only.  The
    // last `late` waves issue theirs after the table: a wave stalls while
    // the memory pipeline cannot take its DMA, and those waves build the
    // table meanwhile.
    const int late = kLateWaves < nwc / 2 ? kLateWaves : nwc / 2;
    const bool early = wv < nwc - late;
    const int first = my_units < NSLOT ? my_units : NSLOT;
    if (early) {
        if (moe) {
#pragma unroll
            for (int k = 0; k < NSLOT; k++)
                if (k < first) issue(k, segl);
        } else {
#pragma unroll
            for (int k = 0; k < NSLOT; k++)
                if (k < first) issue(k, t.seg);
        }
        if (first >= 2) wait_vm<2 * CH>();
        else if (first == 1) wait_vm<CH>();
        else wait_vm<0>();
    } else {
        wait_vm<0>();
    }

    // ---- digit table of x
    for (int i = threadIdx.x; i < kZero / 4; i += blockDim.x) reinterpret_cast<uint32_t *>(zero)[i] = 0u;
#pragma unroll
    for (int u = 0; u < kXPasses; u++) {
        const int f = (threadIdx.x >> 2) + u * (blockDim.x >> 2);
        const int xr = NX > 1 ? f / nsb : 0, sb = NX > 1 ? f - xr * nsb : f;
        if (u * (blockDim.x >> 2) >= nxs) break;   // uniform
        const float *v = xv[u];
        float amax = 0.0f, sum = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            amax = fmaxf(amax, fabsf(v[k]));
            sum += v[k];
        }
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);
        if (f >= nxs) continue;
        // 2^e with |x| * 2^e < 2^22: from amax's exponent field E (amax in
        // [2^(E-127), 2^(E-126))), e = 148 - E puts amax * 2^e in
        // [2^21, 2^22), so the top digit stays within [-64, 64]; kept where
        // 2^e and 2^-e are normal floats; zero and non-finite sub-blocks get
        // no digits
        const uint32_t Eb = (__float_as_uint(amax) >> 23) & 255u;
        const bool live = amax > 0.0f && Eb < 255u;
        int e = live ? 148 - static_cast<int>(Eb) : 0;
        e = e > 126 ? 126 : e;
        const float up = __uint_as_float(static_cast<uint32_t>(127 + e) << 23);
        const float dn = __uint_as_float(static_cast<uint32_t>(127 - e) << 23);
        uint32_t p0[2] = {0u, 0u}, p1[2] = {0u, 0u}, p2[2] = {0u, 0u};
        int xsum = 0;   // Q6_K: exact integer sum of this thread's 8 X
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int X = live ? static_cast<int>(__builtin_rintf(v[k] * up)) : 0;
            xsum += X;
            const int d0 = ((X + 128) & 255) - 128;
            const int X1 = (X - d0) >> 8;
            const int d1 = ((X1 + 128) & 255) - 128;
            const int d2 = (X1 - d1) >> 8;    // |d2| <= 64
            const int sh = 8 * (k & 3);
            p0[k >> 2] |= (static_cast<uint32_t>(d0) & 255u) << sh;
            p1[k >> 2] |= (static_cast<uint32_t>(d1) & 255u) << sh;
            p2[k >> 2] |= (static_cast<uint32_t>(d2) & 255u) << sh;
        }
        uint8_t *o = tab + xr * tstride + (sb >> 3) * kTabBlk + (sb & 7) * 96 + 8 * q;
        *reinterpret_cast<u32x2 *>(o) = u32x2{p0[0], p0[1]};
        *reinterpret_cast<u32x2 *>(o + 32) = u32x2{p1[0], p1[1]};
        *reinterpret_cast<u32x2 *>(o + 64) = u32x2{p2[0], p2[1]};
        // Q6_K: sum of X over each 16-value half (threads q, q ^ 1)
        xsum += __shfl_xor(xsum, 1, 64);
        const int xsum_hi = __shfl_xor(xsum, 2, 64);
        if (q == 0) {
            // down mode: the slot weight scales the sub-block's activations
            const float ws = DOWN ? wl[sb / static_cast<int>(t.moe_kslot / 32)] : 1.0f;
            ex[xr * nsb + sb] = float2{(live ? dn : 1.0f) * ws, sum * ws};
            if (Q6 || DT == DT_Q4_0) ex16[xr * nsb + sb] = float2{__int_as_float(xsum), __int_as_float(xsum_hi)};
        }
    }
    if (!moe && threadIdx.x < nseg) segl[threadIdx.x] = t.seg[threadIdx.x];
    if (!early) {
        if (moe) {
#pragma unroll
            for (int k = 0; k < NSLOT; k++)
                if (k < first) issue(k, segl);
        } else {
#pragma unroll
            for (int k = 0; k < NSLOT; k++)
                if (k < first) issue(k, t.seg);
        }
    }
    const float inv_acc = t.rexp ? exp2f(-static_cast<float>(t.rexp[0])) : 1.0f;
    __syncthreads();

    // ---- per-lane roles
    const int c16 = lane & 15;      // B column = row within a row group; A row
    const int gq = lane >> 4;       // k group of the lane (bytes 16 gq .. +15 of a 64-byte half)
    const int ap = c16 & 3, as = c16 >> 2;  // A row = 4 * sub-block' + digit plane
    const int sl = 2 * (gq >> 1);           // sub-block' of this lane's low-nibble MFMA
    const bool a_lo = ap < 3 && as == sl, a_hi = ap < 3 && as == sl + 1;
    const int a_off = as * 96 + ap * 32 + 16 * (gq & 1);
    // A addresses advance by one table block per 256 values; empty lanes stay
    // on the zero area (the h = 1 half is reached by an immediate offset)
    const uint8_t *a_lo_p = a_lo ? tab + a_off : zero;
    const uint8_t *a_hi_p = a_hi ? tab + a_off : zero;
    const int a_lo_inc = a_lo ? kTabBlk : 0, a_hi_inc = a_hi ? kTabBlk : 0;
    // Q6_K: MFMA chunk qd of a block takes, in lane group gq = 2h + lh, the
    // 16 values 128h + 32qd + 16lh + i -- one scale sub-block; the A row
    // 4gq + p holds their digit plane p (sub-block 4h + qd of the table)
    const int h6 = gq >> 1, lh6 = gq & 1;
    const bool a6 = ap < 3 && as == gq;
    const uint8_t *a6_p = a6 ? tab + 4 * h6 * 96 + ap * 32 + 16 * lh6 : zero;
    const int a6_inc = a6 ? kTabBlk : 0, a6_qd = a6 ? 96 : 0;
    // QS: MFMA chunk m of 256 values takes blocks 2m, 2m + 1; lane group gq
    // holds 16 codes of block 2m + (gq >> 1), half gq & 1; A row 4s' + p
    // (s' = 0, 1) holds plane p of block 2m + s'; C rows 4gq + j of lanes
    // gq < 2 are block 2m + gq's plane sums
    const bool aq = ap < 3 && as == (gq >> 1);
    const uint8_t *aq_p = aq ? tab + (gq >> 1) * 96 + ap * 32 + 16 * (gq & 1) : zero;
    const int aq_inc = aq ? kTabBlk : 0, aq_m = aq ? 2 * 96 : 0;
    const uint32_t M = 0x0F0F0F0Fu;
    const uint32_t bsh = 8u * static_cast<uint32_t>(gq);

    int j = 0;
    for (int ti = 0; ti < my_tiles; ti++) {
        float acc[NX][RGN];
#pragma unroll
        for (int xr = 0; xr < NX; xr++)
#pragma unroll
            for (int r = 0; r < RGN; r++) acc[xr][r] = 0.0f;
        for (int kk = 0; kk < cnt; kk++, j++) {
            // units j + 1 .. j + NSLOT - 1 may still be in flight
            const int ahead = my_units - 1 - j;
            if (ahead >= NSLOT - 1) wait_vm<(NSLOT - 1) * CH>();
            else if (NSLOT > 2 && ahead == 1) wait_vm<CH>();
            else wait_vm<0>();
            const int ks = rsplit ? kk : wv + kk * nwc;
            const uint8_t *slot = slots + static_cast<int>(j % NSLOT) * SLOT;
            // the unit's bytes -> registers, then its slot takes unit j + NSLOT
            // (Q4_K: header, low and high code halves; Q6_K: both ql halves,
            // qh, this lane's 8 scale bytes and d)
            u32x4 hdr[KB][RGN], qa[KB][RGN], qb[KB][RGN], qc[KB][RGN];
            uint2 sc6[KB][RGN];
            uint32_t d6[KB][RGN];
            u32x4 dq[KB][RGN];   // QS: d of block 2m + (gq & 1), m = 0..3
#pragma unroll
            for (int b = 0; b < KB; b++)
#pragma unroll
                for (int rg = 0; rg < RGN; rg++) {
                    // rows past ROWS (a partial last group) read row ROWS - 1; discarded
                    const int rr = rg * 16 + c16 < ROWS ? rg * 16 + c16 : ROWS - 1;
                    const uint8_t *rp = slot + rr * PL + b * BL;
                    if constexpr (QS) {
                        // codes of block 2m + (gq >> 1): Q8_0 half gq & 1, Q4_0 all 16 bytes
                        const int co = 16 + (Q8 ? 16 * (gq & 1) : 0);
                        const uint8_t *bq = rp + (gq >> 1) * sbl + co, *bd = rp + (gq & 1) * sbl;
                        hdr[b][rg] = *reinterpret_cast<const u32x4 *>(bq);
                        qa[b][rg] = *reinterpret_cast<const u32x4 *>(bq + 2 * sbl);
                        qb[b][rg] = *reinterpret_cast<const u32x4 *>(bq + 4 * sbl);
                        qc[b][rg] = *reinterpret_cast<const u32x4 *>(bq + 6 * sbl);
                        dq[b][rg] = u32x4{*reinterpret_cast<const uint32_t *>(bd),
                                          *reinterpret_cast<const uint32_t *>(bd + 2 * sbl),
                                          *reinterpret_cast<const uint32_t *>(bd + 4 * sbl),
                                          *reinterpret_cast<const uint32_t *>(bd + 6 * sbl)};
                    } else if constexpr (Q6) {
                        hdr[b][rg] = *reinterpret_cast<const u32x4 *>(rp + 64 * h6 + 16 * lh6);        // ql, qd even
                        qa[b][rg] = *reinterpret_cast<const u32x4 *>(rp + 64 * h6 + 32 + 16 * lh6);    // ql, qd odd
                        qb[b][rg] = *reinterpret_cast<const u32x4 *>(rp + 128 + 32 * h6 + 16 * lh6);   // qh
                        sc6[b][rg] = *reinterpret_cast<const uint2 *>(rp + 192 + 8 * h6);
                        d6[b][rg] = *reinterpret_cast<const uint32_t *>(rp + 220);   // d in the high half
                    } else {
                        hdr[b][rg] = *reinterpret_cast<const u32x4 *>(rp);
                        qa[b][rg] = *reinterpret_cast<const u32x4 *>(rp + 16 + 16 * gq);
                        qb[b][rg] = *reinterpret_cast<const u32x4 *>(rp + 80 + 16 * gq);
                    }
                }
            __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0)
            if (j + NSLOT < my_units) issue(j + NSLOT, segl);
#pragma unroll
            for (int b = 0; b < KB; b++) {
                const int blk = ks * KB + b;
                if (KB > 1 && blk >= nb) break;
#pragma unroll
                for (int rg = 0; rg < RGN; rg++) {
                    const v4i z = {0, 0, 0, 0};
                    if constexpr (QS) {
                        // Q8_0: y = d * sum q x (dequant_q8_0, src/quant.cpp:381-387);
                        // Q4_0: y = d * sum (q - 8) x (dequant_q4_0, quant.cpp:331-339),
                        // the offset 8 applied through exact integer digit sums
                        const uint32_t hsh = (gq & 1) ? 4u : 0u;
#pragma unroll
                        for (int m = 0; m < 4; m++) {
                            const u32x4 qv = m == 0 ? hdr[b][rg] : m == 1 ? qa[b][rg] : m == 2 ? qb[b][rg] : qc[b][rg];
                            v4i B;
                            if constexpr (Q8) {
                                B = v4i{static_cast<int>(qv.x), static_cast<int>(qv.y), static_cast<int>(qv.z),
                                        static_cast<int>(qv.w)};
                            } else {
                                B = v4i{static_cast<int>((qv.x >> hsh) & M), static_cast<int>((qv.y >> hsh) & M),
                                        static_cast<int>((qv.z >> hsh) & M), static_cast<int>((qv.w >> hsh) & M)};
                            }
                            const uint32_t dw = m == 0 ? dq[b][rg].x : m == 1 ? dq[b][rg].y : m == 2 ? dq[b][rg].z
                                                                                                 : dq[b][rg].w;
                            const float d = h2f(dw & 0xFFFFu);
#pragma unroll
                            for (int xr = 0; xr < NX; xr++) {
                                const uint8_t *apq = aq_p + (aq ? xr * tstride : 0) + blk * aq_inc + m * aq_m;
                                const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(ld_v4i(apq), B, z, 0, 0, 0);
                                // lanes gq >= 2 hold empty C rows; they add nothing
                                const int sbi = xr * nsb + blk * 8 + 2 * m + (gq & 1);
                                float sv;
                                if constexpr (Q8) {
                                    // |sum q X| < 2^34: combine the exact plane sums in f32
                                    sv = __builtin_fmaf(65536.0f, static_cast<float>(C[2]),
                                                        __builtin_fmaf(256.0f, static_cast<float>(C[1]),
                                                                       static_cast<float>(C[0])));
                                } else {
                                    // sum (q - 8) X over 32 values: |S| <= 2^30, exact in int32
                                    const float2 h2 = ex16[sbi];
                                    const uint32_t xs = static_cast<uint32_t>(__float_as_int(h2.x)) +
                                                        static_cast<uint32_t>(__float_as_int(h2.y));
                                    const int S = static_cast<int>(static_cast<uint32_t>(C[0]) +
                                                                   (static_cast<uint32_t>(C[1]) << 8) +
                                                                   (static_cast<uint32_t>(C[2]) << 16) - 8u * xs);
                                    sv = static_cast<float>(S);
                                }
                                if (gq < 2) acc[xr][rg] = __builtin_fmaf(d, ex[sbi].x * sv, acc[xr][rg]);
                            }
                        }
                    } else if constexpr (Q6) {
                        // q = low 4 bits from ql | 2 high bits from qh (dequant_q6_K,
                        // src/quant.cpp:462-512), codes 0..63 as int8; the code
                        // offset 32 is applied through the 16-value sums of x
                        const u32x4 l0 = hdr[b][rg], l1 = qa[b][rg], qh = qb[b][rg];
                        const float d = h2f(d6[b][rg] >> 16);
#pragma unroll
                        for (int qd = 0; qd < 4; qd++) {
                            const u32x4 ql = (qd & 1) ? l1 : l0;
                            const uint32_t ns = (qd >> 1) * 4u, hs = 2u * qd;
                            const v4i B = {static_cast<int>(((ql.x >> ns) & M) | (((qh.x >> hs) & 0x03030303u) << 4)),
                                           static_cast<int>(((ql.y >> ns) & M) | (((qh.y >> hs) & 0x03030303u) << 4)),
                                           static_cast<int>(((ql.z >> ns) & M) | (((qh.z >> hs) & 0x03030303u) << 4)),
                                           static_cast<int>(((ql.w >> ns) & M) | (((qh.w >> hs) & 0x03030303u) << 4))};
                            // scale of sub-block 16 (8h + 2qd + lh): byte 2qd + lh of this lane's 8
                            const int jj = 2 * qd + lh6;
                            const uint32_t sw = jj < 4 ? sc6[b][rg].x : sc6[b][rg].y;
                            const float ds = d * static_cast<float>(static_cast<int8_t>(sw >> (8 * (jj & 3))));
#pragma unroll
                            for (int xr = 0; xr < NX; xr++) {
                                const uint8_t *ap6 = a6_p + (a6 ? xr * tstride : 0) + blk * a6_inc + qd * a6_qd;
                                const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(ld_v4i(ap6), B, z, 0, 0, 0);
                                const int sbi = xr * nsb + blk * 8 + 4 * h6 + qd;
                                const float2 e2 = ex[sbi], h2 = ex16[sbi];
                                // S = sum (q - 32) X over the 16 values: |S| <= 16 * 32 * 2^22
                                // fits int32, so wrapping unsigned arithmetic gives it exactly
                                const uint32_t xs = static_cast<uint32_t>(__float_as_int(lh6 ? h2.y : h2.x));
                                const int S = static_cast<int>(static_cast<uint32_t>(C[0]) +
                                                               (static_cast<uint32_t>(C[1]) << 8) +
                                                               (static_cast<uint32_t>(C[2]) << 16) - 32u * xs);
                                acc[xr][rg] = __builtin_fmaf(ds, e2.x * static_cast<float>(S), acc[xr][rg]);
                            }
                        }
                    } else {
                        const u32x4 hd = hdr[b][rg], q0 = qa[b][rg], q1 = qb[b][rg];
                        const v4i B0l = {static_cast<int>(q0.x & M), static_cast<int>(q0.y & M),
                                         static_cast<int>(q0.z & M), static_cast<int>(q0.w & M)};
                        const v4i B0h = {static_cast<int>((q0.x >> 4) & M), static_cast<int>((q0.y >> 4) & M),
                                         static_cast<int>((q0.z >> 4) & M), static_cast<int>((q0.w >> 4) & M)};
                        const v4i B1l = {static_cast<int>(q1.x & M), static_cast<int>(q1.y & M),
                                         static_cast<int>(q1.z & M), static_cast<int>(q1.w & M)};
                        const v4i B1h = {static_cast<int>((q1.x >> 4) & M), static_cast<int>((q1.y >> 4) & M),
                                         static_cast<int>((q1.z >> 4) & M), static_cast<int>((q1.w >> 4) & M)};
                        // scales of sub-blocks gq and 4 + gq (get_scale_min_k4,
                        // src/quant.cpp:427-435): bytes gq of scales[0..3], [4..7], [8..11]
                        const uint32_t s1 = hd.y >> bsh, s2 = hd.z >> bsh, s3 = hd.w >> bsh;
                        const float d = h2f(hd.x & 0xFFFFu), dmin = h2f(hd.x >> 16);
                        const float sc0 = static_cast<float>(s1 & 63u), m0 = static_cast<float>(s2 & 63u);
                        const float sc1 = static_cast<float>((s3 & 15u) | ((s1 >> 2) & 0x30u));
                        const float m1 = static_cast<float>(((s3 >> 4) & 15u) | ((s2 >> 2) & 0x30u));
                        const float ds0 = d * sc0, ds1 = d * sc1, dm0 = -dmin * m0, dm1 = -dmin * m1;
#pragma unroll
                        for (int xr = 0; xr < NX; xr++) {
                            // this activation row's digit table
                            const uint8_t *alp = a_lo_p + (a_lo ? xr * tstride : 0) + blk * a_lo_inc;
                            const uint8_t *ahp = a_hi_p + (a_hi ? xr * tstride : 0) + blk * a_hi_inc;
                            const v4i A0l = ld_v4i(alp), A1l = ld_v4i(alp + 384);
                            const v4i A0h = ld_v4i(ahp), A1h = ld_v4i(ahp + 384);
                            // this lane's sub-blocks gq (h = 0) and 4 + gq (h = 1) of block blk
                            const float2 ex0 = ex[xr * nsb + blk * 8 + gq], ex1 = ex[xr * nsb + blk * 8 + 4 + gq];
                            v4i C0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0l, B0l, z, 0, 0, 0);
                            C0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0h, B0h, C0, 0, 0, 0);
                            v4i C1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1l, B1l, z, 0, 0, 0);
                            C1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1h, B1h, C1, 0, 0, 0);
                            const int S0 = C0[0] + (C0[1] << 8) + (C0[2] << 16);
                            const int S1 = C1[0] + (C1[1] << 8) + (C1[2] << 16);
                            float a = acc[xr][rg];
                            a = __builtin_fmaf(ds0, ex0.x * static_cast<float>(S0), a);
                            a = __builtin_fmaf(dm0, ex0.y, a);
                            a = __builtin_fmaf(ds1, ex1.x * static_cast<float>(S1), a);
                            a = __builtin_fmaf(dm1, ex1.y, a);
                            acc[xr][rg] = a;
                        }
                    }
                }
            }
        }
        // one output row: a gate/up pair (gs, us) or a plain dot (gs)
        auto emit = [&](int si, int xr, int64_t n, float gs, float us) {
            const int kind = segl[si].kind;
            OT *o = static_cast<OT *>(segl[si].out) + static_cast<int64_t>(xr) * t.out_stride + n;
            if (kind == SEG_SILU) {
                if constexpr (sizeof(OT) == 2) {
                    // fused_gate_silu_kernel (fused.hpp:161-166): both dots
                    // rounded to f16, activation in f32, saturated
                    const float hg = static_cast<float>(static_cast<_Float16>(gs));
                    const float hu = static_cast<float>(static_cast<_Float16>(us));
                    *o = sat_f16(silu_f(hg) * hu);
                } else {
                    *o = (gs / (1.0f + expf(-gs))) * us;   // silu_mul, backend_cpu.cpp:2401-2406
                }
            } else {
                store_out<OT>(o, gs, kind, kind == SEG_ACC ? inv_acc : 1.0f);
            }
        };
        const int64_t g = wid + static_cast<int64_t>(ti) * wstride;
        if constexpr (RSPLIT) {
            // the wave's own rows: sum over the four k groups, lanes of group
            // 0 hold rows rg * 16 + c16 (gate/up pairs: rg 0 gate, rg 1 up)
            float v[NX][RGN];
#pragma unroll
            for (int xr = 0; xr < NX; xr++)
#pragma unroll
                for (int rg = 0; rg < RGN; rg++) {
                    v[xr][rg] = acc[xr][rg];
                    v[xr][rg] += __shfl_xor(v[xr][rg], 16, 64);
                    v[xr][rg] += __shfl_xor(v[xr][rg], 32, 64);
                }
            if (gq == 0) {
                const int si = seg_w(g, segl);
                const bool pair = segl[si].kind == SEG_SILU;
#pragma unroll
                for (int xr = 0; xr < NX; xr++) {
                    if (xr >= nrows) break;
                    if (pair) {
                        const int64_t n = (g - segl[si].blk_begin) * 16 + c16;
                        if (n < segl[si].n_out) emit(si, xr, n, v[xr][0], RGN > 1 ? v[xr][RGN - 1] : 0.0f);
                    } else {
#pragma unroll
                        for (int rg = 0; rg < RGN; rg++) {
                            const int tr = rg * 16 + c16;
                            const int64_t n = (g - segl[si].blk_begin) * ROWS + tr;
                            if (tr < ROWS && n < segl[si].n_out) emit(si, xr, n, v[xr][rg], 0.0f);
                        }
                    }
                }
            }
            continue;
        }
        // K split: partial sums of the waves -> LDS as [x row][row][wave],
        // then one thread per (x row, row) reads its eight partials at once
        // (two b128 reads) and adds them in wave order
        float *rbuf = red + (ti & 1) * NX * RS * kRedWaves;
#pragma unroll
        for (int xr = 0; xr < NX; xr++)
#pragma unroll
            for (int rg = 0; rg < RGN; rg++) {
                float v = acc[xr][rg];
                v += __shfl_xor(v, 16, 64);
                v += __shfl_xor(v, 32, 64);
                if (gq == 0) rbuf[((xr * RS) + rg * 16 + c16) * kRedWaves + wv] = v;
            }
        __syncthreads();
        auto row_sum = [&](int r) {
            const floatx4 a = *reinterpret_cast<const floatx4 *>(rbuf + r * kRedWaves);
            const floatx4 b = *reinterpret_cast<const floatx4 *>(rbuf + r * kRedWaves + 4);
            const float p[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            float v = 0.0f;
#pragma unroll
            for (int k = 0; k < kRedWaves; k++)
                if (k < nwc) v += p[k];
            return v;
        };
        if (threadIdx.x < NX * ROWS) {
            const int xr = NX > 1 ? static_cast<int>(threadIdx.x) / ROWS : 0;
            const int tr = static_cast<int>(threadIdx.x) - xr * ROWS;   // row within the tile
            const int si = seg_w(g, segl);
            if (xr < nrows && segl[si].kind == SEG_SILU) {
                // rows t and 16 + t of the tile are gate and up of output n0 + t
                const int64_t n = (g - segl[si].blk_begin) * 16 + tr;
                if (tr < 16 && n < segl[si].n_out)
                    emit(si, xr, n, row_sum(xr * RS + tr), row_sum(xr * RS + 16 + tr));
            } else if (xr < nrows) {
                const int64_t n = (g - segl[si].blk_begin) * ROWS + tr;
                if (n < segl[si].n_out) emit(si, xr, n, row_sum(xr * RS + tr), 0.0f);
            }
        }
    }
}

constexpr size_t kLdsBudget = 160u * 1024u - sizeof(Seg) * kMaxSegs;   // dynamic LDS per workgroup

// LDS shared by the waves of a workgroup: NX digit tables with their scale
// pairs, the zero area and the double-buffered reduction
size_t fixed_lds(int nb, int rs, int nx, bool q6) {
    return static_cast<size_t>(nx) * nb * (kTabBlk + (q6 ? 2 : 1) * 8 * sizeof(float2)) + kZero +
           2 * static_cast<size_t>(nx) * rs * kRedWaves * sizeof(float);
}
// LDS bytes of one 256-value row piece of a unit (see the kernel's layout)
constexpr int lds_per_256(int dt) {
    return dt == DT_Q6_K ? 224 : dt == DT_Q8_0 ? 384 : dt == DT_Q4_0 ? 256 : 144;
}
constexpr size_t slot_bytes(int rows, int dt = DT_Q4_K) {
    return ((rows * 2 * lds_per_256(dt) + 1023) / 1024) * 1024;
}

template <int DT, typename XT, typename OT, int ROWS, int KB, int NSLOT, bool DOWN, int NX, bool MT,
          bool RSPLIT = false>
hipError_t launch(SegTable t, hipStream_t st) {
    constexpr bool Q6 = DT == DT_Q6_K;
    constexpr int RS = 16 * ((ROWS + 15) / 16);
    constexpr int SLOT = ((ROWS * KB * lds_per_256(DT) + 1023) / 1024) * 1024;
    int64_t total = 0;
    for (int i = 0; i < t.n; i++) {
        t.seg[i].blk_begin = total;
        const int64_t tr = t.seg[i].kind == SEG_SILU ? 16 : ROWS;   // gate/up: 16 + 16 rows
        total += (t.seg[i].n_out + tr - 1) / tr;
    }
    const int nb = t.n_in / 256;
    const int nks = (nb + KB - 1) / KB;
    if (total * nks >= (int64_t{1} << 31)) return hipErrorNotSupported;   // 32-bit unit indices
    const size_t fixed = fixed_lds(nb, RS, NX, Q6 || DT == DT_Q4_0);
    const size_t per_wave = static_cast<size_t>(NSLOT) * SLOT;
    // kXPasses sub-blocks per thread (4 threads each) must cover NX * nb * 8
    const int min_nw = (NX * nb * 8 * 4 + 64 * kXPasses - 1) / (64 * kXPasses);
    struct Pick { int nb, nw, per_cu; };
    static thread_local Pick cache[16] = {};
    int nw = 0, per_cu = 0;
    for (const Pick &c : cache)
        if (c.nw && c.nb == nb) { nw = c.nw; per_cu = c.per_cu; break; }
    if (!nw) {
        int best = 0;
        for (int cand = min_nw; cand <= 8; cand++) {
            const size_t l = fixed + cand * per_wave;
            if (l > kLdsBudget) break;
            int blocks = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                    &blocks, gemv_digits_kernel<DT, XT, OT, ROWS, KB, NSLOT, DOWN, NX, MT, RSPLIT>, 64 * cand, l) !=
                hipSuccess)
                blocks = 0;
            // waves doing useful work per CU: with K split over the waves a
            // tile lasts ceil(nks / waves) units (seven waves over eight
            // units run at 8/14); with the row split every wave owns tiles
            const int score = RSPLIT ? 64 * blocks * cand : 64 * blocks * nks / ((nks + cand - 1) / cand);
            if (blocks > 0 && score >= best) { best = score; nw = cand; per_cu = blocks; }
        }
        if (!nw) return hipErrorNotSupported;
        for (Pick &c : cache)
            if (!c.nw) { c = Pick{nb, nw, per_cu}; break; }
    }
    static thread_local int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cus = 256;
    }
    int64_t grid = static_cast<int64_t>(cus) * per_cu;
    // row split when every wave of a full grid gets at least two tiles
    if constexpr (!RSPLIT && NX == 1 && !DOWN && !MT) {
        if (total >= 2 * grid * nw) return launch<DT, XT, OT, ROWS, KB, NSLOT, DOWN, NX, MT, true>(t, st);
    }
    if (MT) {
        // a group of workgroups per token, the groups filling the chip together
        int64_t wpt = grid / t.moe_tokens;
        if (wpt > total) wpt = total;
        if (wpt < 1) wpt = 1;
        t.moe_wpt = static_cast<int>(wpt);
        grid = wpt * t.moe_tokens;
    } else if (grid > total) {
        grid = total;
    }
    hipLaunchKernelGGL((gemv_digits_kernel<DT, XT, OT, ROWS, KB, NSLOT, DOWN, NX, MT, RSPLIT>),
                       dim3(static_cast<unsigned>(grid)), dim3(64 * nw), fixed + nw * per_wave, st, t, total,
                       nks, nw);
    return hipGetLastError();
}

template <typename XT, typename OT, bool DOWN, int NX, bool MT = false>
hipError_t launch_rows(int rows, const SegTable &t, hipStream_t st) {
    constexpr int DT = DT_Q4_K;
    if constexpr (NX == 1) {
        switch (rows) {
            case 32: return launch<DT, XT, OT, 32, 2, 2, DOWN, NX, MT>(t, st);
            case 28: return launch<DT, XT, OT, 28, 2, 2, DOWN, NX, MT>(t, st);
            case 24: return launch<DT, XT, OT, 24, 2, 2, DOWN, NX, MT>(t, st);
            case 20: return launch<DT, XT, OT, 20, 2, 2, DOWN, NX, MT>(t, st);
            default: return launch<DT, XT, OT, 16, 2, 2, DOWN, NX, MT>(t, st);
        }
    } else {
        switch (rows) {
            case 32: return launch<DT, XT, OT, 32, 2, 2, DOWN, NX, MT>(t, st);
            case 24: return launch<DT, XT, OT, 24, 2, 2, DOWN, NX, MT>(t, st);
            default: return launch<DT, XT, OT, 16, 2, 2, DOWN, NX, MT>(t, st);
        }
    }
}

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

// Tile height: gate/up pairs take 32 rows (16 + 16).  Otherwise, among the
// heights whose slots leave room for 8 waves next to the NX digit tables
// (16 if none does), the one that minimises rounds x height: the time of the
// workgroup with the most tiles when one workgroup runs per CU (e.g. 14336
// rows at NX = 1: 28-row tiles, 512 = 2 per CU, instead of 448 32-row tiles
// of which 192 CUs run two and 64 run one).
int pick_rows(const SegTable &t, int nx) {
    for (int i = 0; i < t.n; i++)
        if (t.seg[i].kind == SEG_SILU) return 32;
    const int nb = t.n_in / 256;
    const int cus = device_cus();
    int best = 16;
    int64_t best_cost = INT64_MAX;
    for (int r = 32; r >= 16; r -= (nx == 1 ? 4 : 8)) {
        if (fixed_lds(nb, 16 * ((r + 15) / 16), nx, false) + 8 * 2 * slot_bytes(r) > kLdsBudget) continue;
        int64_t tiles = 0;
        for (int i = 0; i < t.n; i++) tiles += (t.seg[i].n_out + r - 1) / r;
        if (t.moe_tokens > 1) tiles *= t.moe_tokens;
        const int64_t cost = (tiles + cus - 1) / cus * r;
        if (cost < best_cost) { best_cost = cost; best = r; }
    }
    return best;
}

// Activation rows per pass: the largest of 4, 2, 1 whose sub-blocks the x
// staging covers (kXPasses sub-blocks per 4 threads, at most 8 waves) with
// LDS left for the waves that staging needs (at least four) at 16-row slots
int nx_cap(int n_in, int dt) {
    const int nb = n_in / 256;
    for (int nx = 4; nx > 1; nx >>= 1) {
        const int min_nw = (nx * nb * 8 * 4 + 64 * kXPasses - 1) / (64 * kXPasses);
        const int nw = min_nw < 4 ? 4 : min_nw;
        if (nw <= 8 &&
            fixed_lds(nb, 16, nx, dt == DT_Q6_K || dt == DT_Q4_0) + nw * 2 * slot_bytes(16, dt) <= kLdsBudget)
            return nx;
    }
    return 1;
}

template <typename XT, typename OT, int NX>
hipError_t dispatch_nx(int dt, const SegTable &t, hipStream_t st) {
    // Q6_K, Q8_0, Q4_0: 16-row tiles (Q8_0's 384-byte LDS pieces one per
    // unit, the others two), plain segments
    if (dt == DT_Q6_K) return launch<DT_Q6_K, XT, OT, 16, 2, 2, false, NX, false>(t, st);
    if (dt == DT_Q8_0) return launch<DT_Q8_0, XT, OT, 16, 1, 2, false, NX, false>(t, st);
    if (dt == DT_Q4_0) return launch<DT_Q4_0, XT, OT, 16, 2, 2, false, NX, false>(t, st);
    const int rows = pick_rows(t, NX);
    if constexpr (sizeof(XT) == 4 && NX == 1) {
        if (t.moe_tab && t.moe_down)
            return t.moe_tokens > 1 ? launch_rows<XT, OT, true, 1, true>(rows, t, st)
                                    : launch_rows<XT, OT, true, 1, false>(rows, t, st);
        if (t.moe_tab && t.moe_tokens > 1)   // gate/up pairs: 32-row tiles
            return launch<DT_Q4_K, XT, OT, 32, 2, 2, false, 1, true>(t, st);
    } else {
        // down mode and several tokens: f32 activations, one row
        if (t.moe_tab && (t.moe_down || t.moe_tokens > 1)) return hipErrorNotSupported;
    }
    return launch_rows<XT, OT, false, NX>(rows, t, st);
}

// rows 2..8: passes of up to nx_cap activation rows, each reading W once
template <typename XT, typename OT>
hipError_t dispatch(int dt, const SegTable &t, hipStream_t st) {
    if (t.rows == 1) return dispatch_nx<XT, OT, 1>(dt, t, st);
    const int cap = nx_cap(t.n_in, dt);
    for (int64_t r0 = 0; r0 < t.rows; r0 += cap) {
        SegTable p = t;
        const int64_t c = t.rows - r0 < cap ? t.rows - r0 : cap;
        p.rows = c;
        for (int i = 0; i < p.n; i++) {
            p.seg[i].x = static_cast<const XT *>(t.seg[i].x) + r0 * t.x_stride;
            p.seg[i].out = static_cast<OT *>(t.seg[i].out) + r0 * t.out_stride;
        }
        const hipError_t e = c == 1 ? dispatch_nx<XT, OT, 1>(dt, p, st)
                           : c == 2 ? dispatch_nx<XT, OT, 2>(dt, p, st)
                                    : dispatch_nx<XT, OT, 4>(dt, p, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

bool gemv_digits_ok(int dt, const SegTable &t) {
    if (t.rows < 1 || t.rows > 8 || t.n_in > kMaxK) return false;
    if (dt == DT_Q6_K || dt == DT_Q8_0 || dt == DT_Q4_0) {
        // whole units (Q8_0: 256 values, the others 512), plain segments only.
        // Q8_0 and Q4_0 at one row stay on the VALU stream kernel, which
        // measured faster there (their decode is cheap); from two rows on the
        // digit planes share each weight unit and win
        if ((dt != DT_Q6_K && t.rows < 2) || t.n_in % (dt == DT_Q8_0 ? 256 : 512) || t.row_bytes % 4 ||
            t.moe_tab)
            return false;
        for (int i = 0; i < t.n; i++)
            if (t.seg[i].x != t.seg[0].x || t.seg[i].kind == SEG_SILU ||
                (reinterpret_cast<uintptr_t>(t.seg[i].w) & 3))
                return false;
        return true;
    }
    if (dt != DT_Q4_K || t.n_in % 256 || t.row_bytes % 16) return false;
    if (t.em_runs) return false;   // expert-major runs are the streaming kernel's
    if (t.moe_tab && t.rows != 1) return false;
    if (t.moe_tab && t.moe_down &&
        (t.n != 1 || t.moe_k < 1 || t.moe_k > kMaxDownSlots || t.moe_kslot % 512 ||
         t.n_in != t.moe_k * t.moe_kslot || t.seg[0].kind != SEG_PLAIN))
        return false;   // down mode: whole units (2 blocks) per slot
    for (int i = 0; i < t.n; i++) {
        if (t.seg[i].x != t.seg[0].x) return false;
        if (t.seg[i].kind == SEG_SILU && (t.n_in > 8192 || (reinterpret_cast<uintptr_t>(t.seg[i].w2) & 15)))
            return false;   // gate/up pairs use the 32-row tiles
        if (reinterpret_cast<uintptr_t>(t.seg[i].w) & 15) return false;
    }
    return true;
}

hipError_t gemv_digits(int dt, bool act_f16, const SegTable &t, hipStream_t st) {
    return act_f16 ? dispatch<_Float16, _Float16>(dt, t, st) : dispatch<float, float>(dt, t, st);
}

}  // namespace krk
