// synth.cpp -- seeded synthetic inputs for the benchmark configurations, and
// the host-side weight quantizers that turn f32 matrices into GGUF blocks.
//
// Q8_0 and Q4_0 follow the reference's own fixture generator
// (tools/make_bench_gguf.py:191-218: f64 arithmetic, Python round() = half to
// even, struct.pack('<e') = one RNE rounding to f16).  The reference ships no
// Q4_K or Q6_K quantizer (its K-quant fixtures are random bytes,
// tools/bench_ops.cpp:96-140), so those two are this library's own min/scale
// fits; they only generate inputs, and every parity check runs on the bytes
// they produce.
#include "krk_mi355x.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

// The c-th output of a splitmix64 stream started at `seed`.
inline uint64_t splitmix_at(uint64_t seed, uint64_t c) {
    uint64_t z = seed + (c + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline double normal_at(uint64_t seed, int64_t i) {
    const uint64_t p = static_cast<uint64_t>(i) >> 1;
    const double u1 = static_cast<double>((splitmix_at(seed, 2 * p) >> 11) + 1) *
                      0x1.0p-53;  // (0, 1]
    const double u2 = static_cast<double>(splitmix_at(seed, 2 * p + 1) >> 11) *
                      0x1.0p-53;  // [0, 1)
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double th = 6.283185307179586476925286766559 * u2;
    return (i & 1) ? r * std::sin(th) : r * std::cos(th);
}

template <class F>
void par_rows(int64_t n, int nthreads, F &&fn) {
    if (nthreads <= 1 || n < 2) { fn(int64_t{0}, n); return; }
    nthreads = static_cast<int>(std::min<int64_t>(std::min(nthreads, 256), n));
    std::vector<std::thread> th;
    const int64_t per = (n + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        const int64_t b = per * t, e = std::min(n, b + per);
        if (b >= e) break;
        th.emplace_back([&fn, b, e] { fn(b, e); });
    }
    for (auto &t : th) t.join();
}

// f64 -> IEEE half, one rounding, ties to even (what struct.pack('<e') does).
uint16_t f64_to_half(double v) {
    const uint16_t sign = std::signbit(v) ? 0x8000u : 0u;
    if (std::isnan(v)) return 0x7E00u;
    const double a = std::fabs(v);
    if (a >= 65520.0) return static_cast<uint16_t>(sign | 0x7C00u);
    int e = 0;
    std::frexp(a, &e);
    int ue = std::max(e - 1, -14);
    double q = std::nearbyint(std::ldexp(a, 10 - ue));
    if (q >= 2048.0) { q *= 0.5; ue++; }
    const uint32_t qi = static_cast<uint32_t>(q);
    if (qi < 1024u) return static_cast<uint16_t>(sign | qi);
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(ue + 15) << 10) |
                                 (qi - 1024u));
}

double half_to_f64(uint16_t h) {
    const int e = (h >> 10) & 31, m = h & 1023;
    double v;
    if (e == 0) v = std::ldexp(static_cast<double>(m), -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = std::ldexp(static_cast<double>(m + 1024), e - 25);
    return (h & 0x8000u) ? -v : v;
}

inline void put16(uint8_t *p, uint16_t h) {
    p[0] = static_cast<uint8_t>(h & 0xFF);
    p[1] = static_cast<uint8_t>(h >> 8);
}

inline int clampi(double v, int lo, int hi) {
    return static_cast<int>(std::min<double>(hi, std::max<double>(lo, v)));
}

// make_bench_gguf.py:191-202
void quant_q8_0(const float *v, int64_t n, uint8_t *dst) {
    for (int64_t b = 0; b < n; b += 32, dst += 34) {
        double amax = 0.0;
        for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(double(v[b + i])));
        if (amax == 0.0) amax = 1e-8;
        const double d = amax / 127.0;
        put16(dst, f64_to_half(d));
        for (int i = 0; i < 32; i++)
            dst[2 + i] = static_cast<uint8_t>(static_cast<int8_t>(
                clampi(std::nearbyint(double(v[b + i]) / d), -127, 127)));
    }
}

// make_bench_gguf.py:205-218: d = (signed extreme) / -8 where the extreme is
// max(-min, max) -- a magnitude, so d <= 0 -- and q = round(v / d + 8).
void quant_q4_0(const float *v, int64_t n, uint8_t *dst) {
    for (int64_t b = 0; b < n; b += 32, dst += 18) {
        double mn = v[b], mx = v[b];
        for (int i = 1; i < 32; i++) {
            mn = std::min(mn, double(v[b + i]));
            mx = std::max(mx, double(v[b + i]));
        }
        const double amax = std::max(-mn, mx);
        const double d = amax != 0.0 ? amax / -8.0 : 0.0;
        const double id = d != 0.0 ? 1.0 / d : 0.0;
        put16(dst, f64_to_half(d));
        int q[32];
        for (int i = 0; i < 32; i++)
            q[i] = clampi(std::nearbyint(double(v[b + i]) * id + 8.0), 0, 15);
        for (int k = 0; k < 16; k++)
            dst[2 + k] = static_cast<uint8_t>((q[k] & 15) | ((q[k + 16] & 15) << 4));
    }
}

// Q4_K (144 B / 256 values): per 32-value sub-block an affine fit
// v ~ sc*d * q - m*dmin with q in [0,15]; the eight 6-bit (sc, m) pairs are
// packed the way get_scale_min_k4 (quant.cpp:427-435) unpacks them.
void quant_q4_k(const float *v, int64_t n, uint8_t *dst) {
    for (int64_t b = 0; b < n; b += 256, dst += 144) {
        double scale[8], minv[8];
        double smax = 0.0, mmax = 0.0;
        for (int j = 0; j < 8; j++) {
            double lo = 0.0, hi = 0.0;
            for (int l = 0; l < 32; l++) {
                lo = std::min(lo, double(v[b + 32 * j + l]));
                hi = std::max(hi, double(v[b + 32 * j + l]));
            }
            scale[j] = (hi - lo) / 15.0;
            minv[j] = -lo;  // >= 0
            smax = std::max(smax, scale[j]);
            mmax = std::max(mmax, minv[j]);
        }
        const uint16_t hd = f64_to_half(smax / 63.0), hm = f64_to_half(mmax / 63.0);
        const double d = half_to_f64(hd), dmin = half_to_f64(hm);
        int sc[8], mq[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = d > 0 ? clampi(std::nearbyint(scale[j] / d), 0, 63) : 0;
            mq[j] = dmin > 0 ? clampi(std::nearbyint(minv[j] / dmin), 0, 63) : 0;
        }
        put16(dst, hd);
        put16(dst + 2, hm);
        uint8_t *s = dst + 4;
        for (int j = 0; j < 4; j++) {
            s[j] = static_cast<uint8_t>((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            s[j + 4] = static_cast<uint8_t>((mq[j] & 63) | ((mq[j + 4] >> 4) << 6));
            s[j + 8] = static_cast<uint8_t>((sc[j + 4] & 15) | ((mq[j + 4] & 15) << 4));
        }
        int q[256];
        for (int j = 0; j < 8; j++) {
            const double ds = d * sc[j], dm = dmin * mq[j];
            for (int l = 0; l < 32; l++) {
                const double x = double(v[b + 32 * j + l]);
                q[32 * j + l] = ds > 0 ? clampi(std::nearbyint((x + dm) / ds), 0, 15) : 0;
            }
        }
        uint8_t *qs = dst + 16;
        for (int g = 0; g < 4; g++)
            for (int l = 0; l < 32; l++)
                qs[32 * g + l] = static_cast<uint8_t>(q[64 * g + l] | (q[64 * g + 32 + l] << 4));
    }
}

// IQ4_NL (18 B / 32 values): d = amax / 127 rounded to f16 (the grid spans
// -127..113), each value to the nearest grid point of v / d.
void quant_iq4_nl(const float *v, int64_t n, uint8_t *dst) {
    static const int grid[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
    for (int64_t b = 0; b < n; b += 32, dst += 18) {
        double amax = 0.0;
        for (int l = 0; l < 32; l++) amax = std::max(amax, std::fabs(double(v[b + l])));
        const uint16_t hd = f64_to_half(amax / 127.0);
        const double d = half_to_f64(hd);
        int q[32];
        for (int l = 0; l < 32; l++) {
            const double t = d > 0 ? double(v[b + l]) / d : 0.0;
            int best = 0;
            for (int k = 1; k < 16; k++)
                if (std::fabs(t - grid[k]) < std::fabs(t - grid[best])) best = k;
            q[l] = best;
        }
        put16(dst, hd);
        for (int l = 0; l < 16; l++) dst[2 + l] = static_cast<uint8_t>(q[l] | (q[l + 16] << 4));
    }
}

// Q4_1 / Q5_1 (20 / 24 B per 32 values): d = (max - min) / (2^bits - 1),
// m = min, codes round((v - m) / d); Q5_0 (22 B): ggml's signed-max rule as
// for Q4_0 (d = max / -16, codes round(v / d + 16) in 0..31).
template <int BITS, bool MIN>
void quant_l32(const float *v, int64_t n, uint8_t *dst) {
    const int bb = MIN ? (BITS == 4 ? 20 : 24) : 22, qs = MIN ? (BITS == 4 ? 4 : 8) : 6;
    const int qmax = (1 << BITS) - 1;
    for (int64_t b = 0; b < n; b += 32, dst += bb) {
        double lo = v[b], hi = v[b], amax = 0.0, smax = 0.0;
        for (int l = 0; l < 32; l++) {
            const double t = v[b + l];
            lo = std::min(lo, t);
            hi = std::max(hi, t);
            if (std::fabs(t) > amax) { amax = std::fabs(t); smax = t; }
        }
        uint16_t hd, hm = 0;
        if (MIN) {
            hd = f64_to_half((hi - lo) / qmax);
            hm = f64_to_half(lo);
        } else {
            hd = f64_to_half(smax / -16.0);
        }
        const double d = half_to_f64(hd), m = half_to_f64(hm);
        put16(dst, hd);
        if (MIN) put16(dst + 2, hm);
        uint32_t qh = 0;
        int q[32];
        for (int l = 0; l < 32; l++) {
            const double t = MIN ? (d > 0 ? (double(v[b + l]) - m) / d : 0.0)
                                 : (d != 0 ? double(v[b + l]) / d + 16.0 : 16.0);
            q[l] = clampi(std::nearbyint(t), 0, qmax);
            if (BITS == 5) qh |= static_cast<uint32_t>((q[l] >> 4) & 1) << l;
        }
        for (int l = 0; l < 16; l++) dst[qs + l] = static_cast<uint8_t>((q[l] & 15) | ((q[l + 16] & 15) << 4));
        if (BITS == 5) {
            uint8_t *h = dst + (MIN ? 4 : 2);
            for (int k = 0; k < 4; k++) h[k] = static_cast<uint8_t>(qh >> (8 * k));
        }
    }
}

// F16 / BF16 weights: each value rounded to nearest even
void quant_f16(const float *v, int64_t n, uint8_t *dst) {
    for (int64_t i = 0; i < n; i++) put16(dst + 2 * i, f64_to_half(double(v[i])));
}
void quant_bf16(const float *v, int64_t n, uint8_t *dst) {
    for (int64_t i = 0; i < n; i++) {
        uint32_t b;
        std::memcpy(&b, &v[i], 4);
        b += 0x7FFFu + ((b >> 16) & 1u);   // finite inputs only
        put16(dst + 2 * i, static_cast<uint16_t>(b >> 16));
    }
}

// MXFP4 (17 B / 32 values): the exponent e with 12 * 2^(e - 128) >= amax
// (the doubled grid's largest magnitude), then each value's nearest grid
// point of v / 2^(e - 128).
void quant_mxfp4(const float *v, int64_t n, uint8_t *dst) {
    static const int grid[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    for (int64_t b = 0; b < n; b += 32, dst += 17) {
        double amax = 0.0;
        for (int l = 0; l < 32; l++) amax = std::max(amax, std::fabs(double(v[b + l])));
        int e = 0;
        if (amax > 0) e = clampi(128 + std::ceil(std::log2(amax / 12.0)), 0, 254);
        dst[0] = static_cast<uint8_t>(e);
        const double d = std::ldexp(1.0, e - 128);
        int q[32];
        for (int l = 0; l < 32; l++) {
            const double t = double(v[b + l]) / d;
            int best = 0;
            for (int k = 1; k < 16; k++)
                if (std::fabs(t - grid[k]) < std::fabs(t - grid[best])) best = k;
            q[l] = best;
        }
        for (int l = 0; l < 16; l++) dst[1 + l] = static_cast<uint8_t>(q[l] | (q[l + 16] << 4));
    }
}

// Q2_K (84 B / 256 values): per 16-value group a 4-bit scale of
// (max - min) / 3 and a 4-bit min of -min (min clamped to <= 0) on grids of
// d = max scale / 15 and dmin = max min / 15; codes round((v + m) / s) in 0..3.
void quant_q2_k(const float *v, int64_t n, uint8_t *dst) {
    for (int64_t b = 0; b < n; b += 256, dst += 84) {
        double sc[16], mn[16], smax = 0.0, mmax = 0.0;
        for (int g = 0; g < 16; g++) {
            double lo = 0.0, hi = 0.0;
            for (int l = 0; l < 16; l++) {
                lo = std::min(lo, double(v[b + 16 * g + l]));
                hi = std::max(hi, double(v[b + 16 * g + l]));
            }
            sc[g] = (hi - lo) / 3.0;
            mn[g] = -lo;
            smax = std::max(smax, sc[g]);
            mmax = std::max(mmax, mn[g]);
        }
        const uint16_t hd = f64_to_half(smax / 15.0), hm = f64_to_half(mmax / 15.0);
        const double d = half_to_f64(hd), dmin = half_to_f64(hm);
        put16(dst + 80, hd);
        put16(dst + 82, hm);
        for (int k = 0; k < 64; k++) dst[16 + k] = 0;
        // group g = value index / 16 = 8h + 2j + s
        for (int g = 0; g < 16; g++) {
            const int is = d > 0 ? clampi(std::nearbyint(sc[g] / d), 0, 15) : 0;
            const int im = dmin > 0 ? clampi(std::nearbyint(mn[g] / dmin), 0, 15) : 0;
            dst[g] = static_cast<uint8_t>(is | (im << 4));
            const double dl = d * is, ml = dmin * im;
            const int h = g >> 3, j = (g >> 1) & 3, s = g & 1;
            for (int l = 0; l < 16; l++) {
                const int q = dl > 0 ? clampi(std::nearbyint((double(v[b + 16 * g + l]) + ml) / dl), 0, 3) : 0;
                dst[16 + 32 * h + 16 * s + l] = static_cast<uint8_t>(dst[16 + 32 * h + 16 * s + l] | (q << (2 * j)));
            }
        }
    }
}

// Q3_K (110 B / 256 values): per 16-value group a positive scale amax / 4
// on a 6-bit grid (stored sc - 32 in 1..31 of d = max scale / 31); codes
// round(v / s) in -4..3, stored as 2 bits plus an hmask bit set for codes >= 0.
void quant_q3_k(const float *v, int64_t n, uint8_t *dst) {
    for (int64_t b = 0; b < n; b += 256, dst += 110) {
        double sc[16], smax = 0.0;
        for (int g = 0; g < 16; g++) {
            double amax = 0.0;
            for (int l = 0; l < 16; l++) amax = std::max(amax, std::fabs(double(v[b + 16 * g + l])));
            sc[g] = amax / 4.0;
            smax = std::max(smax, sc[g]);
        }
        const uint16_t hd = f64_to_half(smax / 31.0);
        const double d = half_to_f64(hd);
        for (int k = 0; k < 108; k++) dst[k] = 0;
        put16(dst + 108, hd);
        for (int g = 0; g < 16; g++) {
            const int is = d > 0 ? clampi(std::nearbyint(sc[g] / d), 1, 31) : 1;
            const int s6 = is + 32;
            if (g < 8)
                dst[96 + g] = static_cast<uint8_t>(dst[96 + g] | (s6 & 15));
            else
                dst[96 + g - 8] = static_cast<uint8_t>(dst[96 + g - 8] | ((s6 & 15) << 4));
            dst[104 + (g & 3)] = static_cast<uint8_t>(dst[104 + (g & 3)] | (((s6 >> 4) & 3) << (2 * (g >> 2))));
            const double dl = d * is;
            const int h = g >> 3, j = (g >> 1) & 3, s = g & 1;
            for (int l = 0; l < 16; l++) {
                const int c = dl > 0 ? clampi(std::nearbyint(double(v[b + 16 * g + l]) / dl), -4, 3) : 0;
                const int q = c >= 0 ? c : c + 4;
                dst[32 + 32 * h + 16 * s + l] = static_cast<uint8_t>(dst[32 + 32 * h + 16 * s + l] | (q << (2 * j)));
                if (c >= 0) dst[16 * s + l] = static_cast<uint8_t>(dst[16 * s + l] | (1 << (4 * h + j)));
            }
        }
    }
}

// IQ4_XS (136 B / 256 values): per 32-value sub-block a positive scale
// s = amax / 127 on a 6-bit grid ls - 32 in 1..31 of d = max s / 31, then
// IQ4_NL's nearest grid index of v / (d (ls - 32)).
void quant_iq4_xs(const float *v, int64_t n, uint8_t *dst) {
    static const int grid[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
    for (int64_t b = 0; b < n; b += 256, dst += 136) {
        double s[8], smax = 0.0;
        for (int ib = 0; ib < 8; ib++) {
            double amax = 0.0;
            for (int l = 0; l < 32; l++) amax = std::max(amax, std::fabs(double(v[b + 32 * ib + l])));
            s[ib] = amax / 127.0;
            smax = std::max(smax, s[ib]);
        }
        const uint16_t hd = f64_to_half(smax / 31.0);
        const double d = half_to_f64(hd);
        put16(dst, hd);
        uint16_t sh = 0;
        uint8_t *sl = dst + 4, *qs = dst + 8;
        for (int k = 0; k < 4; k++) sl[k] = 0;
        for (int ib = 0; ib < 8; ib++) {
            const int ls = 32 + (d > 0 ? clampi(std::nearbyint(s[ib] / d), 1, 31) : 1);
            sl[ib / 2] = static_cast<uint8_t>(sl[ib / 2] | ((ls & 15) << (4 * (ib % 2))));
            sh = static_cast<uint16_t>(sh | (((ls >> 4) & 3) << (2 * ib)));
            const double dl = d * (ls - 32);
            int q[32];
            for (int l = 0; l < 32; l++) {
                const double t = dl > 0 ? double(v[b + 32 * ib + l]) / dl : 0.0;
                int best = 0;
                for (int k = 1; k < 16; k++)
                    if (std::fabs(t - grid[k]) < std::fabs(t - grid[best])) best = k;
                q[l] = best;
            }
            for (int l = 0; l < 16; l++) qs[16 * ib + l] = static_cast<uint8_t>(q[l] | (q[l + 16] << 4));
        }
        put16(dst + 2, sh);
    }
}

// Q5_K (176 B / 256 values): Q4_K's header and packed (sc, m) pairs, codes
// in [0, 31] whose bit 4 goes to qh[l] bit 2g (low-nibble sub-block of chunk
// pair g) or 2g+1 (high-nibble sub-block), as deq_q5_k (quant.cpp:462-489)
// reads them back.
void quant_q5_k(const float *v, int64_t n, uint8_t *dst) {
    for (int64_t b = 0; b < n; b += 256, dst += 176) {
        double scale[8], minv[8];
        double smax = 0.0, mmax = 0.0;
        for (int j = 0; j < 8; j++) {
            double lo = 0.0, hi = 0.0;
            for (int l = 0; l < 32; l++) {
                lo = std::min(lo, double(v[b + 32 * j + l]));
                hi = std::max(hi, double(v[b + 32 * j + l]));
            }
            scale[j] = (hi - lo) / 31.0;
            minv[j] = -lo;
            smax = std::max(smax, scale[j]);
            mmax = std::max(mmax, minv[j]);
        }
        const uint16_t hd = f64_to_half(smax / 63.0), hm = f64_to_half(mmax / 63.0);
        const double d = half_to_f64(hd), dmin = half_to_f64(hm);
        int sc[8], mq[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = d > 0 ? clampi(std::nearbyint(scale[j] / d), 0, 63) : 0;
            mq[j] = dmin > 0 ? clampi(std::nearbyint(minv[j] / dmin), 0, 63) : 0;
        }
        put16(dst, hd);
        put16(dst + 2, hm);
        uint8_t *s = dst + 4;
        for (int j = 0; j < 4; j++) {
            s[j] = static_cast<uint8_t>((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            s[j + 4] = static_cast<uint8_t>((mq[j] & 63) | ((mq[j + 4] >> 4) << 6));
            s[j + 8] = static_cast<uint8_t>((sc[j + 4] & 15) | ((mq[j + 4] & 15) << 4));
        }
        int q[256];
        for (int j = 0; j < 8; j++) {
            const double ds = d * sc[j], dm = dmin * mq[j];
            for (int l = 0; l < 32; l++) {
                const double x = double(v[b + 32 * j + l]);
                q[32 * j + l] = ds > 0 ? clampi(std::nearbyint((x + dm) / ds), 0, 31) : 0;
            }
        }
        uint8_t *qh = dst + 16, *qs = dst + 48;
        for (int l = 0; l < 32; l++) qh[l] = 0;
        for (int g = 0; g < 4; g++)
            for (int l = 0; l < 32; l++) {
                const int a = q[64 * g + l], c = q[64 * g + 32 + l];
                qs[32 * g + l] = static_cast<uint8_t>((a & 15) | ((c & 15) << 4));
                qh[l] = static_cast<uint8_t>(qh[l] | ((a >> 4) << (2 * g)) | ((c >> 4) << (2 * g + 1)));
            }
    }
}

// Q6_K (210 B / 256 values): sixteen int8 scales, one per 16 values, codes in
// [-32, 31] stored as q+32 split into ql (4 bits) and qh (2 bits) in the
// plane order deq_q6_k (quant.cpp:491-512) reads them back.
void quant_q6_k(const float *v, int64_t n, uint8_t *dst) {
    for (int64_t b = 0; b < n; b += 256, dst += 210) {
        double scale[16], smax = 0.0;
        for (int j = 0; j < 16; j++) {
            double amax = 0.0, sv = 0.0;
            for (int l = 0; l < 16; l++) {
                const double x = double(v[b + 16 * j + l]);
                if (std::fabs(x) > amax) { amax = std::fabs(x); sv = x; }
            }
            scale[j] = sv / -32.0;  // the signed extreme lands on code -32
            smax = std::max(smax, std::fabs(scale[j]));
        }
        const uint16_t hd = f64_to_half(smax / 127.0);
        const double d = half_to_f64(hd);
        int8_t sc[16];
        for (int j = 0; j < 16; j++)
            sc[j] = static_cast<int8_t>(d > 0 ? clampi(std::nearbyint(scale[j] / d), -127, 127) : 0);
        int q[256];  // q + 32, in [0, 63]
        for (int j = 0; j < 16; j++) {
            const double ds = d * sc[j];
            for (int l = 0; l < 16; l++) {
                const double x = double(v[b + 16 * j + l]);
                q[16 * j + l] = (ds != 0 ? clampi(std::nearbyint(x / ds), -32, 31) : 0) + 32;
            }
        }
        uint8_t *ql = dst, *qh = dst + 128;
        std::memset(dst, 0, 210);
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                const int *qq = q + 128 * h;
                const int q1 = qq[l], q2 = qq[l + 32], q3 = qq[l + 64], q4 = qq[l + 96];
                ql[64 * h + l] = static_cast<uint8_t>((q1 & 15) | ((q3 & 15) << 4));
                ql[64 * h + l + 32] = static_cast<uint8_t>((q2 & 15) | ((q4 & 15) << 4));
                qh[32 * h + l] = static_cast<uint8_t>((q1 >> 4) | ((q2 >> 4) << 2) |
                                                      ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
        std::memcpy(dst + 192, sc, 16);
        put16(dst + 208, hd);
    }
}

}  // namespace

extern "C" void krk_synth_normal(float *v, int64_t n, uint64_t seed, float mean,
                                 float std_, int nthreads) {
    if (!v || n <= 0) return;
    par_rows(n, nthreads, [&](int64_t b, int64_t e) {
        for (int64_t i = b; i < e; i++)
            v[i] = static_cast<float>(double(mean) + double(std_) * normal_at(seed, i));
    });
}

extern "C" int krk_quantize_weights(int wt, const float *v, int64_t n_rows,
                                    int64_t n_in, void *dst, int nthreads) {
    if (!v || !dst || n_rows <= 0 || n_in <= 0) return KRK_ERR_ARG;
    void (*fn)(const float *, int64_t, uint8_t *) = nullptr;
    switch (wt) {
        case KRK_DT_Q8_0: fn = quant_q8_0; break;
        case KRK_DT_Q4_0: fn = quant_q4_0; break;
        case KRK_DT_IQ4_NL: fn = quant_iq4_nl; break;
        case KRK_DT_IQ4_XS: fn = quant_iq4_xs; break;
        case KRK_DT_Q2_K: fn = quant_q2_k; break;
        case KRK_DT_Q3_K: fn = quant_q3_k; break;
        case KRK_DT_MXFP4: fn = quant_mxfp4; break;
        case KRK_DT_Q4_1: fn = quant_l32<4, true>; break;
        case KRK_DT_Q5_0: fn = quant_l32<5, false>; break;
        case KRK_DT_Q5_1: fn = quant_l32<5, true>; break;
        case KRK_DT_F16: fn = quant_f16; break;
        case KRK_DT_BF16: fn = quant_bf16; break;
        case KRK_DT_Q4_K: fn = quant_q4_k; break;
        case KRK_DT_Q5_K: fn = quant_q5_k; break;
        case KRK_DT_Q6_K: fn = quant_q6_k; break;
        default: return KRK_ERR_DTYPE;
    }
    if (!krk_dtype_row_aligned(wt, n_in)) return KRK_ERR_SHAPE;
    const int64_t rb = krk_dtype_row_bytes(wt, n_in);
    uint8_t *out = static_cast<uint8_t *>(dst);
    par_rows(n_rows, nthreads, [&](int64_t b, int64_t e) {
        for (int64_t r = b; r < e; r++) fn(v + r * n_in, n_in, out + r * rb);
    });
    return KRK_OK;
}
