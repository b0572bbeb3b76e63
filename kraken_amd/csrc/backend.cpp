// backend.cpp -- the C ABI (include/krk_mi355x.h): argument checks, the
// dispatch per dtype and row count that HipBackend::gemm does
// (backend_hip.hip:3175-3490), and the persistent device scratch the backend
// owns (split/int8/MoE workspaces, backend_hip.hip:3330-3440, 2560-2585).
// Errors are returned as krk_status codes with a message on the handle,
// where the reference aborts (backend_hip.hip:78-82).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "krk_gguf.h"
#include "krk_formats.hpp"
#include "krk_kernels.hpp"
#include "krk_mi355x.h"

// (table, layer, geometry) of an MoE dispatch whose table entry was checked
struct MoeKey {
    const void *table;
    int layer, n_expert;
    int64_t n_embd, n_ff;
    bool operator==(const MoeKey &o) const {
        return table == o.table && layer == o.layer && n_expert == o.n_expert && n_embd == o.n_embd &&
               n_ff == o.n_ff;
    }
};

struct krk_backend {
    int device = 0;
    void *scratch = nullptr;   // this device's address of `scratch` (krk_gemm_noalloc)
    int act = KRK_ACT_F32;
    int path = KRK_PATH_AUTO;
    hipStream_t stream = nullptr;
    void *ws = nullptr;
    size_t ws_bytes = 0;
    // per-tile counters of the MFMA GEMM's in-kernel split-K sum, zeroed at
    // creation and left zero by every call (null: the reduce kernel instead)
    unsigned *tile_cnt = nullptr;
    std::string err;
    static constexpr int kMoeCache = 256;  // layers of MoE tables checked once
    struct MoeOk { MoeKey key; krk_moe_entry e0; bool aligned; bool uniform; };
    MoeOk moe_ok[kMoeCache];
    int n_moe_ok = 0;
};

// Device scratch of krk_gemm_noalloc: split-K partials and int8 activation
// codes live here instead of in the handle's workspace, so that entry point
// never allocates.  Every device the library runs on holds one copy until
// the process ends; calls that overlap on one device share it (and race).
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices];

// this device's address of `scratch` (the host-side name is only a
// stand-in); taken once per device, with that device current
hipError_t scratch_address(int device, void **out) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch[device] = p;
    }
    *out = g_scratch[device];
    return hipSuccess;
}

int fail(krk_backend *b, int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (b) b->err = buf;
    return code;
}

int hip_fail(krk_backend *b, hipError_t e, const char *what) {
    return fail(b, KRK_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// the byte alignment a weight type's loads need at a row start
uintptr_t weight_align(int wt) {
    switch (wt) {
        case KRK_DT_Q4_K: case KRK_DT_Q5_K: case KRK_DT_F16: case KRK_DT_BF16: return 16;
        case KRK_DT_IQ4_XS: return 8;
        case KRK_DT_Q2_K: return 4;
        case KRK_DT_MXFP4: return 1;
        default: return krk::chunk_fmt(wt) ? 1 : 2;   // the generic chunk path: byte loads
    }
}

bool dtype_on_path(int wt) {
    return wt == KRK_DT_Q4_0 || wt == KRK_DT_Q8_0 || wt == KRK_DT_Q4_K || wt == KRK_DT_Q5_K ||
           wt == KRK_DT_Q6_K || wt == KRK_DT_IQ4_NL || wt == KRK_DT_IQ4_XS || wt == KRK_DT_Q2_K ||
           wt == KRK_DT_Q3_K || wt == KRK_DT_MXFP4 || wt == KRK_DT_Q4_1 || wt == KRK_DT_Q5_0 ||
           wt == KRK_DT_Q5_1 || wt == KRK_DT_F16 || wt == KRK_DT_BF16 || krk::chunk_fmt(wt);
}

int make_current(krk_backend *b) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess || cur != b->device) {
        const hipError_t e = hipSetDevice(b->device);
        if (e != hipSuccess) return hip_fail(b, e, "hipSetDevice");
    }
    return KRK_OK;
}

int ensure_ws(krk_backend *b, size_t bytes) {
    if (bytes <= b->ws_bytes) return KRK_OK;
    if (b->ws) {
        // the old scratch may still be read by queued work on this stream
        (void)hipStreamSynchronize(b->stream);
        (void)hipFree(b->ws);
        b->ws = nullptr;
        b->ws_bytes = 0;
    }
    const size_t want = (bytes + (1u << 20) - 1) & ~size_t((1u << 20) - 1);
    const hipError_t e = hipMalloc(&b->ws, want);
    if (e != hipSuccess) {
        b->ws = nullptr;
        return fail(b, KRK_ERR_NOMEM, "scratch of %zu bytes: %s", want, hipGetErrorString(e));
    }
    b->ws_bytes = want;
    return KRK_OK;
}

// Shape and pointer rules shared by every weight-math entry point.
int check_mm(krk_backend *b, const void *out, const void *x, const void *w, int wt,
             int64_t n_out, int64_t n_in, int64_t rows) {
    if (!b) return KRK_ERR_ARG;
    if (!out || !x || !w) return fail(b, KRK_ERR_ARG, "null pointer (out=%p x=%p w=%p)", out, x, w);
    if (n_out <= 0 || n_in <= 0 || rows <= 0)
        return fail(b, KRK_ERR_ARG, "non-positive size n_out=%lld n_in=%lld rows=%lld",
                    (long long)n_out, (long long)n_in, (long long)rows);
    if (!dtype_on_path(wt)) return fail(b, KRK_ERR_DTYPE, "weight type %d is not served", wt);
    if (n_in % 32 != 0 || !krk_dtype_row_aligned(wt, n_in))
        return fail(b, KRK_ERR_SHAPE, "n_in=%lld is not a whole number of %d-value blocks",
                    (long long)n_in, krk_dtype_block_size(wt));
    if (n_in > (int64_t(1) << 30)) return fail(b, KRK_ERR_SHAPE, "n_in=%lld too large", (long long)n_in);
    const uintptr_t wa = reinterpret_cast<uintptr_t>(w);
    if (wa & (weight_align(wt) - 1))
        return fail(b, KRK_ERR_ARG, "weight pointer %p under-aligned for type %d", w, wt);
    if (reinterpret_cast<uintptr_t>(x) & 15)
        return fail(b, KRK_ERR_ARG, "activation pointer %p is not 16-byte aligned", x);
    return KRK_OK;
}

int run_gemv(krk_backend *b, int wt, krk::SegTable &t) {
    const hipError_t e = krk::gemv_segments(wt, b->act == KRK_ACT_F16, t, b->stream);
    if (e != hipSuccess) return hip_fail(b, e, "gemv launch");
    return KRK_OK;
}

krk::SegTable one_seg(const void *w, const void *x, void *out, int wt, int64_t n_out,
                      int64_t n_in, int64_t rows, int kind, const int32_t *rexp) {
    krk::SegTable t{};
    t.n = 1;
    t.n_in = static_cast<int>(n_in);
    t.row_bytes = krk_dtype_row_bytes(wt, n_in);
    t.rows = rows;
    t.x_stride = n_in;
    t.out_stride = n_out;
    t.rexp = rexp;
    t.seg[0] = krk::Seg{w, nullptr, x, out, n_out, 0, kind, 0};
    return t;
}

}  // namespace

extern "C" {

const char *krk_status_string(int s) {
    switch (s) {
        case KRK_OK: return "ok";
        case KRK_ERR_ARG: return "invalid argument";
        case KRK_ERR_DTYPE: return "weight type not served";
        case KRK_ERR_SHAPE: return "shape not addressable";
        case KRK_ERR_HIP: return "HIP runtime error";
        case KRK_ERR_NOMEM: return "out of device memory";
        case KRK_ERR_UNSUPPORTED: return "unsupported";
        default: return "unknown status";
    }
}

int krk_dtype_block_size(int wt) {
    switch (wt) {
        case KRK_DT_F32: case KRK_DT_F16: case KRK_DT_BF16: return 1;
        case KRK_DT_Q4_0: case KRK_DT_Q8_0: case KRK_DT_IQ4_NL: case KRK_DT_MXFP4:
        case KRK_DT_Q4_1: case KRK_DT_Q5_0: case KRK_DT_Q5_1: return 32;
        case KRK_DT_Q2_K: case KRK_DT_Q3_K: case KRK_DT_Q4_K: case KRK_DT_Q5_K: case KRK_DT_Q6_K:
        case KRK_DT_IQ4_XS: return 256;
        default: return krk::chunk_fmt(wt) ? krk::blk_vals(wt) : 0;
    }
}

int krk_dtype_block_bytes(int wt) {
    switch (wt) {
        case KRK_DT_F32: return 4;
        case KRK_DT_F16: case KRK_DT_BF16: return 2;
        case KRK_DT_Q4_0: case KRK_DT_IQ4_NL: return 18;
        case KRK_DT_Q8_0: return 34;
        case KRK_DT_Q4_K: return 144;
        case KRK_DT_Q5_K: return 176;
        case KRK_DT_IQ4_XS: return 136;
        case KRK_DT_Q2_K: return 84;
        case KRK_DT_MXFP4: return 17;
        case KRK_DT_Q4_1: return 20;
        case KRK_DT_Q5_0: return 22;
        case KRK_DT_Q5_1: return 24;
        case KRK_DT_Q3_K: return 110;
        case KRK_DT_Q6_K: return 210;
        default: return krk::chunk_fmt(wt) ? krk::blk_bytes(wt) : 0;
    }
}

int64_t krk_dtype_row_bytes(int wt, int64_t n) {
    const int bs = krk_dtype_block_size(wt);
    if (bs <= 0 || n < 0) return 0;
    return ((n + bs - 1) / bs) * static_cast<int64_t>(krk_dtype_block_bytes(wt));
}

int krk_dtype_row_aligned(int wt, int64_t n) {
    const int bs = krk_dtype_block_size(wt);
    if (bs <= 0) return 0;
    return bs <= 1 || (n % bs) == 0;
}

int krk_backend_create(int device, int act, krk_backend **out) {
    if (!out) return KRK_ERR_ARG;
    *out = nullptr;
    if (act != KRK_ACT_F32 && act != KRK_ACT_F16) return KRK_ERR_ARG;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return KRK_ERR_HIP;
    if (device < 0 || device >= n) return KRK_ERR_ARG;
    if (hipSetDevice(device) != hipSuccess) return KRK_ERR_HIP;
    krk_backend *b = new krk_backend();
    b->device = device;
    b->act = act;
    // krk_gemm_noalloc's scratch address on this device; a failure here
    // leaves it null, and only that entry point reports it
    if (scratch_address(device, &b->scratch) != hipSuccess) b->scratch = nullptr;
    const size_t cb = sizeof(unsigned) * krk::kTileCounters;
    if (hipMalloc(&b->tile_cnt, cb) != hipSuccess) {
        b->tile_cnt = nullptr;
    } else if (hipMemset(b->tile_cnt, 0, cb) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        (void)hipFree(b->tile_cnt);
        b->tile_cnt = nullptr;
    }
    *out = b;
    return KRK_OK;
}

int krk_backend_destroy(krk_backend *b) {
    if (!b) return KRK_ERR_ARG;
    if (b->ws || b->tile_cnt) {
        (void)hipSetDevice(b->device);
        (void)hipStreamSynchronize(b->stream);
        if (b->ws) (void)hipFree(b->ws);
        if (b->tile_cnt) (void)hipFree(b->tile_cnt);
    }
    delete b;
    return KRK_OK;
}

int krk_set_stream(krk_backend *b, void *stream) {
    if (!b) return KRK_ERR_ARG;
    b->stream = static_cast<hipStream_t>(stream);
    return KRK_OK;
}

int krk_set_gemm_path(krk_backend *b, int path) {
    if (!b) return KRK_ERR_ARG;
    if (path < KRK_PATH_AUTO || path > KRK_PATH_INT8) return fail(b, KRK_ERR_ARG, "gemm path %d", path);
    b->path = path;
    return KRK_OK;
}

int krk_act_type(const krk_backend *b) { return b ? b->act : KRK_ERR_ARG; }

int krk_sync(krk_backend *b) {
    if (!b) return KRK_ERR_ARG;
    if (int s = make_current(b)) return s;
    const hipError_t e = hipStreamSynchronize(b->stream);
    return e == hipSuccess ? KRK_OK : hip_fail(b, e, "hipStreamSynchronize");
}

const char *krk_last_error(const krk_backend *b) { return b ? b->err.c_str() : "null handle"; }

int krk_gemm_k_ok(const krk_backend *b, int64_t k) {
    (void)b;
    return k > 0 && (k % 32) == 0 && k <= (int64_t(1) << 30);
}

}  // extern "C"

namespace {

// gemm with its scratch either in the handle's workspace (grown on demand,
// ws == nullptr) or in a caller-fixed buffer of ws_bytes (never allocates)
int gemm_impl(krk_backend *b, void *out, const void *x, const void *w, int wt, int64_t n_out, int64_t n_in,
              int64_t rows, void *ws, size_t ws_bytes) {
    if (int s = check_mm(b, out, x, w, wt, n_out, n_in, rows)) return s;
    if (int s = make_current(b)) return s;
    const bool f16 = b->act == KRK_ACT_F16;
    const bool fixed = ws != nullptr;
    if (rows <= 8 || b->path == KRK_PATH_EXACT) {
        krk::SegTable t = one_seg(w, x, out, wt, n_out, n_in, rows, krk::SEG_PLAIN, nullptr);
        if (rows > 1 && rows <= 8) {
            // the streaming kernel's digit tables of the rows, built once per call
            const size_t need = krk::gemv_stream_xtab_bytes(rows, n_in);
            if (fixed) {
                if (need > ws_bytes)
                    return fail(b, KRK_ERR_NOMEM, "gemv rows need %zu bytes of scratch; the fixed scratch holds %zu",
                                need, ws_bytes);
            } else {
                if (int s = ensure_ws(b, need)) return s;
                ws = b->ws;
            }
            t.xtab = static_cast<uint8_t *>(ws);
        }
        return run_gemv(b, wt, t);
    }
    const int64_t rb = krk_dtype_row_bytes(wt, n_in);
    if (b->path == KRK_PATH_INT8) {
        if (!krk::gemm_int8_serves(wt))
            return fail(b, KRK_ERR_UNSUPPORTED, "the int8 rung serves Q8_0, Q4_K, Q5_K and Q6_K weights");
        const size_t need = krk::gemm_int8_workspace(rows, n_in);
        if (fixed && need > ws_bytes)
            return fail(b, KRK_ERR_NOMEM, "int8 gemm needs %zu bytes of scratch; the fixed scratch holds %zu",
                        need, ws_bytes);
        if (!fixed) {
            if (int s = ensure_ws(b, need)) return s;
            ws = b->ws;
            ws_bytes = b->ws_bytes;
        }
        const hipError_t e = krk::gemm_int8(wt, w, rb, x, f16, out, rows, n_out, n_in, ws, ws_bytes, b->stream);
        return e == hipSuccess ? KRK_OK : hip_fail(b, e, "int8 gemm");
    }
    // a fixed scratch needs the least the GEMM runs with; the growing
    // workspace takes what its fastest form needs
    const size_t need = krk::gemm_mfma_workspace(wt, rows, n_out, n_in, fixed);
    if (fixed && need > ws_bytes)
        return fail(b, KRK_ERR_NOMEM, "mfma gemm needs %zu bytes of split-K scratch; the fixed scratch holds %zu",
                    need, ws_bytes);
    if (!fixed) {
        if (int s = ensure_ws(b, need)) return s;
        ws = b->ws;
        ws_bytes = b->ws_bytes;
    }
    const hipError_t e = krk::gemm_mfma(wt, w, rb, x, f16, out, rows, n_out, n_in, ws, ws_bytes,
                                           b->tile_cnt, b->stream);
    return e == hipSuccess ? KRK_OK : hip_fail(b, e, "mfma gemm");
}

}  // namespace

extern "C" {

int krk_gemm(krk_backend *b, void *out, const void *x, const void *w, int wt, int64_t n_out,
             int64_t n_in, int64_t rows) {
    return gemm_impl(b, out, x, w, wt, n_out, n_in, rows, nullptr, 0);
}

int krk_gemm_noalloc(krk_backend *b, void *out, const void *x, const void *w, int wt, int64_t n_out,
                     int64_t n_in, int64_t rows) {
    if (!b) return KRK_ERR_ARG;
    if (!b->scratch) return fail(b, KRK_ERR_HIP, "gemm_noalloc: no scratch address on device %d", b->device);
    return gemm_impl(b, out, x, w, wt, n_out, n_in, rows, b->scratch, kScratchBytes);
}

size_t krk_gemm_noalloc_scratch_bytes(void) { return kScratchBytes; }

int krk_gemm_accumulate(krk_backend *b, void *dst, const void *x, const void *w, int wt,
                        int64_t n_out, int64_t n_in, int64_t rows, const int32_t *rexp,
                        int *fused) {
    if (fused) *fused = 0;
    if (int s = check_mm(b, dst, x, w, wt, n_out, n_in, rows)) return s;
    if (dst == x) return fail(b, KRK_ERR_ARG, "gemm_accumulate: x must not alias dst");
    if (rows != 1) return KRK_OK;  // declined: the caller does gemm + add
    if (int s = make_current(b)) return s;
    krk::SegTable t = one_seg(w, x, dst, wt, n_out, n_in, rows, krk::SEG_ACC, rexp);
    if (int s = run_gemv(b, wt, t)) return s;
    if (fused) *fused = 1;
    return KRK_OK;
}

int krk_gemm_group(krk_backend *b, void *const out[], const void *x, const void *const w[],
                   int wt, const int64_t n_out[], int64_t n_in, int n_mat, int64_t rows,
                   int silu, int *silu_fused, int row_parallel_only, const int wts[],
                   const void *const xs[], int *fused) {
    (void)row_parallel_only;  // every launch here is row-parallel (no split-K)
    if (silu_fused) *silu_fused = 0;
    if (fused) *fused = 0;
    if (!b) return KRK_ERR_ARG;
    if (!out || !w || !n_out || n_mat <= 0) return fail(b, KRK_ERR_ARG, "gemm_group: empty group");
    if (silu && n_mat < 2) return fail(b, KRK_ERR_ARG, "gemm_group: silu needs gate and up");
    bool uniform = true;
    for (int m = 0; m < n_mat; m++) {
        const int t = wts ? wts[m] : wt;
        const void *xm = xs ? xs[m] : x;
        if (int s = check_mm(b, out[m], xm, w[m], t, n_out[m], n_in, rows)) return s;
        if (t != (wts ? wts[0] : wt)) uniform = false;
    }
    if (silu && n_out[0] != n_out[1]) return fail(b, KRK_ERR_SHAPE, "gate/up row counts differ");
    if (int s = make_current(b)) return s;
    const int t0 = wts ? wts[0] : wt;
    const int nseg = n_mat - (silu ? 1 : 0);
    if (rows != 1 || !uniform || nseg > krk::kMaxSegs) {
        // the default Backend::gemm_group: one gemm per matrix, activation
        // left to the caller
        for (int m = 0; m < n_mat; m++)
            if (int s = krk_gemm(b, out[m], xs ? xs[m] : x, w[m], wts ? wts[m] : wt, n_out[m], n_in,
                                 rows))
                return s;
        return KRK_OK;
    }
    krk::SegTable t{};
    t.n_in = static_cast<int>(n_in);
    t.row_bytes = krk_dtype_row_bytes(t0, n_in);
    t.rows = 1;
    t.x_stride = n_in;
    t.out_stride = 0;
    int k = 0;
    if (silu) {
        t.seg[k++] = krk::Seg{w[0], w[1], xs ? xs[0] : x, out[0], n_out[0], 0, krk::SEG_SILU, 0};
    }
    for (int m = silu ? 2 : 0; m < n_mat; m++)
        t.seg[k++] = krk::Seg{w[m], nullptr, xs ? xs[m] : x, out[m], n_out[m], 0, krk::SEG_PLAIN, 0};
    t.n = k;
    if (int s = run_gemv(b, t0, t)) return s;
    if (silu_fused) *silu_fused = silu ? 1 : 0;
    if (fused) *fused = 1;
    return KRK_OK;
}

int krk_router_softmax_supported(const krk_backend *b) { return b ? 1 : 0; }
int krk_router_topk_supported(const krk_backend *b) { return b ? 1 : 0; }

int krk_router_softmax(krk_backend *b, void *probs, const void *logits, int64_t n_rows,
                       int n_expert) {
    if (!b) return KRK_ERR_ARG;
    if (!probs || !logits || n_rows <= 0 || n_expert <= 0 || n_expert > 1024)
        return fail(b, KRK_ERR_ARG, "router_softmax: bad arguments");
    if (int s = make_current(b)) return s;
    const hipError_t e = krk::router_softmax(logits, b->act == KRK_ACT_F16,
                                             static_cast<float *>(probs), n_rows, n_expert, b->stream);
    return e == hipSuccess ? KRK_OK : hip_fail(b, e, "router_softmax");
}

int krk_router_topk(krk_backend *b, const void *probs, int64_t n_rows, int n_expert, int k,
                    void *ids, void *wts, int normalize, float scale) {
    if (!b) return KRK_ERR_ARG;
    if (!probs || !ids || !wts || n_rows <= 0 || n_expert <= 0 || n_expert > 1024 || k <= 0 ||
        k > n_expert || k > 64)
        return fail(b, KRK_ERR_ARG, "router_topk: bad arguments");
    if (int s = make_current(b)) return s;
    const hipError_t e = krk::router_topk(static_cast<const float *>(probs), n_rows, n_expert, k,
                                          static_cast<int32_t *>(ids), static_cast<float *>(wts),
                                          normalize, scale, b->stream);
    return e == hipSuccess ? KRK_OK : hip_fail(b, e, "router_topk");
}

int krk_scan_accum_supported(const krk_backend *b) { return b ? 1 : 0; }

int krk_scan_accum(krk_backend *b, const void *probs, const void *ids, int64_t n_rows, int n_expert, int k,
                   int layer, void *hits, void *mass) {
    if (!b) return KRK_ERR_ARG;
    if (!probs || !ids || !hits || !mass || n_rows <= 0 || n_expert <= 0 || n_expert > 1024 || k <= 0 ||
        layer < 0 || n_rows > (int64_t(1) << 30))
        return fail(b, KRK_ERR_ARG, "scan_accum: bad arguments");
    if (int s = make_current(b)) return s;
    const hipError_t e = krk::scan_accum(static_cast<const float *>(probs), static_cast<const int32_t *>(ids), n_rows,
                                         n_expert, k, layer, static_cast<unsigned *>(hits),
                                         static_cast<float *>(mass), b->stream);
    return e == hipSuccess ? KRK_OK : hip_fail(b, e, "scan_accum");
}

int krk_moe_plan_build(krk_backend *b, const void *ids, int64_t n_rows, int k, int n_expert, void *off,
                       void *rows, void *wt, const void *wts) {
    if (!b) return KRK_ERR_ARG;
    if (!ids || !off || !rows || !wt || n_rows <= 0 || k <= 0 || n_expert <= 0 || n_expert > 1024 ||
        n_rows * k > (int64_t(1) << 30))
        return fail(b, KRK_ERR_ARG, "moe_plan_build: bad arguments");
    if (int s = make_current(b)) return s;
    const hipError_t e = krk::moe_plan_build(static_cast<const int32_t *>(ids), n_rows, k, n_expert,
                                             static_cast<int32_t *>(off), static_cast<int32_t *>(rows),
                                             static_cast<float *>(wt), static_cast<const float *>(wts), b->stream);
    return e == hipSuccess ? KRK_OK : hip_fail(b, e, "moe_plan_build");
}

int krk_moe_dispatch_supported(const krk_backend *b) { return b ? 1 : 0; }

int krk_moe_dispatch(krk_backend *b, const void *table, int layer, int n_expert, const void *ids,
                     const void *wts, const void *xn, void *out, int64_t n_tok, int64_t n_embd,
                     int64_t n_ff, int k) {
    if (!b) return KRK_ERR_ARG;
    if (!table || !ids || !wts || !xn || !out || n_tok <= 0 || k <= 0 || n_expert <= 0 ||
        layer < 0 || k > n_expert)
        return fail(b, KRK_ERR_ARG, "moe_dispatch: bad arguments");
    if ((n_embd % 256) || (n_ff % 256))
        return fail(b, KRK_ERR_SHAPE, "moe_dispatch: n_embd=%lld n_ff=%lld must be multiples of 256",
                    (long long)n_embd, (long long)n_ff);
    if (reinterpret_cast<uintptr_t>(xn) & 15)
        return fail(b, KRK_ERR_ARG, "moe_dispatch: xn is not 16-byte aligned");
    if (int s = make_current(b)) return s;
    // The table lives on the device and the kernels read the routed entries
    // there.  The host checks the layer once per (table, layer): the first
    // call reads the layer's entries back (one synchronous copy), later calls
    // find the result in the cache and stay asynchronous, so a steady-state
    // dispatch can be captured in a graph.  A table rewritten in place after
    // its first use is not re-checked.
    krk_moe_entry e0{};
    bool aligned = false, uniform = true;
    const krk_moe_entry *tab = static_cast<const krk_moe_entry *>(table);
    const MoeKey key{table, layer, n_expert, n_embd, n_ff};
    int hit = -1;
    for (int i = 0; i < b->n_moe_ok; i++)
        if (b->moe_ok[i].key == key) { hit = i; break; }
    if (hit >= 0) {
        e0 = b->moe_ok[hit].e0;
        aligned = b->moe_ok[hit].aligned;
        uniform = b->moe_ok[hit].uniform;
    } else {
        // every bank of the layer: present, of a served type with its rows
        // aligned for that type's loads, the layer's geometry; whether all
        // rows start 16-byte aligned, and whether every expert has expert
        // 0's types with gate = up (the matrix-core paths take uniform Q4_K
        // layers; the VALU kernels read each expert's types from the table)
        std::vector<krk_moe_entry> ents(static_cast<size_t>(n_expert));
        hipError_t he = hipMemcpyAsync(ents.data(), tab + static_cast<int64_t>(layer) * n_expert,
                                       sizeof(krk_moe_entry) * ents.size(), hipMemcpyDeviceToHost, b->stream);
        if (he == hipSuccess) he = hipStreamSynchronize(b->stream);
        if (he != hipSuccess) return hip_fail(b, he, "moe_dispatch: reading the table");
        e0 = ents[0];
        aligned = true;
        for (int e = 0; e < n_expert; e++) {
            const krk_moe_entry &en = ents[static_cast<size_t>(e)];
            for (int m = 0; m < 3; m++) {
                if (!en.present[m] || !dtype_on_path(en.type[m]))
                    return fail(b, KRK_ERR_UNSUPPORTED, "moe_dispatch: expert %d matrix %d absent or of type %d",
                                e, m, en.type[m]);
                // the original bank types run unaligned rows on the VALU path;
                // the others need their loads' alignment at every row start
                const bool legacy = en.type[m] == KRK_DT_Q4_0 || en.type[m] == KRK_DT_Q8_0 ||
                                    en.type[m] == KRK_DT_Q4_K || en.type[m] == KRK_DT_Q6_K;
                if (!legacy && ((reinterpret_cast<uintptr_t>(en.p[m]) | static_cast<uintptr_t>(en.row_bytes[m])) &
                                (weight_align(en.type[m]) - 1)))
                    return fail(b, KRK_ERR_ARG, "moe_dispatch: expert %d matrix %d rows under-aligned for type %d",
                                e, m, en.type[m]);
                // the types may vary from expert to expert and between gate
                // and up
                if (en.type[m] != e0.type[m] || en.type[1] != en.type[0]) uniform = false;
                if (reinterpret_cast<uintptr_t>(en.p[m]) & 15) aligned = false;
                // the kernels step every bank's rows by its type's row size
                if (en.row_bytes[m] != krk_dtype_row_bytes(en.type[m], en.n_in[m]))
                    return fail(b, KRK_ERR_ARG,
                                "moe_dispatch: expert %d matrix %d row_bytes %lld is not the row size %lld of "
                                "type %d at n_in %lld",
                                e, m, (long long)en.row_bytes[m],
                                (long long)krk_dtype_row_bytes(en.type[m], en.n_in[m]), en.type[m],
                                (long long)en.n_in[m]);
            }
            if (en.n_in[0] != n_embd || en.n_out[0] != n_ff || en.n_in[1] != n_embd || en.n_out[1] != n_ff ||
                en.n_in[2] != n_ff || en.n_out[2] != n_embd)
                return fail(b, KRK_ERR_SHAPE, "moe_dispatch: expert %d geometry does not match n_embd/n_ff", e);
        }
        // remember it; a full record drops its oldest entry (that layer is
        // read and checked again on its next dispatch)
        if (b->n_moe_ok < krk_backend::kMoeCache) {
            b->moe_ok[b->n_moe_ok++] = {key, e0, aligned, uniform};
        } else {
            for (int i = 1; i < krk_backend::kMoeCache; i++) b->moe_ok[i - 1] = b->moe_ok[i];
            b->moe_ok[krk_backend::kMoeCache - 1] = {key, e0, aligned, uniform};
        }
    }
    krk::MoeArgs a{};
    a.table = table; a.layer = layer; a.n_expert = n_expert; a.k = k;
    a.ids = static_cast<const int32_t *>(ids);
    a.wts = static_cast<const float *>(wts);
    a.xn = xn; a.out = out;
    a.n_tok = n_tok; a.n_embd = n_embd; a.n_ff = n_ff;
    a.act_f16 = b->act == KRK_ACT_F16;
    // (a layer whose types vary across experts: no single type, the VALU
    // kernels' per-expert switch)
    a.wt = uniform ? e0.type[0] : -1;
    a.wt_down = uniform ? e0.type[2] : -1;
    a.rb_gate = e0.row_bytes[0]; a.rb_up = e0.row_bytes[1]; a.rb_down = e0.row_bytes[2];
    a.aligned16 = aligned;
    a.mfma = b->path != KRK_PATH_EXACT;
    if (int s = ensure_ws(b, krk::moe_workspace(n_tok, k, n_expert, n_embd, n_ff))) return s;
    const hipError_t he = krk::moe_dispatch(a, b->ws, b->ws_bytes, b->stream);
    return he == hipSuccess ? KRK_OK : hip_fail(b, he, "moe_dispatch");
}

int krk_moe_table_forget(krk_backend *b, const void *table) {
    if (!b) return KRK_ERR_ARG;
    int n = 0;
    for (int i = 0; i < b->n_moe_ok; i++)
        if (b->moe_ok[i].key.table != table) b->moe_ok[n++] = b->moe_ok[i];
    b->n_moe_ok = n;
    return KRK_OK;
}

int krk_dequant_rows_f32(krk_backend *b, float *out, const void *w, int wt, int64_t n_rows,
                         int64_t n_in) {
    if (!b) return KRK_ERR_ARG;
    if (!out || !w || n_rows <= 0 || n_in <= 0) return fail(b, KRK_ERR_ARG, "dequant: bad arguments");
    if (!dtype_on_path(wt)) return fail(b, KRK_ERR_DTYPE, "weight type %d is not served", wt);
    if (!krk_dtype_row_aligned(wt, n_in)) return fail(b, KRK_ERR_SHAPE, "dequant: ragged row");
    if (int s = make_current(b)) return s;
    const hipError_t e = krk::dequant_rows(wt, w, krk_dtype_row_bytes(wt, n_in), n_rows, n_in, out,
                                           false, b->stream);
    return e == hipSuccess ? KRK_OK : hip_fail(b, e, "dequant");
}

int krk_dequant_rows_f16(krk_backend *b, void *out, const void *w, int wt, int64_t n_rows,
                         int64_t n_in) {
    if (!b) return KRK_ERR_ARG;
    if (!out || !w || n_rows <= 0 || n_in <= 0) return fail(b, KRK_ERR_ARG, "dequant: bad arguments");
    if (!dtype_on_path(wt)) return fail(b, KRK_ERR_DTYPE, "weight type %d is not served", wt);
    if (!krk_dtype_row_aligned(wt, n_in)) return fail(b, KRK_ERR_SHAPE, "dequant: ragged row");
    if (int s = make_current(b)) return s;
    const hipError_t e = krk::dequant_rows(wt, w, krk_dtype_row_bytes(wt, n_in), n_rows, n_in, out,
                                           true, b->stream);
    return e == hipSuccess ? KRK_OK : hip_fail(b, e, "dequant");
}

int krk_quantize_q8_rows(krk_backend *b, const float *x, int64_t rows, int64_t n, int8_t *xq,
                         float *dx) {
    if (!b) return KRK_ERR_ARG;
    if (!x || !xq || !dx || rows <= 0 || n <= 0 || n % 32)
        return fail(b, KRK_ERR_ARG, "quantize_q8: bad arguments");
    if (int s = make_current(b)) return s;
    const hipError_t e = krk::quantize_q8_rows(x, false, rows, n, xq, dx, b->stream);
    return e == hipSuccess ? KRK_OK : hip_fail(b, e, "quantize_q8");
}

}  // extern "C"

// Verbatim upload of a GGUF tensor (the model loader's upload of raw block
// bytes): the mapping is pageable, so the copy is staged and the call waits
// for it before the source may be unmapped.
extern "C" int krk_gguf_upload(krk_backend *b, const krk_gguf *g, int64_t i, void *dst) {
    if (!b) return KRK_ERR_ARG;
    krk_gguf_tensor_info t{};
    if (!g || !dst || krk_gguf_tensor(g, i, &t) != KRK_OK) return fail(b, KRK_ERR_ARG, "gguf_upload: bad arguments");
    if (!t.dtype_known) return fail(b, KRK_ERR_DTYPE, "gguf_upload: tensor '%s' has type %u", t.name, t.type_id);
    if (int s = make_current(b)) return s;
    hipError_t e = hipMemcpyAsync(dst, t.data, t.n_bytes, hipMemcpyHostToDevice, b->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(b->stream);
    return e == hipSuccess ? KRK_OK : hip_fail(b, e, "gguf_upload");
}
