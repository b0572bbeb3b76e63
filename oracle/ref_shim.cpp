// ref_shim.cpp -- extern "C" entry points over the REFERENCE's own host quant
// code and GGUF reader (src/quant.cpp + src/common.cpp + src/gguf.cpp,
// compiled from /root/reference by oracle/Makefile into
// oracle/_ref/libkrk_ref.so).  Test infrastructure: it
// exists so the C restatement in krk_oracle.c can be compared bit for bit
// with the reference where the reference builds.  The strict scalar tier is
// selected the way the reference's own switches select it
// (include/krk/quant.hpp:245-273): fast, avx2 and int8 tiers off.
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "krk/gguf.hpp"
#include "krk/quant.hpp"

using namespace krk;

static void strict_tier() {
    set_vec_dot_fast(false);
    set_vec_dot_avx2(false);
    set_vec_dot_int8(false);
    set_vec_dot_wide(false);
}

extern "C" {
int64_t ref_row_bytes(int dt, int64_t n) {
    return static_cast<int64_t>(dtype_row_bytes(static_cast<DType>(dt), n));
}
int ref_block_size(int dt) { return dtype_block_size(static_cast<DType>(dt)); }
int ref_block_bytes(int dt) { return dtype_block_bytes(static_cast<DType>(dt)); }
void ref_dequant_row(int dt, const void *src, float *out, int64_t n) {
    dequant_row(static_cast<DType>(dt), src, out, n);
}
void ref_dequant_row_f16(int dt, const void *src, uint16_t *out, int64_t n) {
    dequant_row_f16(static_cast<DType>(dt), src, out, n);
}
float ref_vec_dot(int dt, const void *src, const float *x, int64_t n) {
    strict_tier();
    return vec_dot(static_cast<DType>(dt), src, x, n);
}
// The strict scalar GEMV out[r] = vec_dot(W row r, x), one reference
// vec_dot call per output row, rows split over nthreads std::threads (the
// reference CPU backend's split: src/backend_cpu.cpp:1-8, 914-1320; each row
// is one f32 chain, so the result does not depend on the thread count).
void ref_gemv_strict(int dt, const void *w, int64_t row_bytes, const float *x, int64_t n_out, int64_t n_in,
                     float *out, int nthreads) {
    strict_tier();
    if (nthreads < 1) nthreads = 1;
    std::vector<std::thread> th;
    const int64_t per = (n_out + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        const int64_t r0 = t * per, r1 = r0 + per < n_out ? r0 + per : n_out;
        if (r0 >= r1) break;
        th.emplace_back([=] {
            for (int64_t r = r0; r < r1; r++)
                out[r] = vec_dot(static_cast<DType>(dt), static_cast<const u8 *>(w) + r * row_bytes, x, n_in);
        });
    }
    for (auto &t : th) t.join();
}
void ref_quantize_q8_row(const float *x, int64_t n, int8_t *xq, float *dx) {
    quantize_q8_row(x, n, xq, dx);
}
float ref_dot_q8_0_q8_scalar(const void *w, const int8_t *xq, const float *dx,
                             int64_t n) {
    return dot_q8_0_q8_scalar(static_cast<const u8 *>(w), xq, dx, n);
}
// the CPU int8 twins of the K-quant rung (quant.cpp:3125-3140, 3193-3200)
float ref_dot_q4_K_q8(const void *w, const int8_t *xq, const float *dx, int64_t n) {
    return dot_q4_K_q8(static_cast<const u8 *>(w), xq, dx, n);
}
float ref_dot_q6_K_q8(const void *w, const int8_t *xq, const float *dx, int64_t n) {
    return dot_q6_K_q8(static_cast<const u8 *>(w), xq, dx, n);
}
float ref_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }
uint16_t ref_fp32_to_fp16(float f) { return fp32_to_fp16(f); }

// krk::Gguf (include/krk/gguf.hpp:86-160), for comparing the library's own
// reader with the reference's on the reference's GGUF files
void *ref_gguf_open(const char *path, char *err, size_t n) {
    auto *g = new Gguf;
    std::string e;
    if (!g->load(path, &e)) {
        if (err && n) { std::strncpy(err, e.c_str(), n - 1); err[n - 1] = 0; }
        delete g;
        return nullptr;
    }
    return g;
}
void ref_gguf_close(void *g) { delete static_cast<Gguf *>(g); }
int64_t ref_gguf_tensor_count(void *g) { return static_cast<int64_t>(static_cast<Gguf *>(g)->tensor_count()); }
uint64_t ref_gguf_alignment(void *g) { return static_cast<Gguf *>(g)->alignment(); }
uint64_t ref_gguf_data_offset(void *g) { return static_cast<Gguf *>(g)->data_section_off(); }
uint32_t ref_gguf_version(void *g) { return static_cast<Gguf *>(g)->version(); }
int ref_gguf_tensor(void *gp, int64_t i, char *name, size_t n, uint32_t *type_id, int *known, int *n_dims,
                    uint64_t *ne, uint64_t *offset, int64_t *n_elements, uint64_t *n_bytes) {
    const auto &t = static_cast<Gguf *>(gp)->tensors()[static_cast<size_t>(i)];
    std::strncpy(name, t.name.c_str(), n - 1);
    name[n - 1] = 0;
    *type_id = t.type_id;
    *known = t.dtype_known;
    *n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) ne[d] = t.ne[d];
    *offset = t.offset;
    *n_elements = t.n_elements;
    *n_bytes = t.n_bytes;
    return 0;
}
int64_t ref_gguf_kv_count(void *g) { return static_cast<int64_t>(static_cast<Gguf *>(g)->entries().size()); }
// entry i: key, type, element type and count (arrays), and the scalar
// payload through the reference's own conversions
int ref_gguf_kv(void *gp, int64_t i, char *key, size_t n, uint32_t *type, uint32_t *elem, uint64_t *count,
                int64_t *as_i64, double *as_f64, char *str, size_t sn) {
    const auto &kv = static_cast<Gguf *>(gp)->entries()[static_cast<size_t>(i)];
    std::strncpy(key, kv.first.c_str(), n - 1);
    key[n - 1] = 0;
    const GgufValue &v = kv.second;
    *type = static_cast<uint32_t>(v.type);
    *elem = static_cast<uint32_t>(v.elem);
    // numeric arrays other than f32 / i32 are kept as raw bytes
    const uint32_t e = static_cast<uint32_t>(v.elem);
    const size_t w = e <= 1 || e == 7 ? 1 : e <= 3 ? 2 : e <= 6 ? 4 : 8;
    *count = v.type == GgufType::Array ? (v.elem == GgufType::String ? v.strs.size()
                                          : !v.f32s.empty() ? v.f32s.size()
                                          : !v.i32s.empty() ? v.i32s.size()
                                          : v.raw.size() / w)
                                       : 1;
    *as_i64 = v.as_i64();
    *as_f64 = v.as_f64();
    std::strncpy(str, v.str.c_str(), sn - 1);
    str[sn - 1] = 0;
    return 0;
}
}
