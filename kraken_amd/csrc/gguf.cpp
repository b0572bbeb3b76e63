// gguf.cpp -- GGUF v2/v3 container reader behind the C ABI in krk_gguf.h.
//
// Follows the GGUF specification as the reference reads it
// (src/gguf.cpp:130-470): little-endian header {magic "GGUF", version,
// tensor count u64, metadata count u64}, metadata entries {key, type,
// value}, tensor descriptors {name, n_dims 1..4, ne[], type id, offset},
// then the data section at the next multiple of general.alignment (32 when
// absent or zero); a descriptor's offset is relative to that section.  The
// file is memory-mapped read-only and tensor bytes are never copied on the
// host.  Single files only: a member of a split set is refused by name.
#include "krk_gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

constexpr uint32_t kMagic = 0x46554747u;   // "GGUF"

struct Value {
    uint32_t type = 0, elem = 0;
    uint64_t count = 1;
    int64_t i = 0;      // integral payload (unsigned values zero-extended)
    double f = 0.0;
    bool is_float = false, is_int = false;
    std::string s;
    std::vector<int64_t> ai;
    std::vector<double> af;
    std::vector<std::string> as;
    bool arr_int = false, arr_float = false;
};

struct Cursor {
    const uint8_t *p, *end;
    bool ok = true;
    bool need(uint64_t n) {
        if (!ok || static_cast<uint64_t>(end - p) < n) ok = false;
        return ok;
    }
    template <typename T> T get() {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, p, sizeof(T));
            p += sizeof(T);
        }
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return {};
        std::string s(reinterpret_cast<const char *>(p), static_cast<size_t>(n));
        p += n;
        return s;
    }
};

// one scalar of type t; false for an unknown type
bool scalar(Cursor &c, uint32_t t, Value &v) {
    switch (t) {
        case KRK_GGUF_U8: v.i = c.get<uint8_t>(); v.is_int = true; break;
        case KRK_GGUF_I8: v.i = c.get<int8_t>(); v.is_int = true; break;
        case KRK_GGUF_U16: v.i = c.get<uint16_t>(); v.is_int = true; break;
        case KRK_GGUF_I16: v.i = c.get<int16_t>(); v.is_int = true; break;
        case KRK_GGUF_U32: v.i = c.get<uint32_t>(); v.is_int = true; break;
        case KRK_GGUF_I32: v.i = c.get<int32_t>(); v.is_int = true; break;
        case KRK_GGUF_U64: v.i = static_cast<int64_t>(c.get<uint64_t>()); v.is_int = true; break;
        case KRK_GGUF_I64: v.i = c.get<int64_t>(); v.is_int = true; break;
        case KRK_GGUF_BOOL: v.i = c.get<uint8_t>() != 0; v.is_int = true; break;
        case KRK_GGUF_F32: v.f = c.get<float>(); v.is_float = true; break;
        case KRK_GGUF_F64: v.f = c.get<double>(); v.is_float = true; break;
        case KRK_GGUF_STRING: v.s = c.str(); break;
        default: return false;
    }
    return c.ok;
}

bool value(Cursor &c, Value &v) {
    v.type = c.get<uint32_t>();
    if (!c.ok) return false;
    if (v.type != KRK_GGUF_ARRAY) return scalar(c, v.type, v);
    v.elem = c.get<uint32_t>();
    v.count = c.get<uint64_t>();
    if (!c.ok || v.elem == KRK_GGUF_ARRAY || v.elem > KRK_GGUF_F64) return false;
    // every element takes at least one byte: a count past the file is corrupt
    if (v.count > static_cast<uint64_t>(c.end - c.p)) return false;
    for (uint64_t j = 0; j < v.count; j++) {
        Value e;
        if (!scalar(c, v.elem, e)) return false;
        if (v.elem == KRK_GGUF_STRING) {
            v.as.push_back(std::move(e.s));
        } else if (e.is_float) {
            v.af.push_back(e.f);
            v.arr_float = true;
        } else {
            v.ai.push_back(e.i);
            v.af.push_back(static_cast<double>(e.i));
            v.arr_int = true;
        }
    }
    return true;
}

// geometry of the types this library serves (F32, F16 and krk_dtype)
bool geometry(uint32_t id, int *bs, int *bb) {
    switch (id) {
        case KRK_DT_F32: *bs = 1; *bb = 4; return true;
        case KRK_DT_F16: case KRK_DT_BF16: *bs = 1; *bb = 2; return true;
        case KRK_DT_Q4_0: case KRK_DT_IQ4_NL: *bs = 32; *bb = 18; return true;
        case KRK_DT_Q8_0: *bs = 32; *bb = 34; return true;
        case KRK_DT_Q4_K: *bs = 256; *bb = 144; return true;
        case KRK_DT_Q5_K: *bs = 256; *bb = 176; return true;
        case KRK_DT_IQ4_XS: *bs = 256; *bb = 136; return true;
        case KRK_DT_Q2_K: *bs = 256; *bb = 84; return true;
        case KRK_DT_MXFP4: *bs = 32; *bb = 17; return true;
        case KRK_DT_Q4_1: *bs = 32; *bb = 20; return true;
        case KRK_DT_Q5_0: *bs = 32; *bb = 22; return true;
        case KRK_DT_Q5_1: *bs = 32; *bb = 24; return true;
        case KRK_DT_Q3_K: *bs = 256; *bb = 110; return true;
        case KRK_DT_Q6_K: *bs = 256; *bb = 210; return true;
        // the generic-chunk formats (include/krk/quant.hpp geometry)
        case KRK_DT_Q8_1: *bs = 32; *bb = 36; return true;
        case KRK_DT_Q8_K: *bs = 256; *bb = 292; return true;
        case KRK_DT_TQ1_0: *bs = 256; *bb = 54; return true;
        case KRK_DT_TQ2_0: *bs = 256; *bb = 66; return true;
        case KRK_DT_NVFP4: *bs = 64; *bb = 36; return true;
        case KRK_DT_ROCMFP4: *bs = 32; *bb = 18; return true;
        case KRK_DT_ROCMFP4_FAST: *bs = 32; *bb = 17; return true;
        case KRK_DT_Q6_0_ROCMFPX: *bs = 32; *bb = 26; return true;
        case KRK_DT_Q3_0_ROCMFPX: *bs = 32; *bb = 14; return true;
        case KRK_DT_Q2_0_ROCMFPX: *bs = 32; *bb = 10; return true;
        case KRK_DT_Q1_0: *bs = 128; *bb = 18; return true;
        case KRK_DT_Q2_0: case KRK_DT_PQ2_0: *bs = 128; *bb = 34; return true;
        case KRK_DT_Q2_0_64: *bs = 64; *bb = 18; return true;
        case KRK_DT_PTQ1_0: *bs = 128; *bb = 28; return true;
        default: return false;
    }
}

void say(char *err, size_t len, const char *fmt, ...) {
    if (!err || !len) return;
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(err, len, fmt, ap);
    va_end(ap);
}

}  // namespace

struct krk_gguf {
    void *map = MAP_FAILED;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_off = 0;
    std::vector<std::string> keys;
    std::vector<Value> vals;
    std::unordered_map<std::string, int64_t> kv_index;
    std::vector<std::string> names;
    std::vector<krk_gguf_tensor_info> tensors;
    std::unordered_map<std::string, int64_t> t_index;
    ~krk_gguf() {
        if (map != MAP_FAILED) munmap(map, size);
    }
    const Value *find(const char *key) const {
        if (!key) return nullptr;
        auto it = kv_index.find(key);
        return it == kv_index.end() ? nullptr : &vals[static_cast<size_t>(it->second)];
    }
};

extern "C" {

int krk_gguf_open(const char *path, krk_gguf **out, char *err, size_t err_len) {
    if (!path || !out) return KRK_ERR_ARG;
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        say(err, err_len, "cannot open '%s': %s", path, std::strerror(errno));
        return KRK_ERR_ARG;
    }
    struct stat st{};
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        ::close(fd);
        say(err, err_len, "'%s' is too short for a GGUF header", path);
        return KRK_ERR_SHAPE;
    }
    auto *g = new (std::nothrow) krk_gguf;
    if (!g) {
        ::close(fd);
        return KRK_ERR_NOMEM;
    }
    g->size = static_cast<size_t>(st.st_size);
    g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (g->map == MAP_FAILED) {
        delete g;
        say(err, err_len, "cannot map '%s'", path);
        return KRK_ERR_NOMEM;
    }
    const uint8_t *base = static_cast<const uint8_t *>(g->map);
    Cursor c{base, base + g->size};
    auto fail = [&](const char *what) {
        say(err, err_len, "'%s': %s", path, what);
        delete g;
        return KRK_ERR_SHAPE;
    };
    if (c.get<uint32_t>() != kMagic) return fail("not a GGUF file (bad magic)");
    g->version = c.get<uint32_t>();
    if (g->version < 2 || g->version > 3) return fail("unsupported GGUF version (2 and 3 are read)");
    const uint64_t n_t = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    // each entry and descriptor takes more than 8 bytes
    if (!c.ok || n_t > g->size / 8 || n_kv > g->size / 8) return fail("corrupt header counts");
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key = c.str();
        Value v;
        if (!c.ok || !value(c, v)) return fail("corrupt metadata entry");
        g->kv_index[key] = static_cast<int64_t>(g->keys.size());
        g->keys.push_back(std::move(key));
        g->vals.push_back(std::move(v));
    }
    if (const Value *v = g->find("split.count"); v && v->is_int && v->i > 1)
        return fail("member of a split GGUF set (split.count > 1): not read by this library");
    g->names.reserve(static_cast<size_t>(n_t));
    g->tensors.resize(static_cast<size_t>(n_t));
    for (uint64_t k = 0; k < n_t; k++) {
        krk_gguf_tensor_info &t = g->tensors[static_cast<size_t>(k)];
        g->names.push_back(c.str());
        t.n_dims = static_cast<int>(c.get<uint32_t>());
        if (!c.ok || t.n_dims < 1 || t.n_dims > 4) return fail("corrupt tensor descriptor (n_dims)");
        for (int d = 0; d < 4; d++) t.ne[d] = d < t.n_dims ? c.get<uint64_t>() : 1;
        t.type_id = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (!c.ok) return fail("corrupt tensor descriptor");
        t.n_elements = 1;
        for (int d = 0; d < t.n_dims; d++) t.n_elements *= static_cast<int64_t>(t.ne[d]);
    }
    if (const Value *v = g->find("general.alignment"); v && v->is_int && v->i > 0)
        g->alignment = static_cast<uint64_t>(v->i);
    const uint64_t pos = static_cast<uint64_t>(c.p - base);
    g->data_off = (pos + g->alignment - 1) / g->alignment * g->alignment;
    if (g->data_off > g->size) return fail("tensor data section out of bounds");
    for (uint64_t k = 0; k < n_t; k++) {
        krk_gguf_tensor_info &t = g->tensors[static_cast<size_t>(k)];
        t.name = g->names[static_cast<size_t>(k)].c_str();
        g->t_index[g->names[static_cast<size_t>(k)]] = static_cast<int64_t>(k);
        int bs = 0, bb = 0;
        t.dtype_known = geometry(t.type_id, &bs, &bb);
        t.n_bytes = 0;
        if (t.dtype_known) {
            // row_bytes(ne[0]) * rows, as dtype_row_bytes sizes a row
            const uint64_t row = (t.ne[0] + static_cast<uint64_t>(bs) - 1) / static_cast<uint64_t>(bs) *
                                 static_cast<uint64_t>(bb);
            t.n_bytes = row * static_cast<uint64_t>(t.n_elements / static_cast<int64_t>(t.ne[0] ? t.ne[0] : 1));
            if (t.offset > g->size - g->data_off || t.n_bytes > g->size - g->data_off - t.offset)
                return fail("tensor data out of bounds");
        }
        t.data = t.offset <= g->size - g->data_off ? base + g->data_off + t.offset : nullptr;
    }
    *out = g;
    return KRK_OK;
}

void krk_gguf_close(krk_gguf *g) { delete g; }

uint32_t krk_gguf_version(const krk_gguf *g) { return g ? g->version : 0; }
uint64_t krk_gguf_alignment(const krk_gguf *g) { return g ? g->alignment : 0; }
uint64_t krk_gguf_data_offset(const krk_gguf *g) { return g ? g->data_off : 0; }

int64_t krk_gguf_tensor_count(const krk_gguf *g) { return g ? static_cast<int64_t>(g->tensors.size()) : 0; }

int krk_gguf_tensor(const krk_gguf *g, int64_t i, krk_gguf_tensor_info *out) {
    if (!g || !out || i < 0 || i >= static_cast<int64_t>(g->tensors.size())) return KRK_ERR_ARG;
    *out = g->tensors[static_cast<size_t>(i)];
    return KRK_OK;
}

int64_t krk_gguf_find_tensor(const krk_gguf *g, const char *name) {
    if (!g || !name) return -1;
    auto it = g->t_index.find(name);
    return it == g->t_index.end() ? -1 : it->second;
}

int64_t krk_gguf_kv_count(const krk_gguf *g) { return g ? static_cast<int64_t>(g->keys.size()) : 0; }

const char *krk_gguf_kv_key(const krk_gguf *g, int64_t i) {
    if (!g || i < 0 || i >= static_cast<int64_t>(g->keys.size())) return nullptr;
    return g->keys[static_cast<size_t>(i)].c_str();
}

int krk_gguf_kv_type(const krk_gguf *g, int64_t i, uint32_t *type, uint32_t *elem_type, uint64_t *count) {
    if (!g || i < 0 || i >= static_cast<int64_t>(g->vals.size())) return KRK_ERR_ARG;
    const Value &v = g->vals[static_cast<size_t>(i)];
    if (type) *type = v.type;
    if (elem_type) *elem_type = v.elem;
    if (count) *count = v.type == KRK_GGUF_ARRAY ? v.count : 1;
    return KRK_OK;
}

int64_t krk_gguf_find_kv(const krk_gguf *g, const char *key) {
    if (!g || !key) return -1;
    auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? -1 : it->second;
}

int krk_gguf_get_i64(const krk_gguf *g, const char *key, int64_t *out) {
    const Value *v = g ? g->find(key) : nullptr;
    if (!v || !out || (!v->is_int && !v->is_float)) return KRK_ERR_ARG;
    *out = v->is_float ? static_cast<int64_t>(v->f) : v->i;
    return KRK_OK;
}

int krk_gguf_get_f64(const krk_gguf *g, const char *key, double *out) {
    const Value *v = g ? g->find(key) : nullptr;
    if (!v || !out || (!v->is_int && !v->is_float)) return KRK_ERR_ARG;
    *out = v->is_float ? v->f : static_cast<double>(v->i);
    return KRK_OK;
}

int krk_gguf_get_bool(const krk_gguf *g, const char *key, int *out) {
    const Value *v = g ? g->find(key) : nullptr;
    if (!v || !out || !v->is_int) return KRK_ERR_ARG;
    *out = v->i != 0;
    return KRK_OK;
}

int krk_gguf_get_str(const krk_gguf *g, const char *key, const char **out) {
    const Value *v = g ? g->find(key) : nullptr;
    if (!v || !out || v->type != KRK_GGUF_STRING) return KRK_ERR_ARG;
    *out = v->s.c_str();
    return KRK_OK;
}

int krk_gguf_array_i64(const krk_gguf *g, const char *key, uint64_t j, int64_t *out) {
    const Value *v = g ? g->find(key) : nullptr;
    if (!v || !out || v->type != KRK_GGUF_ARRAY || !v->arr_int || j >= v->ai.size()) return KRK_ERR_ARG;
    *out = v->ai[static_cast<size_t>(j)];
    return KRK_OK;
}

int krk_gguf_array_f64(const krk_gguf *g, const char *key, uint64_t j, double *out) {
    const Value *v = g ? g->find(key) : nullptr;
    if (!v || !out || v->type != KRK_GGUF_ARRAY || v->elem == KRK_GGUF_STRING || j >= v->af.size())
        return KRK_ERR_ARG;
    *out = v->af[static_cast<size_t>(j)];
    return KRK_OK;
}

int krk_gguf_array_str(const krk_gguf *g, const char *key, uint64_t j, const char **out) {
    const Value *v = g ? g->find(key) : nullptr;
    if (!v || !out || v->type != KRK_GGUF_ARRAY || v->elem != KRK_GGUF_STRING || j >= v->as.size())
        return KRK_ERR_ARG;
    *out = v->as[static_cast<size_t>(j)].c_str();
    return KRK_OK;
}

}  // extern "C"
