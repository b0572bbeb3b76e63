/*
 * krk_gguf.h -- C ABI of the GGUF container reader and the verbatim weight
 * upload: real checkpoints' blocks go to the kernels
 * byte for byte, as the reference's model loader uploads them.
 *
 * Replaces krk::Gguf (include/krk/gguf.hpp:86-160, src/gguf.cpp:130-470)
 * for single-file GGUF v2/v3: load(), tensors(), tensor(name), find(key),
 * get_str / get_i64 / get_f64 / get_bool and the array getters, alignment().
 * The file is memory-mapped read-only; tensor data pointers point into the
 * mapping and stay valid until krk_gguf_close.
 */
#ifndef KRK_GGUF_H
#define KRK_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "krk_mi355x.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct krk_gguf krk_gguf;

/* Metadata value types (the GGUF specification; gguf.hpp:13-27). */
enum krk_gguf_type {
    KRK_GGUF_U8 = 0, KRK_GGUF_I8 = 1, KRK_GGUF_U16 = 2, KRK_GGUF_I16 = 3,
    KRK_GGUF_U32 = 4, KRK_GGUF_I32 = 5, KRK_GGUF_F32 = 6, KRK_GGUF_BOOL = 7,
    KRK_GGUF_STRING = 8, KRK_GGUF_ARRAY = 9, KRK_GGUF_U64 = 10, KRK_GGUF_I64 = 11,
    KRK_GGUF_F64 = 12
};

/* One tensor descriptor (GgufTensor, gguf.hpp:64-84).  n_bytes is the data
 * size for the block formats this library serves (krk_dtype, plus F32 and
 * F16); for other type ids it is 0 and dtype_known is 0, as the reference
 * reports ids it has no geometry for. */
typedef struct {
    const char *name;
    uint32_t type_id;
    int dtype_known;
    int n_dims;
    uint64_t ne[4];        /* unused dimensions are 1 */
    uint64_t offset;       /* relative to the tensor data section */
    int64_t n_elements;
    uint64_t n_bytes;
    const void *data;      /* inside the mapping */
} krk_gguf_tensor_info;

/* Gguf::load (gguf.cpp:340-470) for one file.  Errors: KRK_ERR_ARG (null),
 * KRK_ERR_SHAPE (not GGUF, unsupported version, corrupt or out-of-bounds
 * descriptors, a split set), KRK_ERR_NOMEM; err (may be NULL) receives the
 * reason. */
int krk_gguf_open(const char *path, krk_gguf **out, char *err, size_t err_len);
void krk_gguf_close(krk_gguf *g);

uint32_t krk_gguf_version(const krk_gguf *g);
uint64_t krk_gguf_alignment(const krk_gguf *g);          /* general.alignment, default 32 */
uint64_t krk_gguf_data_offset(const krk_gguf *g);        /* file offset of the data section */

int64_t krk_gguf_tensor_count(const krk_gguf *g);
int krk_gguf_tensor(const krk_gguf *g, int64_t i, krk_gguf_tensor_info *out);
int64_t krk_gguf_find_tensor(const krk_gguf *g, const char *name);   /* -1: absent */

/* Metadata in file order (Gguf::entries, gguf.hpp:104).  For an array,
 * elem_type and count describe it; scalars have count 1. */
int64_t krk_gguf_kv_count(const krk_gguf *g);
const char *krk_gguf_kv_key(const krk_gguf *g, int64_t i);
int krk_gguf_kv_type(const krk_gguf *g, int64_t i, uint32_t *type, uint32_t *elem_type, uint64_t *count);
int64_t krk_gguf_find_kv(const krk_gguf *g, const char *key);        /* -1: absent */

/* Scalar getters with the reference's conversions (GgufValue::as_i64 /
 * as_f64, gguf.hpp:47-55; get_bool true for a non-zero integral).  Return
 * KRK_ERR_ARG when the key is absent or not a scalar of a convertible type;
 * *out is then left unchanged (the caller's default). */
int krk_gguf_get_i64(const krk_gguf *g, const char *key, int64_t *out);
int krk_gguf_get_f64(const krk_gguf *g, const char *key, double *out);
int krk_gguf_get_bool(const krk_gguf *g, const char *key, int *out);
int krk_gguf_get_str(const krk_gguf *g, const char *key, const char **out);   /* valid until close */

/* Array elements (get_i32_array / get_f32_array / get_str_array /
 * get_i64_array, gguf.hpp:120-127): element j of array key. */
int krk_gguf_array_i64(const krk_gguf *g, const char *key, uint64_t j, int64_t *out);
int krk_gguf_array_f64(const krk_gguf *g, const char *key, uint64_t j, double *out);
int krk_gguf_array_str(const krk_gguf *g, const char *key, uint64_t j, const char **out);

/* Verbatim upload of tensor i's n_bytes into device memory dst (at least
 * n_bytes), on the handle's stream; the model loader's upload path
 * (model.cpp upload, backend.hpp upload()).  Returns when the source may be
 * released (the copy from the pageable mapping is staged). */
int krk_gguf_upload(krk_backend *b, const krk_gguf *g, int64_t i, void *dst);

#ifdef __cplusplus
}
#endif

#endif /* KRK_GGUF_H */
