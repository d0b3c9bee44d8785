/* Minimal GGUF v2/v3 reader for the oracle (TEST INFRASTRUCTURE ONLY).
 * Restates crates/det-gguf/src/lib.rs:156-520 of mii443/detllm. */
#ifndef DETREF_GGUF_H
#define DETREF_GGUF_H

#include <stddef.h>
#include <stdint.h>

enum {
    G_OK = 0, G_BAD_MAGIC, G_UNSUPPORTED_VERSION, G_TRUNCATED, G_UNSUPPORTED_VALUE_TYPE,
    G_INVALID_UTF8, G_INVALID_TENSOR_OFFSET, G_INVALID_TENSOR_SHAPE, G_TENSOR_NOT_FOUND,
    G_METADATA_NOT_FOUND, G_DUPLICATE_METADATA_KEY, G_DUPLICATE_TENSOR_NAME, G_INVALID_BOOL,
    G_METADATA_TYPE_MISMATCH, G_UNSUPPORTED_TENSOR_TYPE
};

enum { GV_U8 = 0, GV_I8, GV_U16, GV_I16, GV_U32, GV_I32, GV_F32, GV_BOOL, GV_STRING, GV_ARRAY,
       GV_U64, GV_I64, GV_F64 };

typedef struct {
    const char *key;
    size_t key_len;
    uint32_t type;
    union { uint64_t u; int64_t i; double f; int b; } v;
    const char *str;
    size_t str_len;
    uint32_t arr_type;
    uint64_t arr_count;
    size_t arr_offset; /* byte offset of the first element */
} g_kv;

typedef struct {
    const char *name;
    size_t name_len;
    uint32_t ndim;
    uint64_t dims[4];
    uint32_t type;
    uint64_t offset;
} g_tensor;

typedef struct {
    const uint8_t *bytes;
    size_t len;
    uint32_t version;
    g_kv *kv;
    size_t n_kv;
    g_tensor *tensors;
    size_t n_tensors;
    size_t data_offset;
} g_file;

int g_parse(const uint8_t *bytes, size_t len, g_file *out);
void g_free(g_file *f);
const g_kv *g_find_kv(const g_file *f, const char *key);
int g_find_tensor(const g_file *f, const char *name, const g_tensor **out);
int g_meta_u32(const g_file *f, const char *key, uint32_t *out);
int g_meta_f32(const g_file *f, const char *key, float *out);
int g_meta_str(const g_file *f, const char *key, const char **s, size_t *len);
int g_tensor_data(const g_file *f, const g_tensor *t, const uint8_t **data, size_t *len);
int g_tensor_elements(const g_tensor *t, uint64_t *n);
int g_type_size(uint32_t type, uint64_t *type_size, uint64_t *block_size);

#endif
