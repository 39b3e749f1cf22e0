// gguf.h - the subset of ggml's public GGUF reader API used by minimaxmusic.cpp
// (src/gguf-weights.h:16, :76-362: gf_load / gf_load_tensor / gf_get_str /
// the fused QKV and pair loaders), restated by name and meaning from upstream
// ggml (ggml is an absent submodule of the reference).
//
// File format (GGUF v2 / v3, little endian): magic "GGUF", u32 version,
// i64 tensor count, i64 key-value count; the key-value pairs (gguf string key,
// u32 value type, value); the tensor infos (gguf string name, u32 n_dims,
// i64 ne[n_dims], u32 ggml type, u64 offset relative to the data section);
// padding to general.alignment (default 32); the data section.  A gguf string
// is a u64 byte length followed by the bytes (no terminator).
#pragma once

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#include "ggml.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GGUF_MAGIC             "GGUF"
#define GGUF_VERSION           3
#define GGUF_KEY_GENERAL_ALIGNMENT "general.alignment"
#define GGUF_DEFAULT_ALIGNMENT 32

enum gguf_type {
    GGUF_TYPE_UINT8   = 0,
    GGUF_TYPE_INT8    = 1,
    GGUF_TYPE_UINT16  = 2,
    GGUF_TYPE_INT16   = 3,
    GGUF_TYPE_UINT32  = 4,
    GGUF_TYPE_INT32   = 5,
    GGUF_TYPE_FLOAT32 = 6,
    GGUF_TYPE_BOOL    = 7,
    GGUF_TYPE_STRING  = 8,
    GGUF_TYPE_ARRAY   = 9,
    GGUF_TYPE_UINT64  = 10,
    GGUF_TYPE_INT64   = 11,
    GGUF_TYPE_FLOAT64 = 12,
    GGUF_TYPE_COUNT,
};

struct gguf_context;

struct gguf_init_params {
    bool                   no_alloc;
    // when not NULL, *ctx receives a ggml context holding one tensor per
    // tensor info (named, typed and shaped as in the file); with no_alloc
    // false the tensors also hold the file's data
    struct ggml_context ** ctx;
};

GGML_API struct gguf_context * gguf_init_from_file(const char * fname, struct gguf_init_params params);
GGML_API void                  gguf_free(struct gguf_context * ctx);

GGML_API const char * gguf_type_name(enum gguf_type type);

GGML_API uint32_t gguf_get_version(const struct gguf_context * ctx);
GGML_API size_t   gguf_get_alignment(const struct gguf_context * ctx);
GGML_API size_t   gguf_get_data_offset(const struct gguf_context * ctx);

GGML_API int64_t        gguf_get_n_kv(const struct gguf_context * ctx);
GGML_API int64_t        gguf_find_key(const struct gguf_context * ctx, const char * key);  // -1 if not found
GGML_API const char *   gguf_get_key(const struct gguf_context * ctx, int64_t key_id);
GGML_API enum gguf_type gguf_get_kv_type(const struct gguf_context * ctx, int64_t key_id);
GGML_API enum gguf_type gguf_get_arr_type(const struct gguf_context * ctx, int64_t key_id);
GGML_API size_t         gguf_get_arr_n(const struct gguf_context * ctx, int64_t key_id);

// scalar getters abort when the value has another type (as upstream's do)
GGML_API uint8_t      gguf_get_val_u8(const struct gguf_context * ctx, int64_t key_id);
GGML_API int8_t       gguf_get_val_i8(const struct gguf_context * ctx, int64_t key_id);
GGML_API uint16_t     gguf_get_val_u16(const struct gguf_context * ctx, int64_t key_id);
GGML_API int16_t      gguf_get_val_i16(const struct gguf_context * ctx, int64_t key_id);
GGML_API uint32_t     gguf_get_val_u32(const struct gguf_context * ctx, int64_t key_id);
GGML_API int32_t      gguf_get_val_i32(const struct gguf_context * ctx, int64_t key_id);
GGML_API float        gguf_get_val_f32(const struct gguf_context * ctx, int64_t key_id);
GGML_API uint64_t     gguf_get_val_u64(const struct gguf_context * ctx, int64_t key_id);
GGML_API int64_t      gguf_get_val_i64(const struct gguf_context * ctx, int64_t key_id);
GGML_API double       gguf_get_val_f64(const struct gguf_context * ctx, int64_t key_id);
GGML_API bool         gguf_get_val_bool(const struct gguf_context * ctx, int64_t key_id);
GGML_API const char * gguf_get_val_str(const struct gguf_context * ctx, int64_t key_id);

GGML_API int64_t        gguf_get_n_tensors(const struct gguf_context * ctx);
GGML_API int64_t        gguf_find_tensor(const struct gguf_context * ctx, const char * name);  // -1 if not found
GGML_API size_t         gguf_get_tensor_offset(const struct gguf_context * ctx, int64_t tensor_id);
GGML_API const char *   gguf_get_tensor_name(const struct gguf_context * ctx, int64_t tensor_id);
GGML_API enum ggml_type gguf_get_tensor_type(const struct gguf_context * ctx, int64_t tensor_id);
GGML_API size_t         gguf_get_tensor_size(const struct gguf_context * ctx, int64_t tensor_id);

#ifdef __cplusplus
}
#endif
