// gguf.cpp - GGUF v2 / v3 reader (include/gguf.h): the header, key-value
// pairs and tensor infos of a file, and optionally a ggml context of tensor
// descriptors (with the data when no_alloc is false), as src/gguf-weights.h
// uses them (gf_load parses with no_alloc = true and maps the data itself).
// Every length and count read from the file is checked against the file size
// before it is used.
#include "gguf.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

namespace {

struct gguf_kv {
    std::string          key;
    gguf_type            type     = GGUF_TYPE_UINT8;
    gguf_type            arr_type = GGUF_TYPE_UINT8;  // ARRAY: element type
    std::vector<uint8_t> data;                        // scalar / array of fixed-size elements
    std::string          str;                         // STRING
    std::vector<std::string> strs;                    // ARRAY of STRING
    size_t               n = 1;                       // ARRAY: element count
};

struct gguf_tinfo {
    std::string name;
    int         n_dims = 0;
    int64_t     ne[4]  = { 1, 1, 1, 1 };
    ggml_type   type   = GGML_TYPE_F32;
    uint64_t    offset = 0;
};

size_t type_size(gguf_type t) {
    switch (t) {
        case GGUF_TYPE_UINT8:
        case GGUF_TYPE_INT8:
        case GGUF_TYPE_BOOL: return 1;
        case GGUF_TYPE_UINT16:
        case GGUF_TYPE_INT16: return 2;
        case GGUF_TYPE_UINT32:
        case GGUF_TYPE_INT32:
        case GGUF_TYPE_FLOAT32: return 4;
        case GGUF_TYPE_UINT64:
        case GGUF_TYPE_INT64:
        case GGUF_TYPE_FLOAT64: return 8;
        default: return 0;
    }
}

// Bounds-checked reader over the file.
struct reader {
    FILE * f;
    size_t size;
    size_t pos = 0;
    bool   ok  = true;

    bool read(void * dst, size_t n) {
        if (!ok || n > size - pos) {
            ok = false;
            return false;
        }
        if (n && fread(dst, 1, n, f) != n) {
            ok = false;
            return false;
        }
        pos += n;
        return true;
    }

    template <typename T> bool get(T & v) { return read(&v, sizeof(T)); }

    bool str(std::string & s) {
        uint64_t n = 0;
        if (!get(n) || n > size - pos) {
            ok = false;
            return false;
        }
        s.resize((size_t) n);
        return read(&s[0], (size_t) n);
    }
};

void fail(const char * fname, const char * what) {
    fprintf(stderr, "gguf_init_from_file: %s: %s\n", fname, what);
}

}  // namespace

struct gguf_context {
    uint32_t                version   = GGUF_VERSION;
    size_t                  alignment = GGUF_DEFAULT_ALIGNMENT;
    size_t                  data_offset = 0;
    std::vector<gguf_kv>    kv;
    std::vector<gguf_tinfo> tensors;
};

extern "C" struct gguf_context * gguf_init_from_file(const char * fname, struct gguf_init_params params) {
    FILE * f = fopen(fname, "rb");
    if (!f) {
        fail(fname, "cannot open");
        return nullptr;
    }
    fseek(f, 0, SEEK_END);
    const long fsize = ftell(f);
    fseek(f, 0, SEEK_SET);
    reader r{ f, fsize > 0 ? (size_t) fsize : 0 };

    char magic[4];
    if (!r.read(magic, 4) || memcmp(magic, GGUF_MAGIC, 4) != 0) {
        fail(fname, "not a GGUF file");
        fclose(f);
        return nullptr;
    }
    auto *   ctx = new gguf_context();
    int64_t  n_tensors = 0, n_kv = 0;
    if (!r.get(ctx->version) || (ctx->version != 2 && ctx->version != 3) || !r.get(n_tensors) || !r.get(n_kv) ||
        n_tensors < 0 || n_kv < 0 || (uint64_t) n_tensors > r.size || (uint64_t) n_kv > r.size) {
        fail(fname, "bad header");
        fclose(f);
        delete ctx;
        return nullptr;
    }
    for (int64_t i = 0; i < n_kv && r.ok; i++) {
        gguf_kv  kv;
        uint32_t t = 0;
        if (!r.str(kv.key) || !r.get(t) || t >= GGUF_TYPE_COUNT) {
            r.ok = false;
            break;
        }
        kv.type = (gguf_type) t;
        if (kv.type == GGUF_TYPE_STRING) {
            r.str(kv.str);
        } else if (kv.type == GGUF_TYPE_ARRAY) {
            uint32_t at = 0;
            uint64_t n  = 0;
            if (!r.get(at) || at >= GGUF_TYPE_COUNT || at == GGUF_TYPE_ARRAY || !r.get(n) || n > r.size) {
                r.ok = false;
                break;
            }
            kv.arr_type = (gguf_type) at;
            kv.n        = (size_t) n;
            if (kv.arr_type == GGUF_TYPE_STRING) {
                kv.strs.resize(kv.n);
                for (size_t j = 0; j < kv.n && r.ok; j++) {
                    r.str(kv.strs[j]);
                }
            } else {
                const size_t es = type_size(kv.arr_type);
                if (es == 0 || kv.n > (r.size - r.pos) / es) {
                    r.ok = false;
                    break;
                }
                kv.data.resize(kv.n * es);
                r.read(kv.data.data(), kv.data.size());
            }
        } else {
            kv.data.resize(type_size(kv.type));
            r.read(kv.data.data(), kv.data.size());
        }
        if (r.ok && kv.key == GGUF_KEY_GENERAL_ALIGNMENT && kv.type == GGUF_TYPE_UINT32) {
            uint32_t a;
            memcpy(&a, kv.data.data(), 4);
            if (a == 0 || (a & (a - 1)) != 0) {
                r.ok = false;
                break;
            }
            ctx->alignment = a;
        }
        ctx->kv.push_back(std::move(kv));
    }
    for (int64_t i = 0; i < n_tensors && r.ok; i++) {
        gguf_tinfo ti;
        uint32_t   nd = 0, ty = 0;
        if (!r.str(ti.name) || !r.get(nd) || nd < 1 || nd > 4) {
            r.ok = false;
            break;
        }
        ti.n_dims = (int) nd;
        for (uint32_t d = 0; d < nd; d++) {
            if (!r.get(ti.ne[d]) || ti.ne[d] < 0) {
                r.ok = false;
            }
        }
        // the element count must fit int64 (as upstream checks: INT64_MAX / ne)
        for (uint32_t d = 1; d < nd && r.ok; d++) {
            int64_t prod = 1;
            for (uint32_t e = 0; e <= d; e++) {
                if (ti.ne[e] != 0 && prod > INT64_MAX / ti.ne[e]) {
                    r.ok = false;
                    break;
                }
                prod *= ti.ne[e];
            }
        }
        if (!r.get(ty) || ty >= GGML_TYPE_COUNT || ggml_blck_size((ggml_type) ty) <= 0 || !r.get(ti.offset) ||
            ti.ne[0] % ggml_blck_size((ggml_type) ty) != 0 || ti.name.size() >= GGML_MAX_NAME) {
            r.ok = false;
            break;
        }
        ti.type = (ggml_type) ty;
        ctx->tensors.push_back(std::move(ti));
    }
    if (!r.ok) {
        fail(fname, "truncated or malformed header");
        fclose(f);
        delete ctx;
        return nullptr;
    }
    ctx->data_offset = (r.pos + ctx->alignment - 1) / ctx->alignment * ctx->alignment;

    if (params.ctx) {
        size_t data_bytes = 0;
        for (const gguf_tinfo & ti : ctx->tensors) {
            // bytes of the tensor; rows x row size is checked against overflow
            // before it is formed, and the data range against the file size
            // without wrap-around
            const size_t rs   = ggml_row_size(ti.type, ti.ne[0]);
            const size_t rows = (size_t) ti.ne[1] * (size_t) ti.ne[2] * (size_t) ti.ne[3];
            const bool   big  = rs != 0 && rows > SIZE_MAX / rs;
            const size_t nb   = big ? SIZE_MAX : rs * rows;
            if (big) {
                fail(fname, "tensor size overflows");
                fclose(f);
                delete ctx;
                return nullptr;
            }
            if (ti.offset % ctx->alignment != 0 || ctx->data_offset > r.size || ti.offset > r.size - ctx->data_offset ||
                nb > r.size - ctx->data_offset - ti.offset) {
                if (!params.no_alloc) {  // data requested: it must be in the file
                    fail(fname, "tensor data outside the file");
                    fclose(f);
                    delete ctx;
                    return nullptr;
                }
            }
            data_bytes = nb > SIZE_MAX - GGUF_DEFAULT_ALIGNMENT || data_bytes > SIZE_MAX - GGUF_DEFAULT_ALIGNMENT - nb
                             ? SIZE_MAX
                             : data_bytes + nb + GGUF_DEFAULT_ALIGNMENT;
        }
        const size_t meta = (ctx->tensors.size() + 1) * ggml_tensor_overhead();
        struct ggml_init_params ip = { meta + (params.no_alloc ? 0 : data_bytes), nullptr, params.no_alloc };
        struct ggml_context * gctx = ggml_init(ip);
        if (!gctx) {
            fail(fname, "ggml_init failed");
            fclose(f);
            delete ctx;
            return nullptr;
        }
        for (const gguf_tinfo & ti : ctx->tensors) {
            struct ggml_tensor * t = ggml_new_tensor(gctx, ti.type, ti.n_dims, ti.ne);
            ggml_set_name(t, ti.name.c_str());
            if (!params.no_alloc) {
                fseek(f, (long) (ctx->data_offset + ti.offset), SEEK_SET);
                if (fread(t->data, 1, ggml_nbytes(t), f) != ggml_nbytes(t)) {
                    fail(fname, "short read of tensor data");
                    ggml_free(gctx);
                    fclose(f);
                    delete ctx;
                    return nullptr;
                }
            }
        }
        *params.ctx = gctx;
    }
    fclose(f);
    return ctx;
}

extern "C" void gguf_free(struct gguf_context * ctx) {
    delete ctx;
}

extern "C" const char * gguf_type_name(enum gguf_type type) {
    static const char * names[GGUF_TYPE_COUNT] = { "u8",  "i8",   "u16", "i16", "u32", "i32", "f32",
                                                   "bool", "str", "arr", "u64", "i64", "f64" };
    return type >= 0 && type < GGUF_TYPE_COUNT ? names[type] : nullptr;
}

extern "C" uint32_t gguf_get_version(const struct gguf_context * ctx) {
    return ctx->version;
}

extern "C" size_t gguf_get_alignment(const struct gguf_context * ctx) {
    return ctx->alignment;
}

extern "C" size_t gguf_get_data_offset(const struct gguf_context * ctx) {
    return ctx->data_offset;
}

extern "C" int64_t gguf_get_n_kv(const struct gguf_context * ctx) {
    return (int64_t) ctx->kv.size();
}

extern "C" int64_t gguf_find_key(const struct gguf_context * ctx, const char * key) {
    for (size_t i = 0; i < ctx->kv.size(); i++) {
        if (ctx->kv[i].key == key) {
            return (int64_t) i;
        }
    }
    return -1;
}

static const gguf_kv & kv_at(const struct gguf_context * ctx, int64_t id, gguf_type want) {
    if (id < 0 || (size_t) id >= ctx->kv.size() || ctx->kv[(size_t) id].type != want) {
        fprintf(stderr, "gguf: key %lld is not of type %s\n", (long long) id, gguf_type_name(want));
        abort();
    }
    return ctx->kv[(size_t) id];
}

extern "C" const char * gguf_get_key(const struct gguf_context * ctx, int64_t key_id) {
    return key_id >= 0 && (size_t) key_id < ctx->kv.size() ? ctx->kv[(size_t) key_id].key.c_str() : nullptr;
}

extern "C" enum gguf_type gguf_get_kv_type(const struct gguf_context * ctx, int64_t key_id) {
    return key_id >= 0 && (size_t) key_id < ctx->kv.size() ? ctx->kv[(size_t) key_id].type : GGUF_TYPE_COUNT;
}

extern "C" enum gguf_type gguf_get_arr_type(const struct gguf_context * ctx, int64_t key_id) {
    return kv_at(ctx, key_id, GGUF_TYPE_ARRAY).arr_type;
}

extern "C" size_t gguf_get_arr_n(const struct gguf_context * ctx, int64_t key_id) {
    return kv_at(ctx, key_id, GGUF_TYPE_ARRAY).n;
}

#define GGUF_SCALAR(fn, ctype, gtype)                                            \
    extern "C" ctype fn(const struct gguf_context * ctx, int64_t key_id) {      \
        ctype v;                                                               \
        memcpy(&v, kv_at(ctx, key_id, gtype).data.data(), sizeof(ctype));      \
        return v;                                                              \
    }
GGUF_SCALAR(gguf_get_val_u8, uint8_t, GGUF_TYPE_UINT8)
GGUF_SCALAR(gguf_get_val_i8, int8_t, GGUF_TYPE_INT8)
GGUF_SCALAR(gguf_get_val_u16, uint16_t, GGUF_TYPE_UINT16)
GGUF_SCALAR(gguf_get_val_i16, int16_t, GGUF_TYPE_INT16)
GGUF_SCALAR(gguf_get_val_u32, uint32_t, GGUF_TYPE_UINT32)
GGUF_SCALAR(gguf_get_val_i32, int32_t, GGUF_TYPE_INT32)
GGUF_SCALAR(gguf_get_val_f32, float, GGUF_TYPE_FLOAT32)
GGUF_SCALAR(gguf_get_val_u64, uint64_t, GGUF_TYPE_UINT64)
GGUF_SCALAR(gguf_get_val_i64, int64_t, GGUF_TYPE_INT64)
GGUF_SCALAR(gguf_get_val_f64, double, GGUF_TYPE_FLOAT64)
#undef GGUF_SCALAR

extern "C" bool gguf_get_val_bool(const struct gguf_context * ctx, int64_t key_id) {
    return kv_at(ctx, key_id, GGUF_TYPE_BOOL).data[0] != 0;
}

extern "C" const char * gguf_get_val_str(const struct gguf_context * ctx, int64_t key_id) {
    return kv_at(ctx, key_id, GGUF_TYPE_STRING).str.c_str();
}

extern "C" int64_t gguf_get_n_tensors(const struct gguf_context * ctx) {
    return (int64_t) ctx->tensors.size();
}

extern "C" int64_t gguf_find_tensor(const struct gguf_context * ctx, const char * name) {
    for (size_t i = 0; i < ctx->tensors.size(); i++) {
        if (ctx->tensors[i].name == name) {
            return (int64_t) i;
        }
    }
    return -1;
}

static const gguf_tinfo & tinfo_at(const struct gguf_context * ctx, int64_t id) {
    if (id < 0 || (size_t) id >= ctx->tensors.size()) {
        fprintf(stderr, "gguf: no tensor %lld\n", (long long) id);
        abort();
    }
    return ctx->tensors[(size_t) id];
}

extern "C" size_t gguf_get_tensor_offset(const struct gguf_context * ctx, int64_t tensor_id) {
    return (size_t) tinfo_at(ctx, tensor_id).offset;
}

extern "C" const char * gguf_get_tensor_name(const struct gguf_context * ctx, int64_t tensor_id) {
    return tinfo_at(ctx, tensor_id).name.c_str();
}

extern "C" enum ggml_type gguf_get_tensor_type(const struct gguf_context * ctx, int64_t tensor_id) {
    return tinfo_at(ctx, tensor_id).type;
}

extern "C" size_t gguf_get_tensor_size(const struct gguf_context * ctx, int64_t tensor_id) {
    const gguf_tinfo & ti = tinfo_at(ctx, tensor_id);
    return ggml_row_size(ti.type, ti.ne[0]) * (size_t) (ti.ne[1] * ti.ne[2] * ti.ne[3]);
}
