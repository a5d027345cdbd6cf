// GGUF v2/v3 reader (slm_gguf.h): a read-only mapping of the file, its
// metadata and tensor directory, and checked tensor views.  The format and
// its checks follow static-lm's loader (src/memory/loader.rs); the code is
// this library's own.
#include "../../include/slm_gguf.h"

#include <fcntl.h>
#include <stdio.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <new>
#include <string>
#include <unordered_map>

namespace slm_host {
int fail(slm_attn_ctx* c, int code, const std::string& msg);
}

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read little-endian
constexpr uint64_t kDefaultAlignment = 32;

struct Value {
    int32_t type = 0;
    int64_t i64 = 0;
    uint64_t u64 = 0;
    double f64 = 0.0;
    const char* str = nullptr;
    uint64_t str_len = 0;
    int32_t elem_type = 0;
    uint64_t len = 0;
    uint64_t byte_offset = 0;
    uint64_t byte_len = 0;
};

struct Tensor {
    int32_t ggml_type = 0;
    int32_t n_dims = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint64_t offset = 0;
};

// Reads little-endian fields from the mapping; every read is bounds-checked
// and a short read is GgufError::UnexpectedEof (ByteCursor, loader.rs:180-318).
struct Cursor {
    const uint8_t* base;
    uint64_t size;
    uint64_t pos = 0;
    int err = 0;
    std::string what;

    bool take(uint64_t n, const uint8_t** p) {
        if (err) return false;
        if (n > size - pos) {  // pos <= size always
            err = SLM_ERR_EOF;
            what = "UnexpectedEof";
            return false;
        }
        *p = base + pos;
        pos += n;
        return true;
    }
    template <class T>
    bool read(T* out) {
        const uint8_t* p;
        if (!take(sizeof(T), &p)) return false;
        memcpy(out, p, sizeof(T));  // the file is little-endian, so is gfx950's host
        return true;
    }
    bool read_str(const char** s, uint64_t* len) {
        uint64_t n = 0;
        const uint8_t* p;
        if (!read(&n) || !take(n, &p)) return false;
        if (!valid_utf8(p, n)) {
            err = SLM_ERR_UTF8;
            what = "InvalidUtf8";
            return false;
        }
        *s = reinterpret_cast<const char*>(p);
        *len = n;
        return true;
    }
    static bool valid_utf8(const uint8_t* p, uint64_t n) {
        uint64_t i = 0;
        while (i < n) {
            const uint8_t c = p[i];
            int extra;
            uint32_t cp;
            if (c < 0x80) {
                ++i;
                continue;
            } else if ((c & 0xE0) == 0xC0) {
                extra = 1;
                cp = c & 0x1F;
            } else if ((c & 0xF0) == 0xE0) {
                extra = 2;
                cp = c & 0x0F;
            } else if ((c & 0xF8) == 0xF0) {
                extra = 3;
                cp = c & 0x07;
            } else {
                return false;
            }
            if (n - i <= (uint64_t)extra) return false;
            for (int k = 1; k <= extra; ++k) {
                if ((p[i + k] & 0xC0) != 0x80) return false;
                cp = (cp << 6) | (p[i + k] & 0x3F);
            }
            // overlong forms, surrogates and values past U+10FFFF are invalid
            if ((extra == 1 && cp < 0x80) || (extra == 2 && cp < 0x800) ||
                (extra == 3 && cp < 0x10000) || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF))
                return false;
            i += extra + 1;
        }
        return true;
    }
    bool bad_type(uint32_t t) {
        err = SLM_ERR_VALUE_TYPE;
        what = "InvalidValueType(" + std::to_string(t) + ")";
        return false;
    }
    // skip_scalar_or_str (loader.rs:258-282): strings are skipped unchecked
    bool skip(uint32_t type, int depth) {
        const uint8_t* p;
        switch (type) {
            case 0: case 1: case 7: return take(1, &p);
            case 2: case 3: return take(2, &p);
            case 4: case 5: case 6: return take(4, &p);
            case 10: case 11: case 12: return take(8, &p);
            case 8: {
                uint64_t n = 0;
                return read(&n) && take(n, &p);
            }
            case 9: {
                uint32_t et = 0;
                uint64_t count = 0;
                if (depth > 64) return bad_type(type);  // arrays nest at most this deep here
                if (!read(&et) || !read(&count)) return false;
                for (uint64_t i = 0; i < count; ++i)
                    if (!skip(et, depth + 1)) return false;
                return true;
            }
            default:
                return bad_type(type);
        }
    }
    bool read_value(Value* v) {  // read_value (loader.rs:284-317)
        uint32_t t = 0;
        if (!read(&t)) return false;
        v->type = (int32_t)t;
        switch (t) {
            case 0: { uint8_t x; if (!read(&x)) return false; v->i64 = x; v->u64 = x; return true; }
            case 1: { int8_t x; if (!read(&x)) return false; v->i64 = x; return true; }
            case 2: { uint16_t x; if (!read(&x)) return false; v->i64 = x; v->u64 = x; return true; }
            case 3: { int16_t x; if (!read(&x)) return false; v->i64 = x; return true; }
            case 4: { uint32_t x; if (!read(&x)) return false; v->i64 = x; v->u64 = x; return true; }
            case 5: { int32_t x; if (!read(&x)) return false; v->i64 = x; return true; }
            case 6: { float x; if (!read(&x)) return false; v->f64 = x; return true; }
            case 7: { uint8_t x; if (!read(&x)) return false; v->i64 = x != 0; return true; }
            case 8: return read_str(&v->str, &v->str_len);
            case 9: {
                uint32_t et = 0;
                if (!read(&et) || !read(&v->len)) return false;
                v->elem_type = (int32_t)et;
                v->byte_offset = pos;
                for (uint64_t i = 0; i < v->len; ++i)
                    if (!skip(et, 1)) return false;
                v->byte_len = pos - v->byte_offset;
                return true;
            }
            case 10: { uint64_t x; if (!read(&x)) return false; v->u64 = x; return true; }
            case 11: { int64_t x; if (!read(&x)) return false; v->i64 = x; return true; }
            case 12: { double x; if (!read(&x)) return false; v->f64 = x; return true; }
            default:
                return bad_type(t);
        }
    }
};

// GgmlType::{block_elements, block_bytes} (loader.rs:44-64)
bool block_shape(int32_t type, uint64_t* elems, uint64_t* bytes) {
    switch (type) {
        case SLM_GGML_F32: *elems = 1; *bytes = 4; return true;
        case SLM_GGML_F16: *elems = 1; *bytes = 2; return true;
        case SLM_GGML_Q4_0: *elems = 32; *bytes = 18; return true;
        case SLM_GGML_Q8_0: *elems = 32; *bytes = 34; return true;
        default: return false;
    }
}

// the element alignment a typed view needs (bytemuck::try_cast_slice)
uint64_t view_alignment(int32_t type) {
    switch (type) {
        case SLM_GGML_F32: return 4;
        case SLM_GGML_F16: case SLM_GGML_Q4_0: case SLM_GGML_Q8_0: return 2;
        default: return 1;
    }
}

int fail(int code, const std::string& msg) { return slm_host::fail(nullptr, code, msg); }

}  // namespace

struct slm_gguf {
    const uint8_t* base = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = kDefaultAlignment;
    uint64_t data_offset = 0;
    uint64_t n_tensors = 0;
    uint64_t n_kv = 0;
    std::unordered_map<std::string, Value> metadata;
    std::unordered_map<std::string, Tensor> tensors;
};

extern "C" {

int slm_gguf_open(const char* path, slm_gguf** out) {
    if (!out) return fail(SLM_ERR_ARG, "out is NULL");
    *out = nullptr;
    if (!path) return fail(SLM_ERR_ARG, "path is NULL");
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(SLM_ERR_IO, std::string("Io: cannot open ") + path);
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return fail(SLM_ERR_IO, std::string("Io: cannot stat ") + path);
    }
    const uint64_t size = (uint64_t)st.st_size;
    const uint8_t* base = nullptr;
    if (size > 0) {
        void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            close(fd);
            return fail(SLM_ERR_IO, std::string("Io: cannot map ") + path);
        }
        base = static_cast<const uint8_t*>(m);
    }
    close(fd);
    slm_gguf* g = new (std::nothrow) slm_gguf();
    if (!g) {
        if (size) munmap(const_cast<uint8_t*>(base), size);
        return fail(SLM_ERR_IO, "Io: out of host memory for the file handle");
    }
    g->base = base;
    g->size = size;
    auto bail = [&](int code, const std::string& msg) {
        slm_gguf_close(g);
        return fail(code, msg);
    };

    Cursor c{base, size, 0, 0, std::string()};
    uint32_t magic = 0;
    if (!c.read(&magic)) return bail(c.err, c.what);
    if (magic != kMagic) {
        char buf[32];
        snprintf(buf, sizeof buf, "InvalidMagic(0x%08x)", magic);
        return bail(SLM_ERR_MAGIC, buf);
    }
    if (!c.read(&g->version)) return bail(c.err, c.what);
    if (g->version != 2 && g->version != 3)
        return bail(SLM_ERR_VERSION, "UnsupportedVersion(" + std::to_string(g->version) + ")");
    if (!c.read(&g->n_tensors) || !c.read(&g->n_kv)) return bail(c.err, c.what);
    for (uint64_t i = 0; i < g->n_kv; ++i) {
        const char* k;
        uint64_t klen;
        Value v;
        if (!c.read_str(&k, &klen) || !c.read_value(&v)) return bail(c.err, c.what);
        g->metadata[std::string(k, klen)] = v;  // a repeated key keeps the last value
    }
    for (uint64_t i = 0; i < g->n_tensors; ++i) {
        const char* name;
        uint64_t nlen;
        Tensor t;
        uint32_t n_dims = 0, type = 0;
        if (!c.read_str(&name, &nlen) || !c.read(&n_dims)) return bail(c.err, c.what);
        if (n_dims == 0 || n_dims > 4)
            return bail(SLM_ERR_DIMS, "InvalidDimensions(" + std::to_string(n_dims) + ")");
        t.n_dims = (int32_t)n_dims;
        for (uint32_t d = 0; d < n_dims; ++d)
            if (!c.read(&t.dims[d])) return bail(c.err, c.what);
        if (!c.read(&type) || !c.read(&t.offset)) return bail(c.err, c.what);
        t.ggml_type = (int32_t)type;
        g->tensors[std::string(name, nlen)] = t;
    }
    // general.alignment through as_usize, default 32, at least 1 (loader.rs:383-389)
    uint64_t al = kDefaultAlignment;
    auto it = g->metadata.find("general.alignment");
    if (it != g->metadata.end()) {
        const Value& v = it->second;
        if (v.type == SLM_GGUF_U32 || v.type == SLM_GGUF_U64) al = v.u64;
        else if ((v.type == SLM_GGUF_I32 || v.type == SLM_GGUF_I64) && v.i64 >= 0) al = (uint64_t)v.i64;
    }
    g->alignment = al < 1 ? 1 : al;
    g->data_offset = (c.pos + g->alignment - 1) / g->alignment * g->alignment;
    *out = g;
    return SLM_OK;
}

void slm_gguf_close(slm_gguf* g) {
    if (!g) return;
    if (g->base && g->size) munmap(const_cast<uint8_t*>(g->base), g->size);
    delete g;
}

int32_t slm_gguf_version(const slm_gguf* g) { return g ? (int32_t)g->version : 0; }
int64_t slm_gguf_alignment(const slm_gguf* g) { return g ? (int64_t)g->alignment : 0; }
int64_t slm_gguf_data_offset(const slm_gguf* g) { return g ? (int64_t)g->data_offset : 0; }
int64_t slm_gguf_tensor_count(const slm_gguf* g) { return g ? (int64_t)g->n_tensors : 0; }
int64_t slm_gguf_kv_count(const slm_gguf* g) { return g ? (int64_t)g->n_kv : 0; }

int slm_gguf_get(const slm_gguf* g, const char* key, slm_gguf_value* out) {
    if (!g || !key || !out) return fail(SLM_ERR_ARG, "bad argument");
    auto it = g->metadata.find(key);
    if (it == g->metadata.end()) return fail(SLM_ERR_NOT_FOUND, std::string("no key ") + key);
    const Value& v = it->second;
    *out = slm_gguf_value{v.type, v.i64, v.u64, v.f64, v.str, v.str_len, v.elem_type,
                          v.len, v.byte_offset, v.byte_len};
    return SLM_OK;
}

// GgufValue::as_u32 (loader.rs:92-99): U32; U64 that fits; I32 >= 0
int slm_gguf_get_u32(const slm_gguf* g, const char* key, uint32_t* out) {
    slm_gguf_value v;
    int rc = slm_gguf_get(g, key, &v);
    if (rc) return rc;
    if (v.type == SLM_GGUF_U32) *out = (uint32_t)v.u64;
    else if (v.type == SLM_GGUF_U64 && v.u64 <= UINT32_MAX) *out = (uint32_t)v.u64;
    else if (v.type == SLM_GGUF_I32 && v.i64 >= 0) *out = (uint32_t)v.i64;
    else return fail(SLM_ERR_NOT_FOUND, std::string(key) + " is not a u32");
    return SLM_OK;
}

// GgufValue::as_usize (loader.rs:101-109): U32, U64, I32 >= 0, I64 >= 0
int slm_gguf_get_usize(const slm_gguf* g, const char* key, uint64_t* out) {
    slm_gguf_value v;
    int rc = slm_gguf_get(g, key, &v);
    if (rc) return rc;
    if (v.type == SLM_GGUF_U32 || v.type == SLM_GGUF_U64) *out = v.u64;
    else if ((v.type == SLM_GGUF_I32 || v.type == SLM_GGUF_I64) && v.i64 >= 0) *out = (uint64_t)v.i64;
    else return fail(SLM_ERR_NOT_FOUND, std::string(key) + " is not a usize");
    return SLM_OK;
}

// GgufValue::as_f32 (loader.rs:111-117): F32; F64 as f32
int slm_gguf_get_f32(const slm_gguf* g, const char* key, float* out) {
    slm_gguf_value v;
    int rc = slm_gguf_get(g, key, &v);
    if (rc) return rc;
    if (v.type == SLM_GGUF_F32 || v.type == SLM_GGUF_F64) *out = (float)v.f64;
    else return fail(SLM_ERR_NOT_FOUND, std::string(key) + " is not a float");
    return SLM_OK;
}

int slm_gguf_get_str(const slm_gguf* g, const char* key, const char** str, uint64_t* len) {
    slm_gguf_value v;
    int rc = slm_gguf_get(g, key, &v);
    if (rc) return rc;
    if (v.type != SLM_GGUF_STR) return fail(SLM_ERR_NOT_FOUND, std::string(key) + " is not a string");
    *str = v.str;
    *len = v.str_len;
    return SLM_OK;
}

int slm_gguf_tensor_info(const slm_gguf* g, const char* name, slm_gguf_tensor* out) {
    if (!g || !name || !out) return fail(SLM_ERR_ARG, "bad argument");
    auto it = g->tensors.find(name);
    if (it == g->tensors.end())
        return fail(SLM_ERR_NOT_FOUND, std::string("TensorNotFound(") + name + ")");
    const Tensor& t = it->second;
    uint64_t n = 1;
    for (int d = 0; d < t.n_dims; ++d) {
        if (t.dims[d] != 0 && n > UINT64_MAX / t.dims[d])
            return fail(SLM_ERR_BOUNDS, std::string("OutOfBounds(") + name + ")");
        n *= t.dims[d];
    }
    *out = slm_gguf_tensor{t.ggml_type, t.n_dims, {t.dims[0], t.dims[1], t.dims[2], t.dims[3]},
                           t.offset, n};
    return SLM_OK;
}

// raw_tensor_bytes (loader.rs:464-494), then the typed view's alignment
// (tensor_q4_0 / tensor_f32, loader.rs:496-506)
int slm_gguf_tensor_data(const slm_gguf* g, const char* name, int32_t expected_type,
                         const void** data, uint64_t* bytes) {
    slm_gguf_tensor t;
    int rc = slm_gguf_tensor_info(g, name, &t);
    if (rc) return rc;
    if (!data || !bytes) return fail(SLM_ERR_ARG, "bad argument");
    if (t.ggml_type != expected_type)
        return fail(SLM_ERR_TYPE, std::string("TypeMismatch(") + name + ": expected " +
                                      std::to_string(expected_type) + ", actual " +
                                      std::to_string(t.ggml_type) + ")");
    uint64_t be, bb;
    if (!block_shape(t.ggml_type, &be, &bb) || t.n_elements % be != 0 ||
        t.n_elements / be > UINT64_MAX / bb)
        return fail(SLM_ERR_BOUNDS, std::string("OutOfBounds(") + name + ")");
    const uint64_t len = t.n_elements / be * bb;
    if (t.offset > UINT64_MAX - g->data_offset)
        return fail(SLM_ERR_BOUNDS, std::string("OutOfBounds(") + name + ")");
    const uint64_t start = g->data_offset + t.offset;
    if (len > UINT64_MAX - start || start + len > g->size)
        return fail(SLM_ERR_BOUNDS, std::string("OutOfBounds(") + name + ")");
    if (((uintptr_t)(g->base + start)) % view_alignment(t.ggml_type) != 0)
        return fail(SLM_ERR_UNALIGNED, std::string("UnalignedTensor(") + name + ")");
    *data = g->base + start;
    *bytes = len;
    return SLM_OK;
}

// main.rs:282-305, plus {arch}.rope.freq_base
int slm_gguf_model_config(const slm_gguf* g, slm_model_config* out) {
    if (!g || !out) return fail(SLM_ERR_ARG, "bad argument");
    std::string arch = "llama";
    const char* s;
    uint64_t slen;
    if (slm_gguf_get_str(g, "general.architecture", &s, &slen) == SLM_OK) arch.assign(s, slen);
    auto usize_or = [&](const std::string& key, uint64_t dflt) {
        uint64_t v;
        return slm_gguf_get_usize(g, key.c_str(), &v) == SLM_OK ? v : dflt;
    };
    auto f32_or = [&](const std::string& key, float dflt) {
        float v;
        return slm_gguf_get_f32(g, key.c_str(), &v) == SLM_OK ? v : dflt;
    };
    const uint64_t layers = usize_or(arch + ".block_count", 2);
    const uint64_t heads = usize_or(arch + ".attention.head_count", 8);
    const uint64_t dim = usize_or(arch + ".embedding_length", 256);
    const uint64_t hidden = usize_or(arch + ".feed_forward_length", 768);
    const uint64_t kv_heads = usize_or(arch + ".attention.head_count_kv", heads);
    const uint64_t ctx = usize_or(arch + ".context_length", 64);
    for (uint64_t v : {layers, heads, dim, hidden, kv_heads, ctx})
        if (v > (uint64_t)INT32_MAX) return fail(SLM_ERR_CONFIG, "model size out of range");
    out->num_layers = (int32_t)layers;
    out->num_heads = (int32_t)heads;
    out->dim = (int32_t)dim;
    out->hidden_dim = (int32_t)hidden;
    out->num_kv_heads = (int32_t)kv_heads;
    out->max_seq_len = (int32_t)ctx;
    out->rms_eps = f32_or(arch + ".attention.layer_norm_rms_epsilon", 1e-5f);
    out->rope_theta = f32_or(arch + ".rope.freq_base", 10000.0f);
    return SLM_OK;
}

}  // extern "C"
