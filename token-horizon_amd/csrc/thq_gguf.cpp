// thq_gguf.cpp — GGUF file reader behind the C ABI (include/thq.h, "GGUF
// files"): the step the reference's loader runs before any weight reaches a
// matmul (engine/src/model.rs:526-562: gguf_file::Content::read, metadata
// lookups with to_string / to_u32, then ModelWeights::from_gguf taking each
// tensor with Content::tensor).
//
// Restates [ext] candle-core 0.11 quantized/gguf_file.rs (a crates.io
// dependency, engine/Cargo.toml:23):
//   - magic "GGUF" (either byte order of the u32), versions 1, 2, 3; v1
//     stores counts, string / array lengths and dims as u32, v2 / v3 as u64;
//   - metadata values of types 0..12, arrays of any of them (nested too),
//     bool bytes 0 / 1 only, strings with trailing NULs dropped and invalid
//     UTF-8 replaced by U+FFFD (Rust's from_utf8_lossy);
//   - tensor infos: name, n_dims, dims (reversed here to row-major, as
//     candle's Shape), ggml type id, offset;
//   - alignment from general.alignment when it is a U8/U16/U32 or a
//     non-negative I8/I16/I32, else 32; tensor data starts at the first
//     aligned position after the header;
//   - a later duplicate metadata key or tensor name replaces the earlier one
//     (candle keeps both in HashMaps);
//   - a tensor's bytes are elems / block_size * type_size at data start +
//     offset, elems a multiple of the block size.
// The file is memory-mapped read-only; tensor data is handed out as pointers
// into the mapping (no copy) and uploaded from there.
#include <fcntl.h>
#include <hip/hip_runtime.h>
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

#include "../../include/thq.h"

namespace thq {
int fail_v(int code, const char* fmt, va_list ap);  // thq_api.cpp: sets thq_last_error()
}

namespace thq_gguf_impl {

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    const int rc = thq::fail_v(code, fmt, ap);
    va_end(ap);
    return rc;
}

struct Value {
    uint32_t type = 0;
    uint64_t u = 0;  // unsigned / bool payload
    int64_t i = 0;   // signed payload
    double f = 0.0;  // f32 / f64 payload (f32 exact in a double)
    std::string s;   // string payload
    uint32_t elem_type = 0;
    uint64_t count = 0;  // array length
};

struct Tensor {
    std::string name;
    uint32_t type = 0;
    uint32_t n_dims = 0;
    uint64_t dims[4] = {0, 0, 0, 0};  // row-major: dims[0] outermost
    uint64_t rel_offset = 0;
};

// ggml type table: block size and bytes per block ([ext] candle-core 0.11
// GgmlDType::{from_u32, block_size, type_size}); 0 = unknown id
struct TypeInfo {
    uint32_t bs, ts;
};
TypeInfo type_info(uint32_t t) {
    switch (t) {
        case 0: return {1, 4};      // F32
        case 1: return {1, 2};      // F16
        case 2: return {32, 18};    // Q4_0
        case 3: return {32, 20};    // Q4_1
        case 6: return {32, 22};    // Q5_0
        case 7: return {32, 24};    // Q5_1
        case 8: return {32, 34};    // Q8_0
        case 9: return {32, 36};    // Q8_1
        case 10: return {256, 84};  // Q2_K
        case 11: return {256, 110}; // Q3_K
        case 12: return {256, 144}; // Q4_K
        case 13: return {256, 176}; // Q5_K
        case 14: return {256, 210}; // Q6_K
        case 15: return {256, 292}; // Q8_K
        case 30: return {1, 2};     // BF16
        default: return {0, 0};
    }
}

// Rust String::from_utf8_lossy: each maximal prefix of a well-formed
// sequence that cannot be completed (or a lone bad byte) becomes U+FFFD
std::string utf8_lossy(const uint8_t* p, size_t n) {
    std::string out;
    out.reserve(n);
    size_t i = 0;
    while (i < n) {
        const uint8_t b = p[i];
        if (b < 0x80) {
            out.push_back((char)b);
            ++i;
            continue;
        }
        int need;
        uint8_t lo = 0x80, hi = 0xBF;  // bounds of the second byte
        if (b >= 0xC2 && b <= 0xDF) {
            need = 1;
        } else if (b >= 0xE0 && b <= 0xEF) {
            need = 2;
            if (b == 0xE0) lo = 0xA0;
            if (b == 0xED) hi = 0x9F;
        } else if (b >= 0xF0 && b <= 0xF4) {
            need = 3;
            if (b == 0xF0) lo = 0x90;
            if (b == 0xF4) hi = 0x8F;
        } else {
            out += "\xEF\xBF\xBD";
            ++i;
            continue;
        }
        size_t j = i + 1;
        bool ok = true;
        for (int k = 0; k < need; ++k, ++j) {
            const uint8_t l = k == 0 ? lo : 0x80, h = k == 0 ? hi : 0xBF;
            if (j >= n || p[j] < l || p[j] > h) {
                ok = false;
                break;
            }
        }
        if (ok) {
            out.append(reinterpret_cast<const char*>(p + i), j - i);
        } else {
            out += "\xEF\xBF\xBD";
        }
        i = j;
    }
    return out;
}

struct Reader {
    const uint8_t* p;
    size_t n, pos = 0;
    bool v1 = false;
    int err = THQ_OK;

    bool take(void* dst, size_t k) {
        if (err) return false;
        if (k > n - pos) {
            err = fail(THQ_EFORMAT, "GGUF: unexpected end of file at byte %zu (want %zu more)", pos, k);
            return false;
        }
        std::memcpy(dst, p + pos, k);
        pos += k;
        return true;
    }
    template <typename T>
    T rd() {
        T v{};
        take(&v, sizeof(T));
        return v;
    }
    uint64_t len() { return v1 ? rd<uint32_t>() : rd<uint64_t>(); }
    std::string str() {
        const uint64_t l = len();
        if (err) return {};
        if (l > n - pos) {
            err = fail(THQ_EFORMAT, "GGUF: string of %llu bytes runs past the end of the file", (unsigned long long)l);
            return {};
        }
        size_t m = (size_t)l;
        const uint8_t* s = p + pos;
        pos += m;
        while (m && s[m - 1] == 0) --m;
        return utf8_lossy(s, m);
    }
    // a value of type t; arrays keep their length and element type, their
    // elements are validated and skipped
    void value(uint32_t t, Value& v, int depth) {
        v.type = t;
        switch (t) {
            case THQ_GGUF_U8: v.u = rd<uint8_t>(); break;
            case THQ_GGUF_I8: v.i = rd<int8_t>(); break;
            case THQ_GGUF_U16: v.u = rd<uint16_t>(); break;
            case THQ_GGUF_I16: v.i = rd<int16_t>(); break;
            case THQ_GGUF_U32: v.u = rd<uint32_t>(); break;
            case THQ_GGUF_I32: v.i = rd<int32_t>(); break;
            case THQ_GGUF_F32: v.f = rd<float>(); break;
            case THQ_GGUF_BOOL: {
                const uint8_t b = rd<uint8_t>();
                if (!err && b > 1) err = fail(THQ_EFORMAT, "GGUF: unexpected bool value %u", b);
                v.u = b;
                break;
            }
            case THQ_GGUF_STRING: v.s = str(); break;
            case THQ_GGUF_ARRAY: {
                if (depth > 64) {
                    err = fail(THQ_EFORMAT, "GGUF: arrays nested too deeply");
                    return;
                }
                v.elem_type = rd<uint32_t>();
                v.count = len();
                Value e;
                for (uint64_t k = 0; k < v.count && !err; ++k) value(v.elem_type, e, depth + 1);
                break;
            }
            case THQ_GGUF_U64: v.u = rd<uint64_t>(); break;
            case THQ_GGUF_I64: v.i = rd<int64_t>(); break;
            case THQ_GGUF_F64: v.f = rd<double>(); break;
            default:
                if (!err) err = fail(THQ_EFORMAT, "GGUF: unknown value type %u", t);
        }
    }
};

}  // namespace thq_gguf_impl

using namespace thq_gguf_impl;

struct thq_gguf {
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t data_start = 0;
    std::vector<std::pair<std::string, Value>> kv;  // unique keys, file order of first appearance
    std::unordered_map<std::string, size_t> kv_index;
    std::vector<Tensor> tensors;                     // unique names, file order of first appearance
    std::unordered_map<std::string, size_t> t_index;
};

namespace {

void release(thq_gguf* g) {
    if (g->map) munmap(const_cast<uint8_t*>(g->map), g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

const Value* find_kv(const thq_gguf* g, const char* key) {
    auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? nullptr : &g->kv[it->second].second;
}

// element count; false when it overflows 64 bits
bool elems(const Tensor& t, uint64_t& e) {
    e = 1;
    for (uint32_t j = 0; j < t.n_dims; ++j)
        if (__builtin_mul_overflow(e, t.dims[j], &e)) return false;
    return true;
}

int parse(thq_gguf* g) {
    Reader r{g->map, g->size};
    const uint32_t magic = r.rd<uint32_t>();
    if (r.err) return r.err;
    if (magic != 0x46554747u && magic != 0x47475546u) return fail(THQ_EFORMAT, "GGUF: unknown magic 0x%08x", magic);
    g->version = r.rd<uint32_t>();
    if (r.err) return r.err;
    if (g->version < 1 || g->version > 3) return fail(THQ_EFORMAT, "GGUF: unsupported version %u", g->version);
    r.v1 = g->version == 1;
    const uint64_t n_tensors = r.len();
    const uint64_t n_kv = r.len();
    if (r.err) return r.err;
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = r.str();
        const uint32_t t = r.rd<uint32_t>();
        Value v;
        r.value(t, v, 0);
        if (r.err) return r.err;
        auto it = g->kv_index.find(key);
        if (it != g->kv_index.end()) {
            g->kv[it->second].second = std::move(v);
        } else {
            g->kv_index.emplace(key, g->kv.size());
            g->kv.emplace_back(std::move(key), std::move(v));
        }
    }
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Tensor t;
        t.name = r.str();
        t.n_dims = r.rd<uint32_t>();
        if (r.err) return r.err;
        if (t.n_dims > 4) return fail(THQ_EFORMAT, "GGUF: tensor %s has %u dims (at most 4)", t.name.c_str(), t.n_dims);
        uint64_t d[4] = {0, 0, 0, 0};
        for (uint32_t j = 0; j < t.n_dims; ++j) d[j] = r.v1 ? r.rd<uint32_t>() : r.rd<uint64_t>();
        for (uint32_t j = 0; j < t.n_dims; ++j) t.dims[j] = d[t.n_dims - 1 - j];  // candle reverses ne
        t.type = r.rd<uint32_t>();
        t.rel_offset = r.rd<uint64_t>();
        if (r.err) return r.err;
        if (!type_info(t.type).bs) return fail(THQ_EFORMAT, "GGUF: unknown dtype %u for tensor %s", t.type, t.name.c_str());
        uint64_t e, nb;
        if (!elems(t, e)) return fail(THQ_EFORMAT, "GGUF: tensor %s has more than 2^64 elements", t.name.c_str());
        const TypeInfo ti = type_info(t.type);
        if (__builtin_mul_overflow(e / ti.bs, (uint64_t)ti.ts, &nb))
            return fail(THQ_EFORMAT, "GGUF: tensor %s has more than 2^64 bytes", t.name.c_str());
        auto it = g->t_index.find(t.name);
        if (it != g->t_index.end()) {
            g->tensors[it->second] = t;
        } else {
            g->t_index.emplace(t.name, g->tensors.size());
            g->tensors.push_back(t);
        }
    }
    uint64_t align = 32;
    if (const Value* a = find_kv(g, "general.alignment")) {
        switch (a->type) {
            case THQ_GGUF_U8: case THQ_GGUF_U16: case THQ_GGUF_U32: align = a->u; break;
            case THQ_GGUF_I8: case THQ_GGUF_I16: case THQ_GGUF_I32:
                if (a->i >= 0) align = (uint64_t)a->i;
                break;
            default: break;
        }
    }
    if (align == 0) return fail(THQ_EFORMAT, "GGUF: general.alignment is 0");
    g->data_start = (r.pos + align - 1) / align * align;
    return THQ_OK;
}

}  // namespace

extern "C" {

int thq_gguf_open(const char* path, thq_gguf** out) {
    if (!path || !out) return fail(THQ_EINVAL, "null argument");
    *out = nullptr;
    thq_gguf* g = new (std::nothrow) thq_gguf();
    if (!g) return fail(THQ_ENOMEM, "host allocation failed");
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (g->fd < 0) {
        release(g);
        return fail(THQ_EIO, "cannot open %s: %s", path, strerror(errno));
    }
    struct stat st;
    if (fstat(g->fd, &st) != 0) {
        release(g);
        return fail(THQ_EIO, "cannot stat %s: %s", path, strerror(errno));
    }
    g->size = (size_t)st.st_size;
    if (g->size) {
        void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
        if (m == MAP_FAILED) {
            release(g);
            return fail(THQ_EIO, "cannot map %s: %s", path, strerror(errno));
        }
        g->map = static_cast<const uint8_t*>(m);
    }
    int rc = parse(g);
    if (rc) {
        release(g);
        return rc;
    }
    *out = g;
    return THQ_OK;
}

void thq_gguf_close(thq_gguf* g) {
    if (g) release(g);
}

int thq_gguf_version(const thq_gguf* g, uint32_t* version) {
    if (!g || !version) return fail(THQ_EINVAL, "null argument");
    *version = g->version;
    return THQ_OK;
}

int64_t thq_gguf_tensor_count(const thq_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }

int64_t thq_gguf_metadata_count(const thq_gguf* g) { return g ? (int64_t)g->kv.size() : -1; }

int64_t thq_gguf_find_tensor(const thq_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->t_index.find(name);
    return it == g->t_index.end() ? -1 : (int64_t)it->second;
}

int thq_gguf_tensor_info(const thq_gguf* g, int64_t i, const char** name, uint32_t* ggml_type, uint32_t* n_dims,
                         uint64_t* dims, uint64_t* offset, uint64_t* nbytes) {
    if (!g) return fail(THQ_EINVAL, "null file");
    if (i < 0 || i >= (int64_t)g->tensors.size()) return fail(THQ_EINVAL, "tensor index %lld out of range", (long long)i);
    const Tensor& t = g->tensors[(size_t)i];
    const TypeInfo ti = type_info(t.type);
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = t.type;
    if (n_dims) *n_dims = t.n_dims;
    if (dims)
        for (int j = 0; j < 4; ++j) dims[j] = t.dims[j];
    uint64_t e = 0;
    elems(t, e);  // checked at open
    if (offset) *offset = g->data_start + t.rel_offset;
    if (nbytes) *nbytes = e / ti.bs * ti.ts;
    return THQ_OK;
}

int thq_gguf_tensor_data(const thq_gguf* g, int64_t i, const void** data, uint64_t* nbytes) {
    if (!g || !data) return fail(THQ_EINVAL, "null argument");
    if (i < 0 || i >= (int64_t)g->tensors.size()) return fail(THQ_EINVAL, "tensor index %lld out of range", (long long)i);
    const Tensor& t = g->tensors[(size_t)i];
    const TypeInfo ti = type_info(t.type);
    uint64_t e = 0;
    elems(t, e);  // checked at open
    if (e % ti.bs)
        return fail(THQ_ESHAPE, "GGUF: tensor %s: the number of elements %llu is not divisible by the block size %u",
                    t.name.c_str(), (unsigned long long)e, ti.bs);
    const uint64_t nb = e / ti.bs * ti.ts, off = g->data_start + t.rel_offset;
    if (off < g->data_start || off > g->size || nb > g->size - off)
        return fail(THQ_EFORMAT, "GGUF: tensor %s data [%llu, +%llu) lies past the end of the file (%zu bytes)",
                    t.name.c_str(), (unsigned long long)off, (unsigned long long)nb, g->size);
    *data = g->map + off;
    if (nbytes) *nbytes = nb;
    return THQ_OK;
}

int thq_gguf_metadata_key(const thq_gguf* g, int64_t i, const char** key, uint32_t* value_type) {
    if (!g) return fail(THQ_EINVAL, "null file");
    if (i < 0 || i >= (int64_t)g->kv.size()) return fail(THQ_EINVAL, "metadata index %lld out of range", (long long)i);
    if (key) *key = g->kv[(size_t)i].first.c_str();
    if (value_type) *value_type = g->kv[(size_t)i].second.type;
    return THQ_OK;
}

int thq_gguf_metadata_u32(const thq_gguf* g, const char* key, uint32_t* out) {
    if (!g || !key || !out) return fail(THQ_EINVAL, "null argument");
    const Value* v = find_kv(g, key);
    if (!v) return fail(THQ_ENOTFOUND, "GGUF: no metadata key %s", key);
    if (v->type != THQ_GGUF_U32) return fail(THQ_EDTYPE, "GGUF: %s is not a u32 (type %u)", key, v->type);
    *out = (uint32_t)v->u;
    return THQ_OK;
}

int thq_gguf_metadata_f32(const thq_gguf* g, const char* key, float* out) {
    if (!g || !key || !out) return fail(THQ_EINVAL, "null argument");
    const Value* v = find_kv(g, key);
    if (!v) return fail(THQ_ENOTFOUND, "GGUF: no metadata key %s", key);
    if (v->type != THQ_GGUF_F32) return fail(THQ_EDTYPE, "GGUF: %s is not a f32 (type %u)", key, v->type);
    *out = (float)v->f;
    return THQ_OK;
}

int thq_gguf_metadata_str(const thq_gguf* g, const char* key, const char** out, uint64_t* len) {
    if (!g || !key || !out) return fail(THQ_EINVAL, "null argument");
    const Value* v = find_kv(g, key);
    if (!v) return fail(THQ_ENOTFOUND, "GGUF: no metadata key %s", key);
    if (v->type != THQ_GGUF_STRING) return fail(THQ_EDTYPE, "GGUF: %s is not a string (type %u)", key, v->type);
    *out = v->s.c_str();
    if (len) *len = v->s.size();
    return THQ_OK;
}

int thq_gguf_metadata_array(const thq_gguf* g, const char* key, uint32_t* elem_type, uint64_t* count) {
    if (!g || !key) return fail(THQ_EINVAL, "null argument");
    const Value* v = find_kv(g, key);
    if (!v) return fail(THQ_ENOTFOUND, "GGUF: no metadata key %s", key);
    if (v->type != THQ_GGUF_ARRAY) return fail(THQ_EDTYPE, "GGUF: %s is not an array (type %u)", key, v->type);
    if (elem_type) *elem_type = v->elem_type;
    if (count) *count = v->count;
    return THQ_OK;
}

int thq_weight_from_gguf(thq_ctx* ctx, const thq_gguf* g, const char* name, thq_weight** out) {
    if (!ctx || !g || !name || !out) return fail(THQ_EINVAL, "null argument");
    const int64_t i = thq_gguf_find_tensor(g, name);
    if (i < 0) return fail(THQ_ENOTFOUND, "GGUF: cannot find tensor info for %s", name);
    const Tensor& t = g->tensors[(size_t)i];
    if (t.type != THQ_Q8_0 && t.type != THQ_Q4_K && t.type != THQ_Q6_K)
        return fail(THQ_EDTYPE, "GGUF: tensor %s has ggml type %u (the library takes Q8_0, Q4_K, Q6_K)", name, t.type);
    if (t.n_dims != 2) return fail(THQ_ESHAPE, "GGUF: tensor %s has %u dims (a weight has 2)", name, t.n_dims);
    const void* data = nullptr;
    int rc = thq_gguf_tensor_data(g, i, &data, nullptr);
    if (rc) return rc;
    return thq_weight_upload(ctx, (thq_dtype)t.type, data, (int64_t)t.dims[0], (int64_t)t.dims[1], out);
}

}  // extern "C"
