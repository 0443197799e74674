// ft_gguf.cpp -- local GGUF v2/v3 model files: header, metadata, tensor
// table and memory-mapped tensor data (the counterpart of ft-gguf's Gguf,
// ft-gguf/src/lib.rs:141-206), the small-tensor dequantiser and router fold
// of ft-model (lib.rs:128-151, :506-514), and the expert-bank loader that
// moves a file's q4_0 expert tensors into resident device banks (lib.rs:
// 570-609, repacked on the device instead of on the host).
//
// The file is mapped read-only and parsed once at open; every read of the
// header is bounds-checked, so a truncated or malformed file is an
// FT_HIP_E_FORMAT error with the offending offset in ft_hip_last_error().
#include "ft_runtime.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

constexpr uint32_t GT_U8 = 0, GT_I8 = 1, GT_U16 = 2, GT_I16 = 3, GT_U32 = 4, GT_I32 = 5, GT_F32 = 6, GT_BOOL = 7,
                   GT_STR = 8, GT_ARR = 9, GT_U64 = 10, GT_I64 = 11, GT_F64 = 12;

struct Value {
    uint32_t type = 0;
    uint64_t u = 0;   // unsigned ints and bool
    int64_t i = 0;    // signed ints
    double f = 0.0;   // f64 (f32 in f32v)
    float f32v = 0.0f;
    std::string s;
    uint32_t elem_type = 0;
    std::vector<Value> arr;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;  // ne[0] first (the contiguous dimension)
    uint32_t ggml_type = 0;
    uint64_t offset = 0;         // within the data section
    uint64_t nbytes = 0;
};

// (elements per block, bytes per block) of the ggml types a model file may
// hold (ft-gguf/src/lib.rs:51-70); others fail the open, as there.
bool block_layout(uint32_t t, uint64_t& be, uint64_t& bb) {
    switch (t) {
        case 0: be = 1; bb = 4; return true;      // f32
        case 1: be = 1; bb = 2; return true;      // f16
        case 2: be = 32; bb = 18; return true;    // q4_0
        case 3: be = 32; bb = 20; return true;    // q4_1
        case 6: be = 32; bb = 22; return true;    // q5_0
        case 7: be = 32; bb = 24; return true;    // q5_1
        case 8: be = 32; bb = 34; return true;    // q8_0
        case 10: be = 256; bb = 84; return true;  // q2_k
        case 11: be = 256; bb = 110; return true; // q3_k
        case 12: be = 256; bb = 144; return true; // q4_k
        case 13: be = 256; bb = 176; return true; // q5_k
        case 14: be = 256; bb = 210; return true; // q6_k
        case 16: be = 256; bb = 66; return true;  // iq2_xxs
        case 30: be = 1; bb = 2; return true;     // bf16
        default: return false;
    }
}

struct Cursor {
    const uint8_t* p;
    uint64_t n, pos = 0;
    bool take(uint64_t k, const uint8_t*& out) {
        if (k > n - pos) return false;
        out = p + pos;
        pos += k;
        return true;
    }
    template <class T>
    bool get(T& v) {
        const uint8_t* q;
        if (!take(sizeof(T), q)) return false;
        std::memcpy(&v, q, sizeof(T));  // GGUF is little-endian, as is the host
        return true;
    }
    bool str(std::string& s) {
        uint64_t len;
        const uint8_t* q;
        if (!get(len) || !take(len, q)) return false;
        s.assign(reinterpret_cast<const char*>(q), len);
        return true;
    }
};

bool read_value(Cursor& c, uint32_t type, Value& v, int depth) {
    v.type = type;
    switch (type) {
        case GT_U8: { uint8_t x; if (!c.get(x)) return false; v.u = x; return true; }
        case GT_I8: { int8_t x; if (!c.get(x)) return false; v.i = x; return true; }
        case GT_U16: { uint16_t x; if (!c.get(x)) return false; v.u = x; return true; }
        case GT_I16: { int16_t x; if (!c.get(x)) return false; v.i = x; return true; }
        case GT_U32: { uint32_t x; if (!c.get(x)) return false; v.u = x; return true; }
        case GT_I32: { int32_t x; if (!c.get(x)) return false; v.i = x; return true; }
        case GT_F32: { float x; if (!c.get(x)) return false; v.f32v = x; v.f = x; return true; }
        case GT_BOOL: { uint8_t x; if (!c.get(x)) return false; v.u = x != 0; return true; }
        case GT_STR: return c.str(v.s);
        case GT_U64: return c.get(v.u);
        case GT_I64: return c.get(v.i);
        case GT_F64: return c.get(v.f);
        case GT_ARR: {
            uint64_t n;
            if (depth > 4 || !c.get(v.elem_type) || !c.get(n)) return false;
            if (n > c.n - c.pos) return false;  // every element takes at least one byte
            v.arr.resize(n);
            for (uint64_t k = 0; k < n; ++k)
                if (!read_value(c, v.elem_type, v.arr[k], depth + 1)) return false;
            return true;
        }
        default: return false;
    }
}

// as_u64 of ft-gguf's Value (lib.rs:29-41): unsigned ints, and signed ints
// that are not negative.
bool as_u64(const Value& v, uint64_t& out) {
    switch (v.type) {
        case GT_U8: case GT_U16: case GT_U32: case GT_U64: out = v.u; return true;
        case GT_I8: case GT_I16: case GT_I32: case GT_I64:
            if (v.i < 0) return false;
            out = (uint64_t)v.i;
            return true;
        default: return false;
    }
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31, ex = (h >> 10) & 0x1F, man = h & 0x3FF;
    uint32_t bits;
    if (ex == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: exact as f32
            const float v = std::ldexp((float)man, -24);
            std::memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (ex == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

}  // namespace

struct ft_gguf {
    void* map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t data_start = 0;
    std::vector<std::pair<std::string, Value>> kv;  // file order
    std::unordered_map<std::string, size_t> kv_index;
    std::vector<Tensor> tensors;                    // file order
    std::unordered_map<std::string, size_t> t_index;
};

static int parse(ft_gguf* g) {
    Cursor c{static_cast<const uint8_t*>(g->map), g->size};
    const uint8_t* magic;
    if (!c.take(4, magic) || std::memcmp(magic, "GGUF", 4) != 0) return fail(FT_HIP_E_FORMAT, "gguf: not a GGUF file");
    if (!c.get(g->version)) return fail(FT_HIP_E_FORMAT, "gguf: truncated header");
    if (g->version < 2 || g->version > 3)
        return fail(FT_HIP_E_FORMAT, "gguf: unsupported GGUF version %u", g->version);
    uint64_t n_tensors, n_kv;
    if (!c.get(n_tensors) || !c.get(n_kv)) return fail(FT_HIP_E_FORMAT, "gguf: truncated header");
    if (n_kv > g->size || n_tensors > g->size) return fail(FT_HIP_E_FORMAT, "gguf: implausible counts");
    g->kv.reserve(n_kv);
    for (uint64_t k = 0; k < n_kv; ++k) {
        std::string key;
        uint32_t type;
        Value v;
        if (!c.str(key) || !c.get(type)) return fail(FT_HIP_E_FORMAT, "gguf: truncated metadata at %llu", (unsigned long long)c.pos);
        if (type > GT_F64) return fail(FT_HIP_E_FORMAT, "gguf: unknown value type %u (key %s)", type, key.c_str());
        if (!read_value(c, type, v, 0))
            return fail(FT_HIP_E_FORMAT, "gguf: bad or truncated value of %s at %llu", key.c_str(), (unsigned long long)c.pos);
        g->kv_index[key] = g->kv.size();
        g->kv.emplace_back(std::move(key), std::move(v));
    }
    g->tensors.reserve(n_tensors);
    for (uint64_t k = 0; k < n_tensors; ++k) {
        Tensor t;
        uint32_t nd;
        if (!c.str(t.name) || !c.get(nd)) return fail(FT_HIP_E_FORMAT, "gguf: truncated tensor table at %llu", (unsigned long long)c.pos);
        if (nd == 0 || nd > 8) return fail(FT_HIP_E_FORMAT, "gguf: tensor %s has %u dims", t.name.c_str(), nd);
        t.dims.resize(nd);
        uint64_t nel = 1;
        for (uint32_t d = 0; d < nd; ++d) {
            if (!c.get(t.dims[d])) return fail(FT_HIP_E_FORMAT, "gguf: truncated tensor table at %llu", (unsigned long long)c.pos);
            if (t.dims[d] && nel > UINT64_MAX / t.dims[d]) return fail(FT_HIP_E_FORMAT, "gguf: tensor %s too large", t.name.c_str());
            nel *= t.dims[d];
        }
        if (!c.get(t.ggml_type) || !c.get(t.offset)) return fail(FT_HIP_E_FORMAT, "gguf: truncated tensor table at %llu", (unsigned long long)c.pos);
        uint64_t be, bb;
        if (!block_layout(t.ggml_type, be, bb)) return fail(FT_HIP_E_FORMAT, "gguf: unsupported ggml type %u (tensor %s)", t.ggml_type, t.name.c_str());
        if (nel % be) return fail(FT_HIP_E_FORMAT, "gguf: tensor %s: %llu elements not divisible by block %llu", t.name.c_str(), (unsigned long long)nel, (unsigned long long)be);
        if (nel / be > UINT64_MAX / bb) return fail(FT_HIP_E_FORMAT, "gguf: tensor %s too large", t.name.c_str());
        t.nbytes = nel / be * bb;
        g->t_index[t.name] = g->tensors.size();
        g->tensors.push_back(std::move(t));
    }
    uint64_t align = 32;
    auto it = g->kv_index.find("general.alignment");
    if (it != g->kv_index.end()) {
        if (!as_u64(g->kv[it->second].second, align) || align == 0)
            return fail(FT_HIP_E_FORMAT, "gguf: general.alignment is not a positive integer");
    }
    if (align - 1 > UINT64_MAX - c.pos) return fail(FT_HIP_E_FORMAT, "gguf: general.alignment %llu too large", (unsigned long long)align);
    g->data_start = (c.pos + align - 1) / align * align;
    return FT_HIP_OK;
}

extern "C" int ft_gguf_open(const char* path, ft_gguf** out) {
    clear_error();
    if (!path || !out) return fail(FT_HIP_E_INVALID, "gguf_open: null argument");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) return fail(FT_HIP_E_IO, "gguf_open: cannot open %s: %s", path, std::strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        ::close(fd);
        return fail(FT_HIP_E_FORMAT, "gguf_open: %s is empty or unreadable", path);
    }
    void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) return fail(FT_HIP_E_IO, "gguf_open: mmap of %s failed: %s", path, std::strerror(errno));
    ft_gguf* g = new (std::nothrow) ft_gguf;
    if (!g) {
        munmap(m, (size_t)st.st_size);
        return fail(FT_HIP_E_INVALID, "gguf_open: out of host memory");
    }
    g->map = m;
    g->size = (uint64_t)st.st_size;
    int rc;
    try {
        rc = parse(g);
    } catch (const std::bad_alloc&) {
        rc = fail(FT_HIP_E_FORMAT, "gguf_open: metadata of %s does not fit in host memory", path);
    }
    if (rc != FT_HIP_OK) {
        munmap(g->map, g->size);
        delete g;
        return rc;
    }
    *out = g;
    return FT_HIP_OK;
}

extern "C" int ft_gguf_close(ft_gguf* g) {
    clear_error();
    if (!g) return FT_HIP_OK;
    munmap(g->map, g->size);
    delete g;
    return FT_HIP_OK;
}

extern "C" uint32_t ft_gguf_version(const ft_gguf* g) { return g ? g->version : 0; }
extern "C" uint64_t ft_gguf_data_start(const ft_gguf* g) { return g ? g->data_start : 0; }
extern "C" int64_t ft_gguf_n_kv(const ft_gguf* g) { return g ? (int64_t)g->kv.size() : -1; }
extern "C" int64_t ft_gguf_n_tensors(const ft_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }

static const Value* find_kv(const ft_gguf* g, const char* key, const char* nm, int& rc) {
    clear_error();
    if (!g || !key) {
        rc = fail(FT_HIP_E_INVALID, "%s: null argument", nm);
        return nullptr;
    }
    auto it = g->kv_index.find(key);
    if (it == g->kv_index.end()) {
        rc = fail(FT_HIP_E_NOT_FOUND, "%s: no metadata key %s", nm, key);
        return nullptr;
    }
    rc = FT_HIP_OK;
    return &g->kv[it->second].second;
}

extern "C" int ft_gguf_kv_key(const ft_gguf* g, int64_t i, const char** key, uint32_t* value_type) {
    clear_error();
    if (!g || !key || !value_type) return fail(FT_HIP_E_INVALID, "gguf_kv_key: null argument");
    if (i < 0 || i >= (int64_t)g->kv.size()) return fail(FT_HIP_E_NOT_FOUND, "gguf_kv_key: index %lld out of range", (long long)i);
    *key = g->kv[(size_t)i].first.c_str();
    *value_type = g->kv[(size_t)i].second.type;
    return FT_HIP_OK;
}

extern "C" int ft_gguf_meta_type(const ft_gguf* g, const char* key, uint32_t* value_type) {
    int rc;
    const Value* v = find_kv(g, key, "gguf_meta_type", rc);
    if (!v) return rc;
    if (!value_type) return fail(FT_HIP_E_INVALID, "gguf_meta_type: null value_type");
    *value_type = v->type;
    return FT_HIP_OK;
}

extern "C" int ft_gguf_meta_u64(const ft_gguf* g, const char* key, uint64_t* out) {
    int rc;
    const Value* v = find_kv(g, key, "gguf_meta_u64", rc);
    if (!v) return rc;
    if (!out) return fail(FT_HIP_E_INVALID, "gguf_meta_u64: null out");
    if (!as_u64(*v, *out)) return fail(FT_HIP_E_FORMAT, "gguf_meta_u64: %s is not a non-negative integer", key);
    return FT_HIP_OK;
}

extern "C" int ft_gguf_meta_f32(const ft_gguf* g, const char* key, float* out) {
    int rc;
    const Value* v = find_kv(g, key, "gguf_meta_f32", rc);
    if (!v) return rc;
    if (!out) return fail(FT_HIP_E_INVALID, "gguf_meta_f32: null out");
    if (v->type != GT_F32) return fail(FT_HIP_E_FORMAT, "gguf_meta_f32: %s is not f32", key);
    *out = v->f32v;
    return FT_HIP_OK;
}

extern "C" int ft_gguf_meta_str(const ft_gguf* g, const char* key, const char** s, uint64_t* len) {
    int rc;
    const Value* v = find_kv(g, key, "gguf_meta_str", rc);
    if (!v) return rc;
    if (!s || !len) return fail(FT_HIP_E_INVALID, "gguf_meta_str: null out");
    if (v->type != GT_STR) return fail(FT_HIP_E_FORMAT, "gguf_meta_str: %s is not a string", key);
    *s = v->s.data();
    *len = v->s.size();
    return FT_HIP_OK;
}

extern "C" int ft_gguf_meta_array(const ft_gguf* g, const char* key, uint32_t* elem_type, uint64_t* n) {
    int rc;
    const Value* v = find_kv(g, key, "gguf_meta_array", rc);
    if (!v) return rc;
    if (!elem_type || !n) return fail(FT_HIP_E_INVALID, "gguf_meta_array: null out");
    if (v->type != GT_ARR) return fail(FT_HIP_E_FORMAT, "gguf_meta_array: %s is not an array", key);
    *elem_type = v->elem_type;
    *n = v->arr.size();
    return FT_HIP_OK;
}

static const Value* array_elem(const ft_gguf* g, const char* key, uint64_t i, const char* nm, int& rc) {
    const Value* v = find_kv(g, key, nm, rc);
    if (!v) return nullptr;
    if (v->type != GT_ARR) {
        rc = fail(FT_HIP_E_FORMAT, "%s: %s is not an array", nm, key);
        return nullptr;
    }
    if (i >= v->arr.size()) {
        rc = fail(FT_HIP_E_NOT_FOUND, "%s: %s[%llu] out of range", nm, key, (unsigned long long)i);
        return nullptr;
    }
    return &v->arr[i];
}

extern "C" int ft_gguf_meta_array_u64(const ft_gguf* g, const char* key, uint64_t i, uint64_t* out) {
    int rc;
    const Value* e = array_elem(g, key, i, "gguf_meta_array_u64", rc);
    if (!e) return rc;
    if (!out) return fail(FT_HIP_E_INVALID, "gguf_meta_array_u64: null out");
    if (!as_u64(*e, *out)) return fail(FT_HIP_E_FORMAT, "gguf_meta_array_u64: %s[%llu] is not a non-negative integer", key, (unsigned long long)i);
    return FT_HIP_OK;
}

extern "C" int ft_gguf_meta_array_bool(const ft_gguf* g, const char* key, uint64_t i, int* out) {
    int rc;
    const Value* e = array_elem(g, key, i, "gguf_meta_array_bool", rc);
    if (!e) return rc;
    if (!out) return fail(FT_HIP_E_INVALID, "gguf_meta_array_bool: null out");
    *out = e->type == GT_BOOL && e->u != 0;  // ft-model's arr_b: Bool(true) only (lib.rs:70-78)
    return FT_HIP_OK;
}

extern "C" int ft_gguf_meta_array_str(const ft_gguf* g, const char* key, uint64_t i, const char** s, uint64_t* len) {
    int rc;
    const Value* e = array_elem(g, key, i, "gguf_meta_array_str", rc);
    if (!e) return rc;
    if (!s || !len) return fail(FT_HIP_E_INVALID, "gguf_meta_array_str: null out");
    if (e->type != GT_STR) return fail(FT_HIP_E_FORMAT, "gguf_meta_array_str: %s[%llu] is not a string", key, (unsigned long long)i);
    *s = e->s.data();
    *len = e->s.size();
    return FT_HIP_OK;
}

extern "C" int ft_gguf_tensor_name(const ft_gguf* g, int64_t i, const char** name) {
    clear_error();
    if (!g || !name) return fail(FT_HIP_E_INVALID, "gguf_tensor_name: null argument");
    if (i < 0 || i >= (int64_t)g->tensors.size())
        return fail(FT_HIP_E_NOT_FOUND, "gguf_tensor_name: index %lld out of range", (long long)i);
    *name = g->tensors[(size_t)i].name.c_str();
    return FT_HIP_OK;
}

static const Tensor* find_tensor(const ft_gguf* g, const char* name, const char* nm, int& rc) {
    clear_error();
    if (!g || !name) {
        rc = fail(FT_HIP_E_INVALID, "%s: null argument", nm);
        return nullptr;
    }
    auto it = g->t_index.find(name);
    if (it == g->t_index.end()) {
        rc = fail(FT_HIP_E_NOT_FOUND, "%s: tensor %s not found", nm, name);
        return nullptr;
    }
    rc = FT_HIP_OK;
    return &g->tensors[it->second];
}

extern "C" int ft_gguf_tensor_info(const ft_gguf* g, const char* name, uint32_t* n_dims, uint64_t* dims,
                                   uint32_t* ggml_type, uint64_t* offset, uint64_t* nbytes) {
    int rc;
    const Tensor* t = find_tensor(g, name, "gguf_tensor_info", rc);
    if (!t) return rc;
    if (n_dims) *n_dims = (uint32_t)t->dims.size();
    if (dims)
        for (size_t d = 0; d < 8; ++d) dims[d] = d < t->dims.size() ? t->dims[d] : 1;
    if (ggml_type) *ggml_type = t->ggml_type;
    if (offset) *offset = t->offset;
    if (nbytes) *nbytes = t->nbytes;
    return FT_HIP_OK;
}

extern "C" int ft_gguf_tensor_data(const ft_gguf* g, const char* name, const void** data, uint64_t* nbytes) {
    int rc;
    const Tensor* t = find_tensor(g, name, "gguf_tensor_data", rc);
    if (!t) return rc;
    if (!data) return fail(FT_HIP_E_INVALID, "gguf_tensor_data: null data");
    const uint64_t a = g->data_start + t->offset;
    if (t->offset > g->size || a > g->size || t->nbytes > g->size - a)
        return fail(FT_HIP_E_FORMAT, "gguf_tensor_data: tensor %s data out of bounds", name);
    *data = static_cast<const uint8_t*>(g->map) + a;
    if (nbytes) *nbytes = t->nbytes;
    return FT_HIP_OK;
}

// ft-model's to_f32 (lib.rs:128-151): f32 as is, f16 widened, q4_0 blocks
// dequantised (q4_0.rs:43-52: (q - 8) * d, f32 product).
extern "C" int ft_gguf_tensor_to_f32(const ft_gguf* g, const char* name, float* out, uint64_t n) {
    const void* data;
    uint64_t nb;
    if (int rc = ft_gguf_tensor_data(g, name, &data, &nb)) return rc;
    if (!out) return fail(FT_HIP_E_INVALID, "gguf_tensor_to_f32: null out");
    const Tensor* t = &g->tensors[g->t_index.at(name)];
    uint64_t nel = 1;
    for (uint64_t d : t->dims) nel *= d;
    if (n != nel) return fail(FT_HIP_E_SHAPE, "gguf_tensor_to_f32: %s has %llu elements, out has %llu", name, (unsigned long long)nel, (unsigned long long)n);
    const uint8_t* p = static_cast<const uint8_t*>(data);
    switch (t->ggml_type) {
        case 0: std::memcpy(out, p, n * 4); return FT_HIP_OK;
        case 1:
            for (uint64_t i = 0; i < n; ++i) {
                uint16_t h;
                std::memcpy(&h, p + 2 * i, 2);
                out[i] = f16_to_f32(h);
            }
            return FT_HIP_OK;
        case 2:
            for (uint64_t b = 0; b < n / 32; ++b) {
                const uint8_t* blk = p + 18 * b;
                uint16_t h;
                std::memcpy(&h, blk, 2);
                const float d = f16_to_f32(h);
                for (int j = 0; j < 16; ++j) {
                    out[32 * b + j] = (float)((int)(blk[2 + j] & 0x0F) - 8) * d;
                    out[32 * b + j + 16] = (float)((int)(blk[2 + j] >> 4) - 8) * d;
                }
            }
            return FT_HIP_OK;
        default:
            return fail(FT_HIP_E_FORMAT, "gguf_tensor_to_f32: %s: unsupported small-tensor type %u", name, t->ggml_type);
    }
}

// The router of layer l as the expert section consumes it (ft-model,
// lib.rs:506-514): W_r [E][H] from blk.l.ffn_gate_inp.weight with the
// per-column scale blk.l.ffn_gate_inp.scale and H^-1/2 folded in,
// out[e][j] = W_r[e][j] * (scale[j] * H^-1/2) in f32.
extern "C" int ft_gguf_router_f32(const ft_gguf* g, int64_t layer, int64_t hidden, int64_t n_experts, float* out) {
    clear_error();
    if (!g || !out) return fail(FT_HIP_E_INVALID, "gguf_router_f32: null argument");
    if (hidden <= 0 || n_experts <= 0) return fail(FT_HIP_E_SHAPE, "gguf_router_f32: bad shape");
    const std::string w = "blk." + std::to_string(layer) + ".ffn_gate_inp.weight";
    const std::string sc = "blk." + std::to_string(layer) + ".ffn_gate_inp.scale";
    if (int rc = ft_gguf_tensor_to_f32(g, w.c_str(), out, (uint64_t)(hidden * n_experts))) return rc;
    std::vector<float> scale((size_t)hidden);
    if (int rc = ft_gguf_tensor_to_f32(g, sc.c_str(), scale.data(), (uint64_t)hidden)) return rc;
    const float root = std::pow((float)hidden, -0.5f);
    for (int64_t e = 0; e < n_experts; ++e)
        for (int64_t j = 0; j < hidden; ++j) out[e * hidden + j] = out[e * hidden + j] * (scale[(size_t)j] * root);
    return FT_HIP_OK;
}

// Expert banks from a file: blk.l.ffn_gate_up_exps.weight (q4_0, dims
// [H, 2I, E]: per expert the I gate rows then the I up rows) and
// blk.l.ffn_down_exps.weight (q4_0, [I, H, E]) of layers layer0 ..
// layer0+n_layers-1 into banks laid out as ft-model's (lib.rs:570-609):
// expert (l, e) at ((l - layer0) * E + e) * expert_bytes, gate|up rows then
// down rows, each row in `layout`. Each tensor is copied to a device
// staging buffer and repacked there.
extern "C" int ft_hip_load_expert_banks_gguf(ft_hip_ctx* ctx, void* stream, const ft_gguf* g, int64_t layer0,
                                             int64_t n_layers, int64_t hidden, int64_t inter, int64_t n_experts,
                                             void* banks, uint64_t expert_bytes, int layout) {
    clear_error();
    static const char* nm = "load_expert_banks_gguf";
    if (!ctx || !g || !banks) return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    if (layout != FT_LAYOUT_Q4_0 && layout != FT_LAYOUT_Q4R) return fail(FT_HIP_E_INVALID, "%s: bad layout %d", nm, layout);
    if (hidden <= 0 || inter <= 0 || hidden % 32 || inter % 32 || n_experts <= 0 || layer0 < 0 || n_layers < 0)
        return fail(FT_HIP_E_SHAPE, "%s: bad shape", nm);
    const int64_t gu_rb = ft_hip_row_bytes(layout, hidden), dn_rb = ft_hip_row_bytes(layout, inter);
    const uint64_t gu_bytes = (uint64_t)(2 * inter * gu_rb), need = gu_bytes + (uint64_t)(hidden * dn_rb);
    if (expert_bytes < need)
        return fail(FT_HIP_E_SHAPE, "%s: expert_bytes %llu < %llu", nm, (unsigned long long)expert_bytes, (unsigned long long)need);
    if (layout == FT_LAYOUT_Q4R && ((reinterpret_cast<uintptr_t>(banks) | expert_bytes | gu_bytes) & 15))
        return fail(FT_HIP_E_SHAPE, "%s: q4r banks need 16-byte aligned banks and expert_bytes", nm);
    const uint64_t src_gu = (uint64_t)(2 * inter) * (uint64_t)(hidden / 32) * 18;
    const uint64_t src_dn = (uint64_t)hidden * (uint64_t)(inter / 32) * 18;
    // check every tensor before touching the device
    for (int64_t l = layer0; l < layer0 + n_layers; ++l) {
        for (int part = 0; part < 2; ++part) {
            const std::string name = "blk." + std::to_string(l) + (part ? ".ffn_down_exps.weight" : ".ffn_gate_up_exps.weight");
            uint32_t nd, ty;
            uint64_t dims[8], nb;
            const void* data;
            if (int rc = ft_gguf_tensor_info(g, name.c_str(), &nd, dims, &ty, nullptr, &nb)) return rc;
            if (int rc = ft_gguf_tensor_data(g, name.c_str(), &data, &nb)) return rc;
            const uint64_t k = part ? (uint64_t)inter : (uint64_t)hidden, rows = part ? (uint64_t)hidden : (uint64_t)(2 * inter);
            if (ty != 2 || nd != 3 || dims[0] != k || dims[1] != rows || dims[2] != (uint64_t)n_experts)
                return fail(FT_HIP_E_SHAPE, "%s: %s must be q4_0 [%llu, %llu, %lld] (type %u, %u dims [%llu, %llu, %llu])", nm,
                            name.c_str(), (unsigned long long)k, (unsigned long long)rows, (long long)n_experts, ty, nd,
                            (unsigned long long)dims[0], (unsigned long long)dims[1], (unsigned long long)dims[2]);
        }
    }
    if (n_layers == 0) return FT_HIP_OK;
    void* stage = nullptr;
    const uint64_t stage_bytes = (uint64_t)n_experts * std::max(src_gu, src_dn);
    hipError_t e = hipMalloc(&stage, stage_bytes);
    if (e != hipSuccess) return fail(FT_HIP_E_LAUNCH, "%s: staging buffer of %llu B: %s", nm, (unsigned long long)stage_bytes, hipGetErrorString(e));
    int rc = FT_HIP_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    for (int64_t l = layer0; l < layer0 + n_layers && rc == FT_HIP_OK; ++l) {
        for (int part = 0; part < 2 && rc == FT_HIP_OK; ++part) {
            const std::string name = "blk." + std::to_string(l) + (part ? ".ffn_down_exps.weight" : ".ffn_gate_up_exps.weight");
            const void* data;
            uint64_t nb;
            ft_gguf_tensor_data(g, name.c_str(), &data, &nb);
            // pageable source: the copy returns once the data is staged, so
            // the mapping may be dropped afterwards
            if ((e = hipMemcpyAsync(stage, data, nb, hipMemcpyHostToDevice, s)) != hipSuccess) {
                rc = fail(FT_HIP_E_LAUNCH, "%s: upload of %s: %s", nm, name.c_str(), hipGetErrorString(e));
                break;
            }
            const uint64_t per = part ? src_dn : src_gu;
            for (int64_t x = 0; x < n_experts && rc == FT_HIP_OK; ++x) {
                uint8_t* dst = static_cast<uint8_t*>(banks) + (uint64_t)((l - layer0) * n_experts + x) * expert_bytes +
                               (part ? gu_bytes : 0);
                rc = ft_hip_repack_rows(ctx, stream, static_cast<uint8_t*>(stage) + (uint64_t)x * per, FT_LAYOUT_Q4_0,
                                        dst, layout, part ? hidden : 2 * inter, part ? inter : hidden);
            }
        }
    }
    const hipError_t es = hipStreamSynchronize(s);
    if (rc == FT_HIP_OK && es != hipSuccess) rc = fail(FT_HIP_E_LAUNCH, "%s: %s", nm, hipGetErrorString(es));
    (void)hipFree(stage);
    return rc;
}
