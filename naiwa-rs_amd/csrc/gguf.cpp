// gguf.cpp -- read-only GGUF (v2, v3) reader: the file is mapped, every length
// and offset is checked against the mapping, and the tensors and metadata are
// indexed by name.  Expert stacks follow expert_range (src/moe/expert.rs:123-145):
// expert e of a [E, N, K] stack is bytes [e * stride, (e + 1) * stride) with
// stride = N * (K / block) * type size.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/naiwa_gguf.h"
#include "../../include/naiwa_moe.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u; // "GGUF" little-endian
constexpr uint64_t kMaxCount = 1u << 24; // tensors or keys: far beyond any checkpoint
constexpr int kMaxDims = 4;

// GGUF metadata value types.
enum : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12
};

// (block values, block bytes) of the GGML types, from the public block layouts.
struct TypeSize {
    int block, bytes;
};
TypeSize type_size(int t) {
    switch (t) {
    case 0: return {1, 4};     // F32
    case 1: return {1, 2};     // F16
    case 2: return {32, 18};   // Q4_0
    case 3: return {32, 20};   // Q4_1
    case 6: return {32, 22};   // Q5_0
    case 7: return {32, 24};   // Q5_1
    case 8: return {32, 34};   // Q8_0
    case 9: return {32, 36};   // Q8_1
    case 10: return {256, 84}; // Q2_K
    case 11: return {256, 110}; // Q3_K
    case 12: return {256, 144}; // Q4_K
    case 13: return {256, 176}; // Q5_K
    case 14: return {256, 210}; // Q6_K
    case 15: return {256, 292}; // Q8_K
    case 16: return {256, 66};  // IQ2_XXS
    case 17: return {256, 74};  // IQ2_XS
    case 18: return {256, 98};  // IQ3_XXS
    case 19: return {256, 50};  // IQ1_S
    case 20: return {32, 18};   // IQ4_NL
    case 21: return {256, 110}; // IQ3_S
    case 22: return {256, 82};  // IQ2_S
    case 23: return {256, 136}; // IQ4_XS
    case 24: return {1, 1};     // I8
    case 25: return {1, 2};     // I16
    case 26: return {1, 4};     // I32
    case 27: return {1, 8};     // I64
    case 28: return {1, 8};     // F64
    case 29: return {256, 56};  // IQ1_M
    case 30: return {1, 2};     // BF16
    default: return {0, 0};
    }
}

int scalar_bytes(uint32_t t) {
    switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
    }
}

// A bounds-checked little-endian cursor over the mapping.
struct Cursor {
    const uint8_t* p;
    size_t n, at = 0;
    bool take(void* dst, size_t k) {
        if (k > n - at) return false;
        memcpy(dst, p + at, k);
        at += k;
        return true;
    }
    bool skip(uint64_t k) {
        if (k > n - at) return false;
        at += (size_t)k;
        return true;
    }
    bool u32(uint32_t& v) { return take(&v, 4); }
    bool u64(uint64_t& v) { return take(&v, 8); }
    bool str(std::string& s) {
        uint64_t len;
        if (!u64(len) || len > n - at) return false;
        s.assign((const char*)p + at, (size_t)len);
        at += (size_t)len;
        return true;
    }
    // One value of type t (arrays recursively, to a bounded depth).
    bool skip_value(uint32_t t, int depth = 0) {
        if (t == kString) {
            uint64_t len;
            return u64(len) && skip(len);
        }
        if (t == kArray) {
            uint32_t et;
            uint64_t count;
            if (depth > 2 || !u32(et) || !u64(count)) return false;
            if (et == kString || et == kArray) {
                for (uint64_t i = 0; i < count; ++i)
                    if (!skip_value(et, depth + 1)) return false;
                return true;
            }
            const int b = scalar_bytes(et);
            return b > 0 && count <= (n - at) / (uint64_t)b && skip(count * (uint64_t)b);
        }
        const int b = scalar_bytes(t);
        return b > 0 && skip((uint64_t)b);
    }
};

struct Meta {
    uint32_t type;
    size_t at; // offset of the value in the mapping
};

struct Tensor {
    std::string name;
    int n_dims;
    int64_t dims[kMaxDims];
    int dtype;
    uint64_t offset, bytes;
};

} // namespace

struct naiwa_gguf {
    const uint8_t* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
    std::unordered_map<std::string, Meta> meta;

    ~naiwa_gguf() {
        if (map) munmap((void*)map, size);
    }
};

namespace {

int parse(naiwa_gguf& f) {
    Cursor c{f.map, f.size};
    uint32_t magic;
    uint64_t n_tensors, n_kv;
    if (!c.u32(magic) || magic != kMagic || !c.u32(f.version)) return NAIWA_E_FORMAT;
    if (f.version != 2 && f.version != 3) return NAIWA_E_FORMAT; // v1 used 32-bit counts
    if (!c.u64(n_tensors) || !c.u64(n_kv) || n_tensors > kMaxCount || n_kv > kMaxCount) return NAIWA_E_FORMAT;
    // a key takes at least 12 bytes and a tensor info 28: bound both by the file before allocating
    if (n_kv > f.size / 12 || n_tensors > f.size / 28) return NAIWA_E_FORMAT;
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key;
        uint32_t t;
        if (!c.str(key) || !c.u32(t)) return NAIWA_E_FORMAT;
        const size_t at = c.at;
        if (!c.skip_value(t)) return NAIWA_E_FORMAT;
        if (!f.meta.emplace(key, Meta{t, at}).second) return NAIWA_E_FORMAT; // duplicate key
    }
    auto al = f.meta.find("general.alignment");
    if (al != f.meta.end()) {
        if (al->second.type != kU32) return NAIWA_E_FORMAT;
        uint32_t a;
        memcpy(&a, f.map + al->second.at, 4);
        if (a == 0 || (a & (a - 1))) return NAIWA_E_FORMAT; // a power of two
        f.alignment = a;
    }
    f.tensors.resize((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Tensor& t = f.tensors[(size_t)i];
        uint32_t nd, dt;
        if (!c.str(t.name) || !c.u32(nd) || nd < 1 || nd > (uint32_t)kMaxDims) return NAIWA_E_FORMAT;
        t.n_dims = (int)nd;
        uint64_t elems = 1;
        for (int d = 0; d < kMaxDims; ++d) {
            uint64_t v = 1;
            if (d < t.n_dims && (!c.u64(v) || v == 0 || v > (1ull << 40))) return NAIWA_E_FORMAT;
            t.dims[d] = (int64_t)v;
            if (elems > (1ull << 50) / v) return NAIWA_E_FORMAT;
            elems *= v;
        }
        if (!c.u32(dt) || !c.u64(t.offset)) return NAIWA_E_FORMAT;
        t.dtype = (int)dt;
        const TypeSize ts = type_size(t.dtype);
        t.bytes = 0;
        if (ts.block > 0) {
            if (t.dims[0] % ts.block) return NAIWA_E_FORMAT; // rows are whole blocks
            t.bytes = elems / (uint64_t)ts.block * (uint64_t)ts.bytes;
        }
        if (!f.by_name.emplace(t.name, (size_t)i).second) return NAIWA_E_FORMAT; // duplicate name
    }
    // the data section starts at the next multiple of the alignment
    const uint64_t data = (c.at + f.alignment - 1) / f.alignment * f.alignment;
    for (Tensor& t : f.tensors) {
        if (t.offset % f.alignment) return NAIWA_E_FORMAT;
        if (data > f.size || t.offset > f.size - data || t.bytes > f.size - data - t.offset) return NAIWA_E_FORMAT;
        t.offset += data;
    }
    return NAIWA_OK;
}

void fill(const naiwa_gguf* f, const Tensor& t, naiwa_gguf_tensor* out) {
    out->name = t.name.c_str();
    out->n_dims = t.n_dims;
    for (int d = 0; d < kMaxDims; ++d) out->dims[d] = t.dims[d];
    out->dtype = t.dtype;
    out->offset = t.offset;
    out->bytes = t.bytes;
    out->data = t.bytes ? f->map + t.offset : nullptr;
}

} // namespace

extern "C" int naiwa_gguf_open(const char* path, naiwa_gguf** out) {
    if (!path || !out) return NAIWA_E_INVALID;
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return NAIWA_E_IO;
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return NAIWA_E_IO;
    }
    if (st.st_size <= 0) { // an empty file has no header
        close(fd);
        return NAIWA_E_FORMAT;
    }
    void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd); // the mapping keeps the file
    if (m == MAP_FAILED) return NAIWA_E_IO;
    naiwa_gguf* f = new (std::nothrow) naiwa_gguf;
    if (!f) {
        munmap(m, (size_t)st.st_size);
        return NAIWA_E_NOMEM;
    }
    f->map = (const uint8_t*)m;
    f->size = (size_t)st.st_size;
    int rc;
    try {
        rc = parse(*f);
    } catch (...) {
        rc = NAIWA_E_NOMEM;
    }
    if (rc) {
        delete f;
        return rc;
    }
    *out = f;
    return NAIWA_OK;
}

extern "C" int naiwa_gguf_close(naiwa_gguf* f) {
    delete f;
    return NAIWA_OK;
}

extern "C" int naiwa_gguf_version(const naiwa_gguf* f, uint32_t* version) {
    if (!f || !version) return NAIWA_E_INVALID;
    *version = f->version;
    return NAIWA_OK;
}

extern "C" int naiwa_gguf_alignment(const naiwa_gguf* f, uint64_t* alignment) {
    if (!f || !alignment) return NAIWA_E_INVALID;
    *alignment = f->alignment;
    return NAIWA_OK;
}

extern "C" int naiwa_gguf_tensor_count(const naiwa_gguf* f, int* n) {
    if (!f || !n) return NAIWA_E_INVALID;
    *n = (int)f->tensors.size();
    return NAIWA_OK;
}

extern "C" int naiwa_gguf_tensor_at(const naiwa_gguf* f, int i, naiwa_gguf_tensor* out) {
    if (!f || !out || i < 0 || (size_t)i >= f->tensors.size()) return NAIWA_E_INVALID;
    fill(f, f->tensors[(size_t)i], out);
    return NAIWA_OK;
}

extern "C" int naiwa_gguf_find(const naiwa_gguf* f, const char* name, naiwa_gguf_tensor* out) {
    if (!f || !name || !out) return NAIWA_E_INVALID;
    auto it = f->by_name.find(name);
    if (it == f->by_name.end()) return NAIWA_E_NOT_FOUND;
    fill(f, f->tensors[it->second], out);
    return NAIWA_OK;
}

extern "C" int naiwa_gguf_meta_u64(const naiwa_gguf* f, const char* key, uint64_t* value) {
    if (!f || !key || !value) return NAIWA_E_INVALID;
    auto it = f->meta.find(key);
    if (it == f->meta.end()) return NAIWA_E_NOT_FOUND;
    const uint8_t* p = f->map + it->second.at;
    switch (it->second.type) {
    case kU8: case kBool: *value = p[0]; return NAIWA_OK;
    case kU16: { uint16_t v; memcpy(&v, p, 2); *value = v; return NAIWA_OK; }
    case kU32: { uint32_t v; memcpy(&v, p, 4); *value = v; return NAIWA_OK; }
    case kU64: memcpy(value, p, 8); return NAIWA_OK;
    case kI8: { int8_t v; memcpy(&v, p, 1); if (v < 0) return NAIWA_E_FORMAT; *value = (uint64_t)v; return NAIWA_OK; }
    case kI16: { int16_t v; memcpy(&v, p, 2); if (v < 0) return NAIWA_E_FORMAT; *value = (uint64_t)v; return NAIWA_OK; }
    case kI32: { int32_t v; memcpy(&v, p, 4); if (v < 0) return NAIWA_E_FORMAT; *value = (uint64_t)v; return NAIWA_OK; }
    case kI64: { int64_t v; memcpy(&v, p, 8); if (v < 0) return NAIWA_E_FORMAT; *value = (uint64_t)v; return NAIWA_OK; }
    default: return NAIWA_E_FORMAT;
    }
}

extern "C" int naiwa_gguf_meta_string(const naiwa_gguf* f, const char* key, char* buf, int cap, int* len) {
    if (!f || !key) return NAIWA_E_INVALID;
    auto it = f->meta.find(key);
    if (it == f->meta.end()) return NAIWA_E_NOT_FOUND;
    if (it->second.type != kString) return NAIWA_E_FORMAT;
    uint64_t n;
    memcpy(&n, f->map + it->second.at, 8); // validated while parsing
    if (len) *len = n > 0x7fffffffull ? 0x7fffffff : (int)n;
    if (!buf || cap < 0 || n + 1 > (uint64_t)cap) return NAIWA_E_INVALID;
    memcpy(buf, f->map + it->second.at + 8, (size_t)n);
    buf[n] = '\0';
    return NAIWA_OK;
}

extern "C" int naiwa_ggml_type_size(int dtype, int* block, int* bytes) {
    if (!block || !bytes) return NAIWA_E_INVALID;
    const TypeSize ts = type_size(dtype);
    *block = ts.block;
    *bytes = ts.bytes;
    return NAIWA_OK;
}

extern "C" int naiwa_gguf_expert_stack(const naiwa_gguf* f, int layer, int proj, naiwa_expert_stack* out) {
    static const char* kProj[3] = {"ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"};
    if (!f || !out || layer < 0 || proj < 0 || proj > 2) return NAIWA_E_INVALID;
    const std::string name = "blk." + std::to_string(layer) + "." + kProj[proj] + ".weight";
    auto it = f->by_name.find(name);
    if (it == f->by_name.end()) return NAIWA_E_NOT_FOUND;
    const Tensor& t = f->tensors[it->second];
    const TypeSize ts = type_size(t.dtype);
    if (ts.block == 0 || t.bytes == 0) return NAIWA_E_UNSUPPORTED;
    if (t.n_dims < 3 || t.dims[3] != 1) return NAIWA_E_UNSUPPORTED; // [E, N, K]
    if (t.dims[0] > 0x7fffffff || t.dims[1] > 0x7fffffff || t.dims[2] > 0x7fffffff) return NAIWA_E_UNSUPPORTED;
    out->data = f->map + t.offset;
    out->k = (int)t.dims[0];
    out->n = (int)t.dims[1];
    out->experts = (int)t.dims[2];
    out->dtype = t.dtype;
    out->expert_bytes = (uint64_t)t.dims[1] * (uint64_t)(t.dims[0] / ts.block) * (uint64_t)ts.bytes;
    return NAIWA_OK;
}
