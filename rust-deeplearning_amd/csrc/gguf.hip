// gguf.hip -- GGUF reader (include/rdl_gguf.h): the file is memory-mapped and
// parsed in place, tensor bytes go from the mapping to HBM through pinned
// staging buffers.  Host code only.
//
// Parsing follows GGUFFile::parse_bytes (rustml/gguf/main/src/core/parser.rs:
// 151-211) and Cursor::read_value (parser.rs:109-131): the same accepted
// versions, value types, GGML type ids, error kinds and data-section alignment.
// Values are not decoded into a tree: each keeps its type and a pointer into
// the mapping, and the getters decode on demand.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/rdl_gguf.h"
#include "rdl_internal.hpp"

namespace {

using rdl::api_fail;
using rdl::api_ok;

// GGMLType::block_size / block_bytes (types.rs:49-77); -1 for ids that
// GGMLType::from_u32 rejects (types.rs:23-42).
struct GgmlGeom {
    int block_size;
    int block_bytes;
};
GgmlGeom ggml_geom(uint32_t id) {
    switch (id) {
        case 0: return {1, 4};      // F32
        case 1: return {1, 2};      // F16
        case 2: return {32, 18};    // Q4_0
        case 3: return {32, 20};    // Q4_1
        case 6: return {32, 22};    // Q5_0
        case 7: return {32, 24};    // Q5_1
        case 8: return {32, 34};    // Q8_0
        case 9: return {32, 40};    // Q8_1
        case 10: return {256, 84};  // Q2_K
        case 11: return {256, 110}; // Q3_K
        case 12: return {256, 144}; // Q4_K
        case 13: return {256, 176}; // Q5_K
        case 14: return {256, 210}; // Q6_K
        case 15: return {256, 292}; // Q8_K
    }
    return {-1, -1};
}

// Encoded size of a fixed-size scalar value type, 0 for string / array, -1
// for an unknown type id.
int scalar_size(uint32_t type) {
    switch (type) {
        case RDL_GGUF_U8: case RDL_GGUF_I8: case RDL_GGUF_BOOL: return 1;
        case RDL_GGUF_U16: case RDL_GGUF_I16: return 2;
        case RDL_GGUF_U32: case RDL_GGUF_I32: case RDL_GGUF_F32: return 4;
        case RDL_GGUF_U64: case RDL_GGUF_I64: case RDL_GGUF_F64: return 8;
        case RDL_GGUF_STRING: case RDL_GGUF_ARRAY: return 0;
    }
    return -1;
}

// Well-formed UTF-8 (RFC 3629: no overlong forms, no surrogates, at most
// U+10FFFF), the condition String::from_utf8 checks.
bool valid_utf8(const uint8_t* s, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            i++;
            continue;
        }
        int len;
        uint32_t lo = 0x80, hi = 0xBF;  // bounds of the second byte
        if (c >= 0xC2 && c <= 0xDF) len = 2;
        else if (c == 0xE0) len = 3, lo = 0xA0;
        else if (c >= 0xE1 && c <= 0xEC) len = 3;
        else if (c == 0xED) len = 3, hi = 0x9F;
        else if (c >= 0xEE && c <= 0xEF) len = 3;
        else if (c == 0xF0) len = 4, lo = 0x90;
        else if (c >= 0xF1 && c <= 0xF3) len = 4;
        else if (c == 0xF4) len = 4, hi = 0x8F;
        else return false;
        if (n - i < (uint64_t)len) return false;
        if (s[i + 1] < lo || s[i + 1] > hi) return false;
        for (int j = 2; j < len; j++)
            if ((s[i + j] & 0xC0) != 0x80) return false;
        i += len;
    }
    return true;
}

template <typename T>
T load_le(const uint8_t* p) {
    T v;
    memcpy(&v, p, sizeof(T));  // x86-64 and gfx950 hosts are little-endian
    return v;
}

constexpr int MAX_NESTING = 64;  // arrays of arrays deeper than this are rejected

}  // namespace

struct rdl_gguf {
    const uint8_t* data = nullptr;
    uint64_t size = 0;
    void* map = nullptr;  // munmap on close (NULL for caller buffers)
    uint64_t map_len = 0;
    uint32_t version = 0;
    uint64_t data_offset = 0;

    struct Meta {
        std::string key;
        rdl_gguf_value v;
    };
    std::vector<Meta> meta;
    std::unordered_map<std::string, size_t> meta_index;

    struct Tensor {
        std::string name;
        std::vector<uint64_t> dims;
        int32_t type = 0;
        uint64_t offset = 0;
        uint64_t n_bytes = 0;
        uint64_t n_elements = 0;  // product(dims), when it fits (size_overflow otherwise)
        bool size_overflow = false;
    };
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> tensor_index;

    // Element offsets (from `data`) of every array whose elements are strings
    // or arrays, keyed by the array's first-element pointer.
    std::unordered_map<const void*, std::vector<uint64_t>> var_arrays;

    std::mutex stage_mu;
    rdl::Stager* stager = nullptr;

    ~rdl_gguf() {
        delete stager;
        if (map) munmap(map, map_len);
    }
};

namespace {

// Little-endian reader with the reference's EOF checks.  `index`, when set,
// receives the element offsets of every array of strings or arrays.
struct Parser {
    const uint8_t* data;
    uint64_t size;
    std::unordered_map<const void*, std::vector<uint64_t>>* index;
    uint64_t pos = 0;
    rdl_status st = RDL_OK;

    uint64_t remaining() const { return size - pos; }
    bool eof() {
        st = api_fail(RDL_ERR_GGUF_IO, "Unexpected end of GGUF file");
        return false;
    }
    bool need(uint64_t n) { return remaining() >= n ? true : eof(); }
    bool u32(uint32_t* v) {
        if (!need(4)) return false;
        *v = load_le<uint32_t>(data + pos);
        pos += 4;
        return true;
    }
    bool u64(uint64_t* v) {
        if (!need(8)) return false;
        *v = load_le<uint64_t>(data + pos);
        pos += 8;
        return true;
    }
    // read_string (parser.rs:89-96): u64 length, bytes, UTF-8 check
    bool str(const uint8_t** s, uint64_t* len) {
        if (!u64(len) || !need(*len)) return false;
        *s = data + pos;
        if (!valid_utf8(*s, *len)) {
            st = api_fail(RDL_ERR_GGUF_IO, "stream did not contain valid UTF-8");
            return false;
        }
        pos += *len;
        return true;
    }
    // read_value (parser.rs:109-131) for a value of `type` at pos
    bool value(uint32_t type, rdl_gguf_value* v, int depth) {
        v->type = (int32_t)type;
        v->elem_type = -1;
        v->count = 1;
        const int sz = scalar_size(type);
        if (sz < 0) {
            st = api_fail(RDL_ERR_GGUF_UNSUPPORTED_TYPE, "Unknown GGUF value type: %u", type);
            return false;
        }
        if (sz > 0) {
            if (!need((uint64_t)sz)) return false;
            v->raw = data + pos;
            v->raw_len = (uint64_t)sz;
            pos += (uint64_t)sz;
            return true;
        }
        if (type == RDL_GGUF_STRING) {
            const uint8_t* s = nullptr;
            uint64_t len = 0;
            if (!str(&s, &len)) return false;
            v->raw = s;
            v->raw_len = len;
            return true;
        }
        // array: element type, count, elements (each read as read_value reads it)
        if (depth >= MAX_NESTING) {
            st = api_fail(RDL_ERR_GGUF_INVALID_FORMAT, "arrays nested deeper than %d levels", MAX_NESTING);
            return false;
        }
        uint32_t et = 0;
        uint64_t count = 0;
        if (!u32(&et) || !u64(&count)) return false;
        v->elem_type = (int32_t)et;
        v->count = count;
        v->raw = data + pos;
        const uint64_t start = pos;
        if (count > 0) {
            const int esz = scalar_size(et);
            if (esz < 0) {
                st = api_fail(RDL_ERR_GGUF_UNSUPPORTED_TYPE, "Unknown GGUF value type: %u", et);
                return false;
            }
            if (esz > 0) {
                // the reference reads element by element and stops at the end
                if (count > remaining() / (uint64_t)esz) return eof();
                pos += count * (uint64_t)esz;
            } else {
                std::vector<uint64_t> offs;
                for (uint64_t i = 0; i < count; i++) {
                    if (index) offs.push_back(pos);
                    rdl_gguf_value e{};
                    if (!value(et, &e, depth + 1)) return false;
                }
                if (index) (*index)[v->raw] = std::move(offs);
            }
        }
        v->raw_len = pos - start;
        return true;
    }
};

rdl_status parse(rdl_gguf* g) {
    Parser p{g->data, g->size, &g->var_arrays};
    // magic "GGUF" (parser.rs:154-160)
    if (!p.need(4)) return p.st;
    const uint8_t* m = g->data;
    if (memcmp(m, "GGUF", 4) != 0)
        return api_fail(RDL_ERR_GGUF_INVALID_FORMAT,
                        "Invalid GGUF magic: expected [71, 71, 85, 70], got [%u, %u, %u, %u]", m[0], m[1], m[2],
                        m[3]);
    p.pos = 4;
    uint32_t version = 0;
    if (!p.u32(&version)) return p.st;
    if (version < 2 || version > 3)
        return api_fail(RDL_ERR_GGUF_INVALID_FORMAT, "Unsupported GGUF version: %u", version);
    g->version = version;
    uint64_t n_tensors = 0, n_meta = 0;
    if (!p.u64(&n_tensors) || !p.u64(&n_meta)) return p.st;
    // metadata (parser.rs:171-177); a repeated key replaces the value
    for (uint64_t i = 0; i < n_meta; i++) {
        const uint8_t* ks = nullptr;
        uint64_t klen = 0;
        uint32_t vt = 0;
        rdl_gguf_value v{};
        if (!p.str(&ks, &klen) || !p.u32(&vt) || !p.value(vt, &v, 0)) return p.st;
        std::string key((const char*)ks, (size_t)klen);
        auto it = g->meta_index.find(key);
        if (it != g->meta_index.end()) {
            g->meta[it->second].v = v;
        } else {
            g->meta_index.emplace(key, g->meta.size());
            g->meta.push_back({std::move(key), v});
        }
    }
    // tensor infos (parser.rs:179-200); a repeated name: the later one is found
    for (uint64_t i = 0; i < n_tensors; i++) {
        rdl_gguf::Tensor t;
        const uint8_t* ns = nullptr;
        uint64_t nlen = 0;
        uint32_t nd = 0, type = 0;
        if (!p.str(&ns, &nlen) || !p.u32(&nd)) return p.st;
        t.name.assign((const char*)ns, (size_t)nlen);
        if ((uint64_t)nd > p.remaining() / 8) {
            p.eof();
            return p.st;
        }
        t.dims.resize(nd);
        for (uint32_t d = 0; d < nd; d++) p.u64(&t.dims[d]);
        if (!p.u32(&type)) return p.st;
        const GgmlGeom geo = ggml_geom(type);
        if (geo.block_size < 0) return api_fail(RDL_ERR_GGUF_UNSUPPORTED_TYPE, "GGML type: %u", type);
        t.type = (int32_t)type;
        if (!p.u64(&t.offset)) return p.st;
        // load_tensors' size (parser.rs:298-304): product(dims) / block_size
        // blocks, in 128-bit arithmetic; sizes past 64 bits saturate
        using u128 = unsigned __int128;
        u128 ne = 1;
        bool wide = false;  // the product passed 2^128
        bool zero = false;
        for (uint64_t d : t.dims) zero |= d == 0;
        if (!zero)
            for (uint64_t d : t.dims) {
                if (ne > ~(u128)0 / d) wide = true;
                ne *= d;
            }
        const u128 nb = zero ? 0 : (geo.block_size > 1 ? ne / (u128)geo.block_size : ne);
        const u128 bytes = nb * (u128)geo.block_bytes;
        t.size_overflow = !zero && (wide || nb > ~(u128)0 / (u128)geo.block_bytes || bytes > (u128)UINT64_MAX);
        t.n_bytes = t.size_overflow ? UINT64_MAX : (uint64_t)bytes;
        // (a tensor whose bytes lie inside the file has fewer than 2^64 elements)
        t.n_elements = zero ? 0 : (wide || ne > (u128)UINT64_MAX) ? UINT64_MAX : (uint64_t)ne;
        g->tensor_index[t.name] = g->tensors.size();
        g->tensors.push_back(std::move(t));
    }
    // the data section starts at the next multiple of 32 (parser.rs:202)
    g->data_offset = (p.pos + 31) & ~(uint64_t)31;
    return api_ok();
}

rdl_status finish_open(rdl_gguf* h, rdl_gguf** out) {
    const rdl_status st = parse(h);
    if (st != RDL_OK) {
        delete h;
        return st;
    }
    *out = h;
    return api_ok();
}

const rdl_gguf_value* find_meta(const rdl_gguf* g, const char* key) {
    auto it = g->meta_index.find(key);
    return it == g->meta_index.end() ? nullptr : &g->meta[it->second].v;
}

// GGUFValue::as_u32 / as_f32 / as_string (types.rs:97-121)
bool as_u32(const rdl_gguf_value* v, uint32_t* out) {
    if (!v) return false;
    const auto* p = (const uint8_t*)v->raw;
    switch (v->type) {
        case RDL_GGUF_U32: *out = load_le<uint32_t>(p); return true;
        case RDL_GGUF_I32: *out = (uint32_t)load_le<int32_t>(p); return true;
        case RDL_GGUF_U64: *out = (uint32_t)load_le<uint64_t>(p); return true;
    }
    return false;
}
bool as_f32(const rdl_gguf_value* v, float* out) {
    if (!v) return false;
    const auto* p = (const uint8_t*)v->raw;
    if (v->type == RDL_GGUF_F32) return *out = load_le<float>(p), true;
    if (v->type == RDL_GGUF_F64) return *out = (float)load_le<double>(p), true;
    return false;
}

}  // namespace

// ---- pinned staging for host -> device copies -------------------------------
namespace rdl {

Stager::~Stager() {
    for (int b = 0; b < 2; b++) {
        if (ev[b]) (void)hipEventDestroy(ev[b]);
        if (buf[b]) (void)hipHostFree(buf[b]);
    }
}

hipError_t Stager::init() {
    if (buf[0]) return hipSuccess;
    for (int b = 0; b < 2; b++) {
        hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&buf[b]), CHUNK, hipHostMallocDefault);
        if (e != hipSuccess) return e;
        if ((e = hipEventCreateWithFlags(&ev[b], hipEventDisableTiming)) != hipSuccess) return e;
    }
    return hipSuccess;
}

// rows of row_bytes from src (packed) to dst with row pitch dpitch; chunks of
// whole rows alternate between the two pinned buffers, so the host copy of
// one chunk overlaps the DMA of the previous one.
hipError_t Stager::copy2d(const void* src, size_t row_bytes, size_t rows, void* dst, size_t dpitch, hipStream_t s) {
    hipError_t e = init();
    if (e != hipSuccess || rows == 0 || row_bytes == 0) return e;
    const auto* sp = static_cast<const uint8_t*>(src);
    auto* dp = static_cast<uint8_t*>(dst);
    const bool packed = dpitch == row_bytes;
    // a row longer than a chunk is only possible for packed copies (one long row)
    if (!packed && row_bytes > CHUNK) return hipErrorInvalidValue;
    const size_t total = row_bytes * rows;
    const size_t step = packed ? CHUNK : (CHUNK / row_bytes) * row_bytes;
    int b = 0;
    for (size_t off = 0; off < total; off += step, b ^= 1) {
        const size_t n = std::min(step, total - off);
        if ((e = hipEventSynchronize(ev[b])) != hipSuccess) return e;  // buffer b's previous DMA is done
        memcpy(buf[b], sp + off, n);
        if (packed)
            e = hipMemcpyAsync(dp + off, buf[b], n, hipMemcpyHostToDevice, s);
        else
            e = hipMemcpy2DAsync(dp + (off / row_bytes) * dpitch, dpitch, buf[b], row_bytes, row_bytes,
                                 n / row_bytes, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return e;
        if ((e = hipEventRecord(ev[b], s)) != hipSuccess) return e;
    }
    if ((e = hipEventSynchronize(ev[0])) != hipSuccess) return e;
    return hipEventSynchronize(ev[1]);
}

}  // namespace rdl

extern "C" {

rdl_status rdl_gguf_open(const char* path, rdl_gguf** out) {
    if (!path || !out) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return api_fail(RDL_ERR_GGUF_IO, "%s (os error %d)", strerror(errno), errno);
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        const int err = errno;
        close(fd);
        return api_fail(RDL_ERR_GGUF_IO, "%s (os error %d)", strerror(err), err);
    }
    rdl_gguf* h = new rdl_gguf();
    h->size = (uint64_t)sb.st_size;
    if (h->size > 0) {
        void* m = mmap(nullptr, (size_t)h->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            const int err = errno;
            close(fd);
            delete h;
            return api_fail(RDL_ERR_GGUF_IO, "%s (os error %d)", strerror(err), err);
        }
        (void)madvise(m, (size_t)h->size, MADV_SEQUENTIAL);
        h->map = m;
        h->map_len = h->size;
        h->data = static_cast<const uint8_t*>(m);
    }
    close(fd);  // the mapping keeps the file
    return finish_open(h, out);
}

rdl_status rdl_gguf_open_bytes(const void* data, size_t len, rdl_gguf** out) {
    if (!out || (!data && len)) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    *out = nullptr;
    rdl_gguf* h = new rdl_gguf();
    h->data = static_cast<const uint8_t*>(data);
    h->size = len;
    return finish_open(h, out);
}

rdl_status rdl_gguf_close(rdl_gguf* g) {
    delete g;
    return api_ok();
}

#define GGUF_GETTER(fn, T, expr)                                                 \
    rdl_status fn(const rdl_gguf* g, T* out) {                                   \
        if (!g || !out) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument"); \
        *out = (expr);                                                           \
        return api_ok();                                                         \
    }
GGUF_GETTER(rdl_gguf_version, uint32_t, g->version)
GGUF_GETTER(rdl_gguf_data_offset, uint64_t, g->data_offset)
GGUF_GETTER(rdl_gguf_file_size, uint64_t, g->size)
GGUF_GETTER(rdl_gguf_tensor_count, size_t, g->tensors.size())
GGUF_GETTER(rdl_gguf_metadata_count, size_t, g->meta.size())
#undef GGUF_GETTER

rdl_status rdl_gguf_metadata_at(const rdl_gguf* g, size_t i, const char** key, size_t* key_len,
                                rdl_gguf_value* value) {
    if (!g || !key || !key_len || !value) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    if (i >= g->meta.size())
        return api_fail(RDL_ERR_NOT_FOUND, "metadata index %zu out of range (%zu entries)", i, g->meta.size());
    *key = g->meta[i].key.c_str();
    *key_len = g->meta[i].key.size();
    *value = g->meta[i].v;
    return api_ok();
}

rdl_status rdl_gguf_metadata_find(const rdl_gguf* g, const char* key, rdl_gguf_value* value) {
    if (!g || !key || !value) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    const rdl_gguf_value* v = find_meta(g, key);
    if (!v) return api_fail(RDL_ERR_NOT_FOUND, "Key not found: %s", key);
    *value = *v;
    return api_ok();
}

rdl_status rdl_gguf_array_element(const rdl_gguf* g, const rdl_gguf_value* array, uint64_t i, rdl_gguf_value* elem) {
    if (!g || !array || !elem) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    if (array->type != RDL_GGUF_ARRAY) return api_fail(RDL_ERR_INVALID_DATA, "value is not an array");
    if (i >= array->count) return api_fail(RDL_ERR_NOT_FOUND, "element %llu of %llu", (unsigned long long)i,
                                           (unsigned long long)array->count);
    const uint32_t et = (uint32_t)array->elem_type;
    const int esz = scalar_size(et);
    if (esz > 0) {
        *elem = rdl_gguf_value{(int32_t)et, -1, 1, (const uint8_t*)array->raw + i * (uint64_t)esz, (uint64_t)esz};
        return api_ok();
    }
    auto it = g->var_arrays.find(array->raw);
    if (it == g->var_arrays.end()) return api_fail(RDL_ERR_INVALID_DATA, "array value not from this file");
    // decode the element where parsing found it (already validated)
    Parser p{g->data, g->size, nullptr};
    p.pos = it->second[(size_t)i];
    return p.value(et, elem, 1) ? api_ok() : p.st;
}

rdl_status rdl_gguf_get_u32(const rdl_gguf* g, const char* key, uint32_t* out) {
    if (!g || !key || !out) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    if (!as_u32(find_meta(g, key), out)) return api_fail(RDL_ERR_GGUF_MISSING_METADATA, "%s", key);
    return api_ok();
}

rdl_status rdl_gguf_get_f32(const rdl_gguf* g, const char* key, float* out) {
    if (!g || !key || !out) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    if (!as_f32(find_meta(g, key), out)) return api_fail(RDL_ERR_GGUF_MISSING_METADATA, "%s", key);
    return api_ok();
}

rdl_status rdl_gguf_get_string(const rdl_gguf* g, const char* key, const char** out, size_t* len) {
    if (!g || !key || !out || !len) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    const rdl_gguf_value* v = find_meta(g, key);
    if (!v || v->type != RDL_GGUF_STRING) return api_fail(RDL_ERR_GGUF_MISSING_METADATA, "%s", key);
    *out = (const char*)v->raw;
    *len = (size_t)v->raw_len;
    return api_ok();
}

rdl_status rdl_gguf_tensor_info_at(const rdl_gguf* g, size_t i, rdl_gguf_tensor_info* out) {
    if (!g || !out) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    if (i >= g->tensors.size())
        return api_fail(RDL_ERR_NOT_FOUND, "tensor index %zu out of range (%zu tensors)", i, g->tensors.size());
    const rdl_gguf::Tensor& t = g->tensors[i];
    out->name = t.name.c_str();
    out->name_len = t.name.size();
    out->n_dims = (uint32_t)t.dims.size();
    out->dims = t.dims.data();
    out->ggml_type = t.type;
    out->offset = t.offset;
    out->n_bytes = t.n_bytes;
    return api_ok();
}

rdl_status rdl_gguf_find_tensor(const rdl_gguf* g, const char* name, size_t* index) {
    if (!g || !name || !index) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    auto it = g->tensor_index.find(name);
    if (it == g->tensor_index.end()) return api_fail(RDL_ERR_NOT_FOUND, "Missing tensor: %s", name);
    *index = it->second;
    return api_ok();
}

rdl_status rdl_gguf_tensor_data(const rdl_gguf* g, size_t i, const void** data, uint64_t* len) {
    if (!g || !data || !len) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    if (i >= g->tensors.size())
        return api_fail(RDL_ERR_NOT_FOUND, "tensor index %zu out of range (%zu tensors)", i, g->tensors.size());
    const rdl_gguf::Tensor& t = g->tensors[i];
    // load_tensors' bound check (parser.rs:306-312)
    const uint64_t abs = g->data_offset + t.offset;
    if (t.size_overflow || abs < g->data_offset || abs > g->size || t.n_bytes > g->size - abs)
        return api_fail(RDL_ERR_GGUF_IO, "Tensor '%s' data exceeds file bounds", t.name.c_str());
    *data = g->data + abs;
    *len = t.n_bytes;
    return api_ok();
}

rdl_status rdl_gguf_upload_tensor(const rdl_gguf* g, size_t i, void* dst_dev, uint64_t dst_len, void* stream) {
    if (!g || !dst_dev) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    const void* src = nullptr;
    uint64_t len = 0;
    rdl_status st = rdl_gguf_tensor_data(g, i, &src, &len);
    if (st != RDL_OK) return st;
    if (dst_len < len)
        return rdl::api_shape_fail(("tensor '" + g->tensors[i].name + "' bytes (destination holds the second)").c_str(),
                                   {(size_t)len}, {(size_t)dst_len});
    if ((st = rdl::api_require_device()) != RDL_OK) return st;
    auto* gm = const_cast<rdl_gguf*>(g);
    std::lock_guard<std::mutex> lk(gm->stage_mu);
    if (!gm->stager) gm->stager = new rdl::Stager();
    HIP_TRY(gm->stager->copy2d(src, (size_t)len, 1, dst_dev, (size_t)len, (hipStream_t)stream));
    return api_ok();
}

rdl_status rdl_gguf_upload_tensor_f32(const rdl_gguf* g, size_t i, float* dst_dev, uint64_t dst_len, void* stream) {
    if (!g || !dst_dev) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    const void* src = nullptr;
    uint64_t len = 0;
    rdl_status st = rdl_gguf_tensor_data(g, i, &src, &len);
    if (st != RDL_OK) return st;
    const rdl_gguf::Tensor& t = g->tensors[i];
    if (dst_len < t.n_elements)
        return rdl::api_shape_fail(("tensor '" + t.name + "' elements (destination holds the second)").c_str(),
                                   {(size_t)t.n_elements}, {(size_t)dst_len});
    if ((uintptr_t)dst_dev & 15) return api_fail(RDL_ERR_INVALID_DATA, "destination must be 16-byte aligned");
    if ((st = rdl::api_require_device()) != RDL_OK) return st;
    if (t.n_elements == 0) return api_ok();
    hipStream_t s = (hipStream_t)stream;
    auto* gm = const_cast<rdl_gguf*>(g);
    std::lock_guard<std::mutex> lk(gm->stage_mu);
    if (!gm->stager) gm->stager = new rdl::Stager();
    if (t.type == 0) {  // F32: the file bytes are the values
        HIP_TRY(gm->stager->copy2d(src, (size_t)len, 1, dst_dev, (size_t)len, s));
        return api_ok();
    }
    // the raw blocks into device scratch, expanded from there
    void* raw = nullptr;
    HIP_TRY(hipMalloc(&raw, (size_t)len + 16));
    hipError_t e = gm->stager->copy2d(src, (size_t)len, 1, raw, (size_t)len, s);
    if (e == hipSuccess) e = rdl::launch_dequant_gguf(t.type, static_cast<const uint8_t*>(raw), t.n_elements, dst_dev, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipFree(raw);
    if (e != hipSuccess) return api_fail(RDL_ERR_HIP, "f32 upload of '%s' failed: %s", t.name.c_str(), hipGetErrorString(e));
    return api_ok();
}

// to_model_config (parser.rs:214-289)
rdl_status rdl_gguf_model_config_get(const rdl_gguf* g, rdl_gguf_model_config* out) {
    if (!g || !out) return api_fail(RDL_ERR_NULL_POINTER, "NULL argument");
    rdl_gguf_model_config c{};
    std::string arch = "llama";
    const rdl_gguf_value* av = find_meta(g, "general.architecture");
    if (av && av->type == RDL_GGUF_STRING) arch.assign((const char*)av->raw, (size_t)av->raw_len);
    snprintf(c.architecture, sizeof c.architecture, "%.*s", (int)std::min<size_t>(arch.size(), 63), arch.c_str());
    auto key = [&](const char* suffix) { return arch + "." + suffix; };
    auto u32 = [&](const std::string& k, uint32_t* v) { return as_u32(find_meta(g, k.c_str()), v); };
    auto f32 = [&](const std::string& k, float* v) { return as_f32(find_meta(g, k.c_str()), v); };
    for (const char* req : {"embedding_length", "attention.head_count", "block_count"}) {
        uint32_t v = 0;
        if (!u32(key(req), &v)) return api_fail(RDL_ERR_GGUF_MISSING_METADATA, "%s", key(req).c_str());
    }
    u32(key("embedding_length"), &c.dim);
    u32(key("attention.head_count"), &c.n_heads);
    u32(key("block_count"), &c.n_layers);
    // vocab: {arch}.vocab_size, tokenizer.ggml.tokens_count, len(tokenizer.ggml.tokens), 32000
    if (!u32(key("vocab_size"), &c.vocab_size) && !u32("tokenizer.ggml.tokens_count", &c.vocab_size)) {
        const rdl_gguf_value* tv = find_meta(g, "tokenizer.ggml.tokens");
        c.vocab_size = (tv && tv->type == RDL_GGUF_ARRAY) ? (uint32_t)tv->count : 32000u;
    }
    if (!u32(key("feed_forward_length"), &c.hidden_dim)) c.hidden_dim = (uint32_t)((uint64_t)c.dim * 4);
    c.has_n_kv_heads = u32(key("attention.head_count_kv"), &c.n_kv_heads);
    if (!c.has_n_kv_heads) c.n_kv_heads = 0;
    if (!u32(key("context_length"), &c.max_seq_len)) c.max_seq_len = 2048;
    if (!f32(key("attention.layer_norm_rms_epsilon"), &c.norm_eps)) c.norm_eps = 1e-5f;
    if (!f32(key("rope.freq_base"), &c.rope_theta)) c.rope_theta = 10000.0f;
    c.has_head_dim = u32(key("attention.key_length"), &c.head_dim);
    if (!c.has_head_dim) c.head_dim = 0;
    c.has_sliding_window = u32(key("attention.sliding_window"), &c.sliding_window);
    if (!c.has_sliding_window) c.sliding_window = 0;
    uint32_t t = 0;
    c.bos_token_id = u32("tokenizer.ggml.bos_token_id", &t) ? (int64_t)t : -1;
    c.eos_token_id = u32("tokenizer.ggml.eos_token_id", &t) ? (int64_t)t : -1;
    const rdl_gguf_value* ct = find_meta(g, "tokenizer.chat_template");
    c.has_chat_template = ct && ct->type == RDL_GGUF_STRING;
    *out = c;
    return api_ok();
}

}  // extern "C"
