// gguf_reader.cpp -- GGUF model-file reader (C ABI in include/q4k_gguf.h).
//
// File layout (GGUF v2/v3, little-endian; the format ggml's gguf.cpp writes
// and reads):
//   u32 magic "GGUF", u32 version, u64 n_tensors, u64 n_kv
//   n_kv x { string key, u32 type, value }
//       string = u64 length + bytes (no terminator)
//       value  = scalar of the type's size, string, or
//                array = u32 element type, u64 count, count elements
//   n_tensors x { string name, u32 n_dims, u64 ne[n_dims], u32 ggml type,
//                 u64 offset (from the data section, a multiple of the alignment) }
//   padding to general.alignment (u32 metadata, default 32), then the data.
// The whole file is mapped read-only; every length, count and offset is
// checked against the mapping before it is used.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <limits>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/q4k_gguf.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"
constexpr uint64_t kDefaultAlignment = 32;

struct Kv {
    std::string key;
    int32_t type = 0;
    size_t value_off = 0;    // file offset of the value (scalars, array payload)
    int32_t elem_type = -1;  // arrays
    uint64_t count = 0;      // arrays
    std::string str;         // string values
    std::vector<std::string> strs;  // string arrays
};

struct Tensor {
    std::string name;
    int32_t type = 0;
    int32_t n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t rel_offset = 0;
    uint64_t nbytes = 0;
};

// (bytes per block, elements per block) of the ggml types, {0, 0} unknown.
struct BlockSize {
    uint32_t bytes, elems;
};

BlockSize block_size(int32_t type) {
    switch (type) {
        case 0: return {4, 1};      // F32
        case 1: return {2, 1};      // F16
        case 2: return {18, 32};    // Q4_0
        case 3: return {20, 32};    // Q4_1
        case 6: return {22, 32};    // Q5_0
        case 7: return {24, 32};    // Q5_1
        case 8: return {34, 32};    // Q8_0
        case 9: return {36, 32};    // Q8_1
        case 10: return {84, 256};  // Q2_K
        case 11: return {110, 256}; // Q3_K
        case 12: return {144, 256}; // Q4_K
        case 13: return {176, 256}; // Q5_K
        case 14: return {210, 256}; // Q6_K
        case 15: return {292, 256}; // Q8_K
        case 16: return {66, 256};  // IQ2_XXS
        case 17: return {74, 256};  // IQ2_XS
        case 18: return {98, 256};  // IQ3_XXS
        case 19: return {50, 256};  // IQ1_S
        case 20: return {18, 32};   // IQ4_NL
        case 21: return {110, 256}; // IQ3_S
        case 22: return {82, 256};  // IQ2_S
        case 23: return {136, 256}; // IQ4_XS
        case 24: return {1, 1};     // I8
        case 25: return {2, 1};     // I16
        case 26: return {4, 1};     // I32
        case 27: return {8, 1};     // I64
        case 28: return {8, 1};     // F64
        case 29: return {56, 256};  // IQ1_M
        case 30: return {2, 1};     // BF16
        case 34: return {54, 256};  // TQ1_0
        case 35: return {66, 256};  // TQ2_0
        case 39: return {17, 32};   // MXFP4
        default: return {0, 0};
    }
}

// Size of a scalar metadata value, 0 for string/array/unknown.
size_t scalar_size(int32_t t) {
    switch (t) {
        case Q4K_GGUF_UINT8: case Q4K_GGUF_INT8: case Q4K_GGUF_BOOL: return 1;
        case Q4K_GGUF_UINT16: case Q4K_GGUF_INT16: return 2;
        case Q4K_GGUF_UINT32: case Q4K_GGUF_INT32: case Q4K_GGUF_FLOAT32: return 4;
        case Q4K_GGUF_UINT64: case Q4K_GGUF_INT64: case Q4K_GGUF_FLOAT64: return 8;
        default: return 0;
    }
}

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
    const uint8_t *base;
    size_t size;
    size_t pos = 0;
    bool ok = true;

    bool need(uint64_t n) {
        if (!ok || n > size - pos) ok = false;
        return ok;
    }
    template <typename T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, base + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return std::string();
        std::string s(reinterpret_cast<const char *>(base + pos), (size_t)n);
        pos += (size_t)n;
        return s;
    }
    void skip(uint64_t n) {
        if (need(n)) pos += (size_t)n;
    }
};

}  // namespace

struct q4k_gguf {
    int fd = -1;
    const uint8_t *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = kDefaultAlignment;
    uint64_t data_offset = 0;
    std::vector<Kv> kvs;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> tensor_index, key_index;

    ~q4k_gguf() {
        if (map) munmap(const_cast<uint8_t *>(map), size);
        if (fd >= 0) close(fd);
    }
};

namespace {

int parse(q4k_gguf &g) {
    Cursor c{g.map, g.size};
    if (c.get<uint32_t>() != kMagic) return Q4K_EFORMAT;
    g.version = c.get<uint32_t>();
    if (!c.ok || (g.version != 2 && g.version != 3)) return Q4K_EFORMAT;
    const uint64_t n_tensors = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    // every kv needs at least 12 bytes and every tensor info at least 24
    if (!c.ok || n_kv > g.size / 12 || n_tensors > g.size / 24) return Q4K_EFORMAT;
    g.kvs.reserve((size_t)n_kv);
    for (uint64_t i = 0; i < n_kv; ++i) {
        Kv kv;
        kv.key = c.str();
        kv.type = (int32_t)c.get<uint32_t>();
        if (!c.ok) return Q4K_EFORMAT;
        kv.value_off = c.pos;
        if (kv.type == Q4K_GGUF_STRING) {
            kv.str = c.str();
        } else if (kv.type == Q4K_GGUF_ARRAY) {
            kv.elem_type = (int32_t)c.get<uint32_t>();
            kv.count = c.get<uint64_t>();
            if (!c.ok) return Q4K_EFORMAT;
            kv.value_off = c.pos;
            if (kv.elem_type == Q4K_GGUF_STRING) {
                if (kv.count > (g.size - c.pos) / 8) return Q4K_EFORMAT;
                kv.strs.reserve((size_t)kv.count);
                for (uint64_t j = 0; j < kv.count && c.ok; ++j) kv.strs.push_back(c.str());
            } else {
                const size_t es = scalar_size(kv.elem_type);
                if (es == 0 || kv.count > (g.size - c.pos) / es) return Q4K_EFORMAT;
                c.skip(kv.count * es);
            }
        } else {
            const size_t es = scalar_size(kv.type);
            if (es == 0) return Q4K_EFORMAT;
            c.skip(es);
        }
        if (!c.ok) return Q4K_EFORMAT;
        if (kv.key == "general.alignment") {
            if (kv.type != Q4K_GGUF_UINT32) return Q4K_EFORMAT;
            uint32_t a;
            std::memcpy(&a, g.map + kv.value_off, 4);
            if (a == 0 || (a & (a - 1)) != 0) return Q4K_EFORMAT;
            g.alignment = a;
        }
        if (!g.key_index.emplace(kv.key, (int64_t)g.kvs.size()).second) return Q4K_EFORMAT;  // duplicate key
        g.kvs.push_back(std::move(kv));
    }
    g.tensors.reserve((size_t)n_tensors);
    uint64_t data_size = 0;  // running padded size of the tensors so far
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Tensor t;
        t.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        if (!c.ok || nd < 1 || nd > 4) return Q4K_EFORMAT;
        t.n_dims = (int32_t)nd;
        uint64_t nel = 1;
        for (uint32_t d = 0; d < nd; ++d) {
            const uint64_t n = c.get<uint64_t>();
            if (n > (uint64_t)std::numeric_limits<int64_t>::max() || (n && nel > UINT64_MAX / n))
                return Q4K_EFORMAT;
            t.ne[d] = (int64_t)n;
            nel *= n;
        }
        t.type = (int32_t)c.get<uint32_t>();
        t.rel_offset = c.get<uint64_t>();
        if (!c.ok) return Q4K_EFORMAT;
        const BlockSize bs = block_size(t.type);
        if (!bs.elems) return Q4K_EFORMAT;  // unknown or removed type: its size is unknown
        if (t.ne[0] % bs.elems != 0) return Q4K_EFORMAT;  // rows are whole blocks
        const uint64_t blocks = nel / bs.elems;
        if (blocks > UINT64_MAX / bs.bytes) return Q4K_EFORMAT;
        t.nbytes = blocks * bs.bytes;
        // ggml's loader lays the tensors out back to back in directory
        // order, each padded to the alignment, and refuses a file whose
        // offsets differ from that layout (gaps, overlaps, reordering)
        if (t.rel_offset != data_size) return Q4K_EFORMAT;
        const uint64_t padded = t.nbytes + (g.alignment - t.nbytes % g.alignment) % g.alignment;
        if (padded < t.nbytes || data_size > UINT64_MAX - padded) return Q4K_EFORMAT;
        data_size += padded;
        if (!g.tensor_index.emplace(t.name, (int64_t)g.tensors.size()).second) return Q4K_EFORMAT;
        g.tensors.push_back(std::move(t));
    }
    const uint64_t pad = (g.alignment - c.pos % g.alignment) % g.alignment;
    g.data_offset = c.pos + pad;
    if (g.data_offset > g.size && n_tensors) return Q4K_EFORMAT;
    for (const Tensor &t : g.tensors) {
        const uint64_t avail = g.size - g.data_offset;
        if (t.rel_offset > avail || t.nbytes > avail - t.rel_offset) return Q4K_EFORMAT;
    }
    return Q4K_OK;
}

const Kv *kv_at(const q4k_gguf *g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t)g->kvs.size()) return nullptr;
    return &g->kvs[(size_t)i];
}

template <typename T>
T read_at(const q4k_gguf *g, size_t off) {
    T v;
    std::memcpy(&v, g->map + off, sizeof(T));
    return v;
}

}  // namespace

extern "C" {

int q4k_gguf_open(const char *path, q4k_gguf **out) {
    if (!path || !out) return Q4K_EINVAL;
    *out = nullptr;
    q4k_gguf *g = new (std::nothrow) q4k_gguf();
    if (!g) return Q4K_ENOMEM;
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st {};
    if (g->fd < 0 || fstat(g->fd, &st) != 0) {
        delete g;
        return Q4K_EIO;
    }
    if (st.st_size < 24) {  // shorter than the fixed header
        delete g;
        return Q4K_EFORMAT;
    }
    g->size = (size_t)st.st_size;
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        delete g;
        return Q4K_EIO;
    }
    g->map = static_cast<const uint8_t *>(m);
    int status;
    try {
        status = parse(*g);
    } catch (const std::bad_alloc &) {
        status = Q4K_ENOMEM;
    } catch (...) {
        status = Q4K_EFORMAT;
    }
    if (status != Q4K_OK) {
        delete g;
        return status;
    }
    *out = g;
    return Q4K_OK;
}

void q4k_gguf_close(q4k_gguf *g) { delete g; }

uint32_t q4k_gguf_version(const q4k_gguf *g) { return g ? g->version : 0; }
uint64_t q4k_gguf_alignment(const q4k_gguf *g) { return g ? g->alignment : 0; }
uint64_t q4k_gguf_data_offset(const q4k_gguf *g) { return g ? g->data_offset : 0; }

int64_t q4k_gguf_tensor_count(const q4k_gguf *g) { return g ? (int64_t)g->tensors.size() : 0; }

int64_t q4k_gguf_find_tensor(const q4k_gguf *g, const char *name) {
    if (!g || !name) return -1;
    auto it = g->tensor_index.find(name);
    return it == g->tensor_index.end() ? -1 : it->second;
}

int q4k_gguf_get_tensor(const q4k_gguf *g, int64_t i, q4k_gguf_tensor_info *out) {
    if (!g || !out || i < 0 || i >= (int64_t)g->tensors.size()) return Q4K_EINVAL;
    const Tensor &t = g->tensors[(size_t)i];
    out->name = t.name.c_str();
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; ++d) out->ne[d] = t.ne[d];
    out->offset = g->data_offset + t.rel_offset;
    out->nbytes = t.nbytes;
    out->data = g->map + g->data_offset + t.rel_offset;
    return Q4K_OK;
}

uint64_t q4k_ggml_row_size(int32_t type, int64_t n) {
    const BlockSize bs = block_size(type);
    if (!bs.elems || n < 0 || n % bs.elems != 0) return 0;
    return (uint64_t)(n / bs.elems) * bs.bytes;
}

int64_t q4k_gguf_kv_count(const q4k_gguf *g) { return g ? (int64_t)g->kvs.size() : 0; }

int64_t q4k_gguf_find_key(const q4k_gguf *g, const char *key) {
    if (!g || !key) return -1;
    auto it = g->key_index.find(key);
    return it == g->key_index.end() ? -1 : it->second;
}

const char *q4k_gguf_key(const q4k_gguf *g, int64_t i) {
    const Kv *kv = kv_at(g, i);
    return kv ? kv->key.c_str() : nullptr;
}

int32_t q4k_gguf_kv_type(const q4k_gguf *g, int64_t i) {
    const Kv *kv = kv_at(g, i);
    return kv ? kv->type : -1;
}

int q4k_gguf_get_int(const q4k_gguf *g, int64_t i, int64_t *out) {
    const Kv *kv = kv_at(g, i);
    if (!kv || !out) return Q4K_EINVAL;
    const size_t o = kv->value_off;
    switch (kv->type) {
        case Q4K_GGUF_UINT8: *out = read_at<uint8_t>(g, o); return Q4K_OK;
        case Q4K_GGUF_INT8: *out = read_at<int8_t>(g, o); return Q4K_OK;
        case Q4K_GGUF_BOOL: *out = read_at<uint8_t>(g, o) != 0; return Q4K_OK;
        case Q4K_GGUF_UINT16: *out = read_at<uint16_t>(g, o); return Q4K_OK;
        case Q4K_GGUF_INT16: *out = read_at<int16_t>(g, o); return Q4K_OK;
        case Q4K_GGUF_UINT32: *out = read_at<uint32_t>(g, o); return Q4K_OK;
        case Q4K_GGUF_INT32: *out = read_at<int32_t>(g, o); return Q4K_OK;
        case Q4K_GGUF_INT64: *out = read_at<int64_t>(g, o); return Q4K_OK;
        case Q4K_GGUF_UINT64: {
            const uint64_t v = read_at<uint64_t>(g, o);
            if (v > (uint64_t)std::numeric_limits<int64_t>::max()) return Q4K_EINVAL;
            *out = (int64_t)v;
            return Q4K_OK;
        }
        default: return Q4K_EINVAL;
    }
}

int q4k_gguf_get_float(const q4k_gguf *g, int64_t i, double *out) {
    const Kv *kv = kv_at(g, i);
    if (!kv || !out) return Q4K_EINVAL;
    if (kv->type == Q4K_GGUF_FLOAT32) {
        *out = read_at<float>(g, kv->value_off);
        return Q4K_OK;
    }
    if (kv->type == Q4K_GGUF_FLOAT64) {
        *out = read_at<double>(g, kv->value_off);
        return Q4K_OK;
    }
    if (kv->type == Q4K_GGUF_UINT64) {
        *out = (double)read_at<uint64_t>(g, kv->value_off);
        return Q4K_OK;
    }
    int64_t v;
    const int st = q4k_gguf_get_int(g, i, &v);
    if (st == Q4K_OK) *out = (double)v;
    return st;
}

int q4k_gguf_get_str(const q4k_gguf *g, int64_t i, const char **out) {
    const Kv *kv = kv_at(g, i);
    if (!kv || !out || kv->type != Q4K_GGUF_STRING) return Q4K_EINVAL;
    *out = kv->str.c_str();
    return Q4K_OK;
}

int q4k_gguf_get_arr(const q4k_gguf *g, int64_t i, int32_t *elem_type, int64_t *n, const void **data) {
    const Kv *kv = kv_at(g, i);
    if (!kv || kv->type != Q4K_GGUF_ARRAY) return Q4K_EINVAL;
    if (elem_type) *elem_type = kv->elem_type;
    if (n) *n = (int64_t)kv->count;
    if (data) *data = kv->elem_type == Q4K_GGUF_STRING ? nullptr : g->map + kv->value_off;
    return Q4K_OK;
}

int q4k_gguf_get_arr_str(const q4k_gguf *g, int64_t i, int64_t j, const char **out) {
    const Kv *kv = kv_at(g, i);
    if (!kv || !out || kv->type != Q4K_GGUF_ARRAY || kv->elem_type != Q4K_GGUF_STRING) return Q4K_EINVAL;
    if (j < 0 || j >= (int64_t)kv->strs.size()) return Q4K_EINVAL;
    *out = kv->strs[(size_t)j].c_str();
    return Q4K_OK;
}

}  // extern "C"
