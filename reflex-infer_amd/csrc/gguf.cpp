// gguf.cpp -- caller-side GGUF ingest (include/rxq4_gguf.h): a read-only
// mmap of the file, a bounds-checked parse of header, metadata and tensor
// infos, and the device copy of the data section (the `weights_device` alias
// of mmap-backed weights that reflex-infer's callers pass, reference
// include/reflex/infer.h:94-95).  The reference itself parses no GGUF
// (docs/library-architecture.md:60); the format follows the GGUF
// specification (ggml docs/gguf.md, versions 2 and 3).
#include "rxq4_gguf.h"

#include <errno.h>
#include <fcntl.h>
#include <hip/hip_runtime_api.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "rxq4.h"
#include "status.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read as a little-endian uint32
constexpr uint32_t kDefaultAlignment = 32;
constexpr int kMaxDims = 4;

struct TypeInfo {
    int elems, bytes;
};

// GGML block geometry by type id (ggml.h enum ggml_type; ids 4, 5 and 31-33
// are retired and stay unknown).
TypeInfo type_info(int t) {
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
        case 34: return {256, 54};  // TQ1_0
        case 35: return {256, 66};  // TQ2_0
        default: return {0, 0};
    }
}

// Size of a scalar metadata value type; 0 for STRING / ARRAY / unknown.
int scalar_size(uint32_t t) {
    switch (t) {
        case RXQ4_GGUF_UINT8: case RXQ4_GGUF_INT8: case RXQ4_GGUF_BOOL: return 1;
        case RXQ4_GGUF_UINT16: case RXQ4_GGUF_INT16: return 2;
        case RXQ4_GGUF_UINT32: case RXQ4_GGUF_INT32: case RXQ4_GGUF_FLOAT32: return 4;
        case RXQ4_GGUF_UINT64: case RXQ4_GGUF_INT64: case RXQ4_GGUF_FLOAT64: return 8;
        default: return 0;
    }
}

struct Kv {
    std::string key;
    uint32_t type;
    uint64_t value;     // file offset of the value (for arrays: of the first element)
    uint32_t elem_type; // arrays
    uint64_t n;         // arrays: element count; strings: length
};

struct Tensor {
    std::string name;
    int type, n_dims;
    int64_t ne[kMaxDims];
    uint64_t offset, nbytes;
};

// Sequential reader over the mapping; every read is checked against the end.
struct Cursor {
    const uint8_t *base;
    uint64_t size, pos;
    const char *err = nullptr;

    bool need(uint64_t n) {
        if (err) return false;
        if (n > size - pos) {
            err = "truncated file";
            return false;
        }
        return true;
    }
    template <typename T>
    bool get(T *v) {
        if (!need(sizeof(T))) return false;
        memcpy(v, base + pos, sizeof(T));
        pos += sizeof(T);
        return true;
    }
    bool skip(uint64_t n) {
        if (!need(n)) return false;
        pos += n;
        return true;
    }
    // A GGUF string: returns the offset of its bytes and its length.
    bool str(uint64_t *off, uint64_t *len) {
        if (!get(len)) return false;
        *off = pos;
        return skip(*len);
    }
};

}  // namespace

struct rxq4_gguf {
    void *map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0, alignment = kDefaultAlignment;
    uint64_t data_off = 0;
    std::vector<Kv> kv;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> tensor_index, kv_index;

    const uint8_t *bytes() const { return static_cast<const uint8_t *>(map); }
    ~rxq4_gguf() {
        if (map) munmap(map, size);
    }
};

namespace {

int bad(const char *path, const char *what) {
    return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "rxq4_gguf_open: %s: %s", path, what);
}

// Parses the mapping of g; returns a status.
int parse(rxq4_gguf *g, const char *path) {
    Cursor c{g->bytes(), g->size, 0};
    uint32_t magic = 0;
    if (!c.get(&magic) || magic != kMagic) return bad(path, "not a GGUF file (magic)");
    if (!c.get(&g->version)) return bad(path, c.err);
    if (g->version == 1)
        return rxq4::set_error(RXQ4_STATUS_UNSUPPORTED_MODEL,
                               "rxq4_gguf_open: %s: GGUF version 1 is not supported", path);
    if (g->version != 2 && g->version != 3) {
        if ((g->version & 0xFFFFu) == 0)
            return rxq4::set_error(RXQ4_STATUS_UNSUPPORTED_MODEL,
                                   "rxq4_gguf_open: %s: big-endian GGUF is not supported", path);
        return rxq4::set_error(RXQ4_STATUS_UNSUPPORTED_MODEL,
                               "rxq4_gguf_open: %s: unknown GGUF version %u", path, g->version);
    }
    uint64_t n_tensors = 0, n_kv = 0;
    if (!c.get(&n_tensors) || !c.get(&n_kv)) return bad(path, c.err);
    // Each key/value takes at least 13 bytes and each tensor info 28: counts
    // beyond what the file can hold are corrupt (and must not size vectors).
    if (n_kv > g->size / 13 || n_tensors > g->size / 28) return bad(path, "implausible counts");

    g->kv.reserve(n_kv);
    for (uint64_t i = 0; i < n_kv; ++i) {
        Kv kv{};
        uint64_t koff, klen;
        if (!c.str(&koff, &klen) || !c.get(&kv.type)) return bad(path, c.err);
        kv.key.assign(reinterpret_cast<const char *>(g->bytes() + koff), klen);
        if (kv.type == RXQ4_GGUF_STRING) {
            uint64_t off;
            if (!c.str(&off, &kv.n)) return bad(path, c.err);
            kv.value = off;
        } else if (kv.type == RXQ4_GGUF_ARRAY) {
            if (!c.get(&kv.elem_type) || !c.get(&kv.n)) return bad(path, c.err);
            kv.value = c.pos;
            if (kv.elem_type == RXQ4_GGUF_STRING) {
                if (kv.n > (c.size - c.pos) / 8) return bad(path, "truncated string array");
                for (uint64_t j = 0; j < kv.n; ++j) {
                    uint64_t o, l;
                    if (!c.str(&o, &l)) return bad(path, c.err);
                }
            } else {
                const int es = scalar_size(kv.elem_type);
                if (es == 0) return bad(path, "array of unsupported element type");
                if (kv.n > (c.size - c.pos) / es) return bad(path, "truncated array");
                c.skip(kv.n * es);
            }
        } else {
            const int s = scalar_size(kv.type);
            if (s == 0) return bad(path, "unknown metadata value type");
            kv.value = c.pos;
            if (!c.skip(s)) return bad(path, c.err);
        }
        if (g->kv_index.count(kv.key)) return bad(path, "duplicate metadata key");
        g->kv_index.emplace(kv.key, (int64_t)g->kv.size());
        g->kv.push_back(std::move(kv));
    }

    auto al = g->kv_index.find("general.alignment");
    if (al != g->kv_index.end()) {
        const Kv &kv = g->kv[al->second];
        if (kv.type != RXQ4_GGUF_UINT32) return bad(path, "general.alignment is not a uint32");
        memcpy(&g->alignment, g->bytes() + kv.value, 4);
        if (g->alignment == 0 || (g->alignment & (g->alignment - 1)) != 0)
            return bad(path, "general.alignment is not a power of two");
    }

    g->tensors.reserve(n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Tensor t{};
        uint64_t noff, nlen;
        uint32_t n_dims = 0, type = 0;
        if (!c.str(&noff, &nlen) || !c.get(&n_dims)) return bad(path, c.err);
        t.name.assign(reinterpret_cast<const char *>(g->bytes() + noff), nlen);
        if (n_dims < 1 || n_dims > kMaxDims) return bad(path, "tensor n_dims outside 1..4");
        t.n_dims = (int)n_dims;
        for (int d = 0; d < kMaxDims; ++d) t.ne[d] = 1;
        for (uint32_t d = 0; d < n_dims; ++d) {
            uint64_t ne;
            if (!c.get(&ne)) return bad(path, c.err);
            if (ne > (uint64_t)INT64_MAX) return bad(path, "tensor dimension too large");
            t.ne[d] = (int64_t)ne;
        }
        if (!c.get(&type) || !c.get(&t.offset)) return bad(path, c.err);
        t.type = (int)type;
        const TypeInfo ti = type_info(t.type);
        if (ti.elems == 0)
            return rxq4::set_error(RXQ4_STATUS_UNSUPPORTED_QUANT_FORMAT,
                                   "rxq4_gguf_open: %s: tensor '%s' has unknown ggml type %u",
                                   path, t.name.c_str(), type);
        if (t.ne[0] % ti.elems != 0) return bad(path, "row length is not a whole number of blocks");
        // nbytes = ne0/elems*bytes*ne1*ne2*ne3 without overflow (< 2^63).
        unsigned __int128 nb = (unsigned __int128)(t.ne[0] / ti.elems) * (unsigned)ti.bytes;
        for (int d = 1; d < kMaxDims; ++d) {
            nb *= (uint64_t)t.ne[d];
            if (nb > ((unsigned __int128)1 << 62)) return bad(path, "tensor too large");
        }
        t.nbytes = (uint64_t)nb;
        if (t.offset % g->alignment != 0) return bad(path, "tensor offset is not aligned");
        if (g->tensor_index.count(t.name)) return bad(path, "duplicate tensor name");
        g->tensor_index.emplace(t.name, (int64_t)g->tensors.size());
        g->tensors.push_back(std::move(t));
    }

    // The data section starts at the next multiple of the alignment.
    const uint64_t a = g->alignment;
    const uint64_t start = (c.pos + a - 1) / a * a;
    if (start > g->size && !g->tensors.empty()) return bad(path, "truncated file");
    g->data_off = start < g->size ? start : g->size;
    const uint64_t data_size = g->size - g->data_off;
    for (const Tensor &t : g->tensors) {
        if (t.offset > data_size || t.nbytes > data_size - t.offset)
            return bad(path, "tensor data lies past the end of the file");
    }
    return rxq4::set_ok();
}

int null_handle(const char *fn) {
    return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: null handle or output", fn);
}

int kv_at(const rxq4_gguf *g, int64_t i, const char *fn, const Kv **kv) {
    if (!g) return null_handle(fn);
    if (i < 0 || i >= (int64_t)g->kv.size())
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: key index %lld out of range", fn,
                               (long long)i);
    *kv = &g->kv[i];
    return RXQ4_STATUS_SUCCESS;
}

int wrong_type(const char *fn, const Kv &kv) {
    return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: key '%s' has value type %u", fn,
                           kv.key.c_str(), kv.type);
}

}  // namespace

extern "C" {

int rxq4_ggml_block_elems(int t) { return type_info(t).elems; }
int rxq4_ggml_block_bytes(int t) { return type_info(t).bytes; }

int rxq4_gguf_open(const char *path, rxq4_gguf **out) {
    if (!path || !out)
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "rxq4_gguf_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return bad(path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int e = errno;
        close(fd);
        return bad(path, strerror(e));
    }
    auto *g = new rxq4_gguf();
    g->size = (uint64_t)st.st_size;
    if (g->size > 0) {
        void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            const int e = errno;
            close(fd);
            delete g;
            return bad(path, strerror(e));
        }
        g->map = m;
    }
    close(fd);
    const int s = parse(g, path);
    if (s != RXQ4_STATUS_SUCCESS) {
        delete g;
        return s;
    }
    *out = g;
    return RXQ4_STATUS_SUCCESS;
}

void rxq4_gguf_close(rxq4_gguf *g) { delete g; }

uint32_t rxq4_gguf_version(const rxq4_gguf *g) { return g ? g->version : 0; }
uint32_t rxq4_gguf_alignment(const rxq4_gguf *g) { return g ? g->alignment : 0; }
int64_t rxq4_gguf_n_tensors(const rxq4_gguf *g) { return g ? (int64_t)g->tensors.size() : 0; }
int64_t rxq4_gguf_n_kv(const rxq4_gguf *g) { return g ? (int64_t)g->kv.size() : 0; }
const void *rxq4_gguf_data(const rxq4_gguf *g) { return g ? g->bytes() + g->data_off : nullptr; }
uint64_t rxq4_gguf_data_bytes(const rxq4_gguf *g) { return g ? g->size - g->data_off : 0; }

int rxq4_gguf_tensor_info(const rxq4_gguf *g, int64_t i, rxq4_gguf_tensor *out) {
    if (!g || !out) return null_handle("rxq4_gguf_tensor_info");
    if (i < 0 || i >= (int64_t)g->tensors.size())
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT,
                               "rxq4_gguf_tensor_info: index %lld out of range", (long long)i);
    const Tensor &t = g->tensors[i];
    out->name = t.name.c_str();
    out->ggml_type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < kMaxDims; ++d) out->ne[d] = t.ne[d];
    out->offset = t.offset;
    out->nbytes = t.nbytes;
    out->host = g->bytes() + g->data_off + t.offset;
    return rxq4::set_ok();
}

int64_t rxq4_gguf_find_tensor(const rxq4_gguf *g, const char *name) {
    if (!g || !name) return -1;
    auto it = g->tensor_index.find(name);
    return it == g->tensor_index.end() ? -1 : it->second;
}

int64_t rxq4_gguf_find_kv(const rxq4_gguf *g, const char *key) {
    if (!g || !key) return -1;
    auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? -1 : it->second;
}

int rxq4_gguf_kv_key(const rxq4_gguf *g, int64_t i, const char **key, int *type) {
    const Kv *kv = nullptr;
    int s = kv_at(g, i, "rxq4_gguf_kv_key", &kv);
    if (s != RXQ4_STATUS_SUCCESS) return s;
    if (key) *key = kv->key.c_str();
    if (type) *type = (int)kv->type;
    return rxq4::set_ok();
}

int rxq4_gguf_kv_int(const rxq4_gguf *g, int64_t i, int64_t *out) {
    const char *fn = "rxq4_gguf_kv_int";
    const Kv *kv = nullptr;
    int s = kv_at(g, i, fn, &kv);
    if (s != RXQ4_STATUS_SUCCESS) return s;
    if (!out) return null_handle(fn);
    const uint8_t *p = g->bytes() + kv->value;
    switch (kv->type) {
        case RXQ4_GGUF_UINT8: *out = *p; break;
        case RXQ4_GGUF_BOOL: *out = *p != 0; break;
        case RXQ4_GGUF_INT8: *out = (int8_t)*p; break;
        case RXQ4_GGUF_UINT16: { uint16_t v; memcpy(&v, p, 2); *out = v; break; }
        case RXQ4_GGUF_INT16: { int16_t v; memcpy(&v, p, 2); *out = v; break; }
        case RXQ4_GGUF_UINT32: { uint32_t v; memcpy(&v, p, 4); *out = v; break; }
        case RXQ4_GGUF_INT32: { int32_t v; memcpy(&v, p, 4); *out = v; break; }
        case RXQ4_GGUF_INT64: { int64_t v; memcpy(&v, p, 8); *out = v; break; }
        case RXQ4_GGUF_UINT64: {
            uint64_t v;
            memcpy(&v, p, 8);
            if (v > (uint64_t)INT64_MAX)
                return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT,
                                       "%s: key '%s' does not fit int64", fn, kv->key.c_str());
            *out = (int64_t)v;
            break;
        }
        default: return wrong_type(fn, *kv);
    }
    return rxq4::set_ok();
}

int rxq4_gguf_kv_float(const rxq4_gguf *g, int64_t i, double *out) {
    const char *fn = "rxq4_gguf_kv_float";
    const Kv *kv = nullptr;
    int s = kv_at(g, i, fn, &kv);
    if (s != RXQ4_STATUS_SUCCESS) return s;
    if (!out) return null_handle(fn);
    const uint8_t *p = g->bytes() + kv->value;
    if (kv->type == RXQ4_GGUF_FLOAT32) {
        float v;
        memcpy(&v, p, 4);
        *out = v;
    } else if (kv->type == RXQ4_GGUF_FLOAT64) {
        memcpy(out, p, 8);
    } else {
        return wrong_type(fn, *kv);
    }
    return rxq4::set_ok();
}

int rxq4_gguf_kv_str(const rxq4_gguf *g, int64_t i, const char **str, uint64_t *len) {
    const char *fn = "rxq4_gguf_kv_str";
    const Kv *kv = nullptr;
    int s = kv_at(g, i, fn, &kv);
    if (s != RXQ4_STATUS_SUCCESS) return s;
    if (!str || !len) return null_handle(fn);
    if (kv->type != RXQ4_GGUF_STRING) return wrong_type(fn, *kv);
    *str = reinterpret_cast<const char *>(g->bytes() + kv->value);
    *len = kv->n;
    return rxq4::set_ok();
}

int rxq4_gguf_kv_array(const rxq4_gguf *g, int64_t i, int *elem_type, uint64_t *n,
                       const void **data) {
    const char *fn = "rxq4_gguf_kv_array";
    const Kv *kv = nullptr;
    int s = kv_at(g, i, fn, &kv);
    if (s != RXQ4_STATUS_SUCCESS) return s;
    if (kv->type != RXQ4_GGUF_ARRAY) return wrong_type(fn, *kv);
    if (elem_type) *elem_type = (int)kv->elem_type;
    if (n) *n = kv->n;
    if (data) *data = kv->elem_type == RXQ4_GGUF_STRING ? nullptr : g->bytes() + kv->value;
    return rxq4::set_ok();
}

int rxq4_gguf_kv_array_strs(const rxq4_gguf *g, int64_t i, uint64_t first, uint64_t count,
                            const char **str, uint64_t *len) {
    const char *fn = "rxq4_gguf_kv_array_strs";
    const Kv *kv = nullptr;
    int s = kv_at(g, i, fn, &kv);
    if (s != RXQ4_STATUS_SUCCESS) return s;
    if (count > 0 && (!str || !len)) return null_handle(fn);
    if (kv->type != RXQ4_GGUF_ARRAY || kv->elem_type != RXQ4_GGUF_STRING)
        return wrong_type(fn, *kv);
    if (first > kv->n || count > kv->n - first)
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: elements [%llu, +%llu) of %llu",
                               fn, (unsigned long long)first, (unsigned long long)count,
                               (unsigned long long)kv->n);
    // The parse validated every length of the array.
    uint64_t pos = kv->value, l = 0;
    for (uint64_t k = 0; k < first + count; ++k) {
        memcpy(&l, g->bytes() + pos, 8);
        if (k >= first) {
            str[k - first] = reinterpret_cast<const char *>(g->bytes() + pos + 8);
            len[k - first] = l;
        }
        pos += 8 + l;
    }
    return rxq4::set_ok();
}

int rxq4_gguf_upload(const rxq4_gguf *g, void *dst, uint64_t dst_bytes, void *stream) {
    const char *fn = "rxq4_gguf_upload";
    if (!g || !dst) return null_handle(fn);
    const uint64_t n = rxq4_gguf_data_bytes(g);
    if (dst_bytes < n)
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT,
                               "%s: destination holds %llu bytes, the data section %llu", fn,
                               (unsigned long long)dst_bytes, (unsigned long long)n);
    if ((reinterpret_cast<uintptr_t>(dst) & 255u) != 0)
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: destination not 256-byte aligned",
                               fn);
    if (n == 0) return rxq4::set_ok();
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, dst) != hipSuccess ||
        (attr.type != hipMemoryTypeDevice && attr.type != hipMemoryTypeManaged)) {
        (void)hipGetLastError();
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: destination is not device memory",
                               fn);
    }
    // Two pinned staging buffers: the host copy into one overlaps the DMA
    // out of the other.  (Registering the mapping itself would avoid the
    // host copy, but pinning existing pages is not used on this platform.)
    constexpr uint64_t kChunk = 32ull << 20;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    hipError_t e = hipSuccess;
    for (int b = 0; b < 2 && e == hipSuccess; ++b) {
        e = hipHostMalloc(&stage[b], kChunk, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&done[b], hipEventDisableTiming);
    }
    const uint8_t *src = static_cast<const uint8_t *>(rxq4_gguf_data(g));
    uint8_t *out = static_cast<uint8_t *>(dst);
    bool used[2] = {false, false};
    for (uint64_t off = 0, k = 0; e == hipSuccess && off < n; off += kChunk, ++k) {
        const int b = (int)(k & 1);
        const uint64_t len = n - off < kChunk ? n - off : kChunk;
        if (used[b]) e = hipEventSynchronize(done[b]);
        if (e != hipSuccess) break;
        memcpy(stage[b], src + off, len);
        e = hipMemcpyAsync(out + off, stage[b], len, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipEventRecord(done[b], st);
        used[b] = true;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    for (int b = 0; b < 2; ++b) {
        if (done[b]) (void)hipEventDestroy(done[b]);
        if (stage[b]) (void)hipHostFree(stage[b]);
    }
    if (e != hipSuccess)
        return rxq4::set_error(RXQ4_STATUS_INVALID_ARGUMENT, "%s: HIP error %s", fn,
                               hipGetErrorString(e));
    return rxq4::set_ok();
}

}  // extern "C"
