// GGUF wire-byte reader (host code): the C++ half of kq.load_gguf
// (gmlx/loader.py:92-142) and of the fast header scan (gmlx/headerscan.py:
// 122-176).
//
// The file is mapped read-only once; the header, every metadata entry and
// the tensor table are parsed into index arrays that point into the
// mapping, so metadata values and tensor bytes are read in place (a tensor's
// bytes are the GGUF wire bytes the kernels consume unchanged).  Every read
// is bounds-checked against the file size: a malformed or hostile header
// fails with KQ_ERR_BAD_FORMAT, never reads outside the mapping.  A file
// cut short inside the tensor data still opens (its header is whole);
// kq_gguf_header reports the size the tensor table implies, and a tensor
// whose bytes lie past the end has data == NULL.
//
// Format (GGUF v2 / v3, little-endian): "GGUF", u32 version, u64 tensor
// count, u64 metadata count; metadata entries (string key, u32 value type,
// value); tensor infos (string name, u32 n_dims, u64 dims[n_dims], u32 ggml
// type, u64 offset); padding to general.alignment (default 32); tensor data.
// A string is a u64 byte length and the bytes; an array is a u32 element
// type, a u64 count and the elements.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <new>
#include <vector>

#include "kq_common.h"
#include "../../include/kq_gguf.h"

namespace {

enum : uint32_t {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STRING = 8, V_ARRAY = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12,
};

int scalar_size(uint32_t t) {
    switch (t) {
    case V_U8: case V_I8: case V_BOOL: return 1;
    case V_U16: case V_I16: return 2;
    case V_U32: case V_I32: case V_F32: return 4;
    case V_U64: case V_I64: case V_F64: return 8;
    default: return 0;
    }
}

// (values per block, bytes per block) of the ggml tensor types, from the
// public GGML type table; {0, 0} for ids that are unassigned or retired.
struct TypeSize {
    int32_t block, bytes;
};
constexpr TypeSize kTypes[] = {
    {1, 4},      // 0  F32
    {1, 2},      // 1  F16
    {32, 18},    // 2  Q4_0
    {32, 20},    // 3  Q4_1
    {0, 0},      // 4  (retired)
    {0, 0},      // 5  (retired)
    {32, 22},    // 6  Q5_0
    {32, 24},    // 7  Q5_1
    {32, 34},    // 8  Q8_0
    {32, 36},    // 9  Q8_1
    {256, 84},   // 10 Q2_K
    {256, 110},  // 11 Q3_K
    {256, 144},  // 12 Q4_K
    {256, 176},  // 13 Q5_K
    {256, 210},  // 14 Q6_K
    {256, 292},  // 15 Q8_K
    {256, 66},   // 16 IQ2_XXS
    {256, 74},   // 17 IQ2_XS
    {256, 98},   // 18 IQ3_XXS
    {256, 50},   // 19 IQ1_S
    {32, 18},    // 20 IQ4_NL
    {256, 110},  // 21 IQ3_S
    {256, 82},   // 22 IQ2_S
    {256, 136},  // 23 IQ4_XS
    {1, 1},      // 24 I8
    {1, 2},      // 25 I16
    {1, 4},      // 26 I32
    {1, 8},      // 27 I64
    {1, 8},      // 28 F64
    {256, 56},   // 29 IQ1_M
    {1, 2},      // 30 BF16
    {0, 0},      // 31 (retired)
    {0, 0},      // 32 (retired)
    {0, 0},      // 33 (retired)
    {256, 54},   // 34 TQ1_0
    {256, 66},   // 35 TQ2_0
    {0, 0},      // 36 (retired)
    {0, 0},      // 37 (retired)
    {0, 0},      // 38 (retired)
    {32, 17},    // 39 MXFP4
};
constexpr uint32_t kNumTypes = sizeof(kTypes) / sizeof(kTypes[0]);

struct Kv {
    const char *key;
    int64_t key_len;
    uint32_t type, elem_type;
    int64_t count;  // 1 for scalars, bytes for a string, elements for an array
    const uint8_t *data;
};

struct Tensor {
    const char *name;
    int64_t name_len;
    uint32_t n_dims;
    int64_t dims[4];
    uint32_t type;
    int64_t offset, nbytes;
};

// Bounds-checked little-endian reader over the mapping.
struct Cursor {
    const uint8_t *base;
    uint64_t size, off;
    bool ok = true;
    bool need(uint64_t n) {
        if (!ok || n > size - off) ok = false;
        return ok;
    }
    template <class T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, base + off, sizeof(T));
            off += sizeof(T);
        }
        return v;
    }
    // string: returns its bytes, advances past it
    const char *str(int64_t *len) {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return nullptr;
        const char *p = (const char *)(base + off);
        off += n;
        *len = (int64_t)n;
        return p;
    }
    // skip one value of type t (nested arrays allowed up to `depth`)
    bool skip(uint32_t t, int depth) {
        if (const int s = scalar_size(t)) return need(s) && (off += s, true);
        if (t == V_STRING) {
            int64_t n;
            return str(&n) != nullptr || (ok && n == 0);
        }
        if (t == V_ARRAY) {
            if (depth <= 0) return ok = false;
            const uint32_t et = get<uint32_t>();
            const uint64_t count = get<uint64_t>();
            if (!ok) return false;
            if (const int s = scalar_size(et)) {
                if (count > (size - off) / (uint64_t)s) return ok = false;
                off += count * s;
                return true;
            }
            if (et != V_STRING && et != V_ARRAY) return ok = false;
            // every element takes at least 8 bytes
            if (count > (size - off) / 8) return ok = false;
            for (uint64_t i = 0; i < count; ++i)
                if (!skip(et, depth - 1)) return false;
            return true;
        }
        return ok = false;
    }
};

}  // namespace

struct kq_gguf {
    const uint8_t *base = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    int64_t data_offset = 0, alignment = 32, expected_size = 0;
    std::vector<Kv> kv;
    std::vector<Tensor> tensors;
};

namespace {

int parse(kq_gguf *g) {
    Cursor c{g->base, g->size, 0};
    if (g->size < 24 || std::memcmp(g->base, "GGUF", 4) != 0) return KQ_ERR_BAD_FORMAT;
    c.off = 4;
    g->version = c.get<uint32_t>();
    const uint64_t n_tensors = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    if (g->version < 2 || g->version > 3) return KQ_ERR_BAD_FORMAT;
    // each metadata entry and tensor info takes at least 16 bytes
    if (n_kv > g->size / 16 || n_tensors > g->size / 16) return KQ_ERR_BAD_FORMAT;
    g->kv.reserve(n_kv);
    for (uint64_t i = 0; i < n_kv; ++i) {
        Kv e{};
        e.key = c.str(&e.key_len);
        e.type = c.get<uint32_t>();
        if (!c.ok) return KQ_ERR_BAD_FORMAT;
        if (const int s = scalar_size(e.type)) {
            if (!c.need(s)) return KQ_ERR_BAD_FORMAT;
            e.count = 1;
            e.data = g->base + c.off;
            c.off += s;
        } else if (e.type == V_STRING) {
            int64_t n = 0;
            const char *p = c.str(&n);
            if (!c.ok) return KQ_ERR_BAD_FORMAT;
            e.count = n;
            e.data = (const uint8_t *)p;
        } else if (e.type == V_ARRAY) {
            e.elem_type = c.get<uint32_t>();
            const uint64_t count = c.get<uint64_t>();
            if (!c.ok || count > (uint64_t)INT64_MAX) return KQ_ERR_BAD_FORMAT;
            e.count = (int64_t)count;
            e.data = g->base + c.off;
            if (const int s = scalar_size(e.elem_type)) {
                if (count > (g->size - c.off) / (uint64_t)s) return KQ_ERR_BAD_FORMAT;
                c.off += count * s;
            } else if (e.elem_type == V_STRING || e.elem_type == V_ARRAY) {
                if (count > (g->size - c.off) / 8) return KQ_ERR_BAD_FORMAT;
                for (uint64_t j = 0; j < count; ++j)
                    if (!c.skip(e.elem_type, 8)) return KQ_ERR_BAD_FORMAT;
            } else {
                return KQ_ERR_BAD_FORMAT;
            }
        } else {
            return KQ_ERR_BAD_FORMAT;
        }
        if (e.key_len == 17 && std::memcmp(e.key, "general.alignment", 17) == 0) {
            if (e.type != V_U32) return KQ_ERR_BAD_FORMAT;
            uint32_t a;
            std::memcpy(&a, e.data, 4);
            if (a == 0 || (a & (a - 1))) return KQ_ERR_BAD_FORMAT;
            g->alignment = a;
        }
        g->kv.push_back(e);
    }
    g->tensors.reserve(n_tensors);
    int64_t end = 0;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Tensor t{};
        t.name = c.str(&t.name_len);
        t.n_dims = c.get<uint32_t>();
        if (!c.ok || t.n_dims == 0 || t.n_dims > 4) return KQ_ERR_BAD_FORMAT;
        uint64_t n = 1;
        for (uint32_t d = 0; d < 4; ++d) {
            const uint64_t v = d < t.n_dims ? c.get<uint64_t>() : 1;
            if (!c.ok || v > (uint64_t)INT64_MAX || (v && n > (uint64_t)INT64_MAX / v)) return KQ_ERR_BAD_FORMAT;
            n *= v;
            t.dims[d] = (int64_t)v;
        }
        t.type = c.get<uint32_t>();
        const uint64_t off = c.get<uint64_t>();
        if (!c.ok || t.type >= kNumTypes || kTypes[t.type].block == 0) return KQ_ERR_BAD_FORMAT;
        const TypeSize ts = kTypes[t.type];
        if (t.dims[0] % ts.block) return KQ_ERR_BAD_FORMAT;  // rows hold whole blocks
        if (n / ts.block > (uint64_t)INT64_MAX / ts.bytes) return KQ_ERR_BAD_FORMAT;
        t.nbytes = (int64_t)(n / ts.block * ts.bytes);
        if (off > (uint64_t)INT64_MAX - (uint64_t)t.nbytes || off % (uint64_t)g->alignment) return KQ_ERR_BAD_FORMAT;
        t.offset = (int64_t)off;
        if (t.offset + t.nbytes > end) end = t.offset + t.nbytes;
        g->tensors.push_back(t);
    }
    g->data_offset = (int64_t)((c.off + g->alignment - 1) / g->alignment * g->alignment);
    if (end > INT64_MAX - g->data_offset) return KQ_ERR_BAD_FORMAT;
    g->expected_size = n_tensors ? g->data_offset + end : 0;
    return KQ_OK;
}

}  // namespace

extern "C" {

int kq_gguf_open(const char *path, kq_gguf **out) {
    if (!path || !out) return KQ_ERR_NULL_POINTER;
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return KQ_ERR_IO;
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return st.st_size == 0 ? KQ_ERR_BAD_FORMAT : KQ_ERR_IO;
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return KQ_ERR_IO;
    kq_gguf *g = new (std::nothrow) kq_gguf;
    if (!g) {
        munmap(m, (size_t)st.st_size);
        return KQ_ERR_IO;
    }
    g->base = (const uint8_t *)m;
    g->size = (uint64_t)st.st_size;
    int rc;
    try {
        rc = parse(g);
    } catch (const std::bad_alloc &) {
        rc = KQ_ERR_BAD_FORMAT;
    }
    if (rc != KQ_OK) {
        kq_gguf_close(g);
        return rc;
    }
    *out = g;
    return KQ_OK;
}

void kq_gguf_close(kq_gguf *g) {
    if (!g) return;
    if (g->base) munmap(const_cast<uint8_t *>(g->base), (size_t)g->size);
    delete g;
}

int kq_gguf_header(const kq_gguf *g, uint32_t *version, int64_t *n_tensors, int64_t *n_kv, int64_t *data_offset,
                   int64_t *alignment, int64_t *file_size, int64_t *expected_size) {
    if (!g) return KQ_ERR_NULL_POINTER;
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = (int64_t)g->tensors.size();
    if (n_kv) *n_kv = (int64_t)g->kv.size();
    if (data_offset) *data_offset = g->data_offset;
    if (alignment) *alignment = g->alignment;
    if (file_size) *file_size = (int64_t)g->size;
    if (expected_size) *expected_size = g->expected_size;
    return KQ_OK;
}

int kq_gguf_kv(const kq_gguf *g, int64_t i, const char **key, int64_t *key_len, uint32_t *type,
               uint32_t *elem_type, int64_t *count, const void **data) {
    if (!g) return KQ_ERR_NULL_POINTER;
    if (i < 0 || i >= (int64_t)g->kv.size()) return KQ_ERR_BAD_ARGUMENT;
    const Kv &e = g->kv[(size_t)i];
    if (key) *key = e.key;
    if (key_len) *key_len = e.key_len;
    if (type) *type = e.type;
    if (elem_type) *elem_type = e.elem_type;
    if (count) *count = e.count;
    if (data) *data = e.data;
    return KQ_OK;
}

int kq_gguf_tensor(const kq_gguf *g, int64_t i, const char **name, int64_t *name_len, uint32_t *n_dims,
                   int64_t *dims, uint32_t *ggml_type, int64_t *offset, int64_t *nbytes, const void **data) {
    if (!g) return KQ_ERR_NULL_POINTER;
    if (i < 0 || i >= (int64_t)g->tensors.size()) return KQ_ERR_BAD_ARGUMENT;
    const Tensor &t = g->tensors[(size_t)i];
    if (name) *name = t.name;
    if (name_len) *name_len = t.name_len;
    if (n_dims) *n_dims = t.n_dims;
    if (dims)
        for (int d = 0; d < 4; ++d) dims[d] = t.dims[d];
    if (ggml_type) *ggml_type = t.type;
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    if (data) {
        const int64_t at = g->data_offset + t.offset;
        *data = (at + t.nbytes <= (int64_t)g->size) ? (const void *)(g->base + at) : nullptr;
    }
    return KQ_OK;
}

int kq_gguf_type_size(uint32_t ggml_type, int32_t *block, int32_t *bytes) {
    if (ggml_type >= kNumTypes || kTypes[ggml_type].block == 0) return KQ_ERR_UNSUPPORTED_CODEC;
    if (block) *block = kTypes[ggml_type].block;
    if (bytes) *bytes = kTypes[ggml_type].bytes;
    return KQ_OK;
}

}  // extern "C"
