// GGUF v2/v3 container reader and HBM upload (host code of libmaxuna_moe).
//
// Replaces what the reference host gets from candle's gguf_file::Content and
// its own loaders (src/gguf.rs:554-658 expert stacks, :676-687 bias-suffixed
// f32 tensors, config.rs:115-130 metadata): the header, the typed metadata, the
// tensor table and the data section are parsed from the public GGUF layout:
//
//   magic "GGUF" | u32 version | u64 n_tensors | u64 n_kv
//   n_kv x  { string key | u32 type | value }
//   n_tensors x { string name | u32 n_dims | u64 ne[n_dims] | u32 ggml_type | u64 offset }
//   padding to general.alignment (default 32) | tensor data (offsets relative to here)
//
// string = u64 length + bytes; array = u32 element type + u64 count + elements.
// All integers little-endian.  Every length and offset is checked against the
// file size before use: a malformed file gives MX_ERR_FORMAT, never a read
// past the end.
//
// The reference aliases tensor bytes zero-copy out of an mmap (Apple unified
// memory).  The MI355X equivalent moves them into HBM once: the file is read
// in chunks into two pinned host buffers while the previous chunk's DMA to the
// device runs (mx_gguf_read), so the upload runs at the slower of the file
// read and the PCIe copy.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include <hip/hip_runtime.h>

#include "../../include/maxuna_moe.h"

namespace mx {
mx_status fail(mx_status code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
mx_status hip_check(hipError_t e, const char *what);
}  // namespace mx

using mx::fail;

#define MX_HIP_G(expr)                                    \
    do {                                                  \
        const hipError_t e_ = (expr);                     \
        if (e_ != hipSuccess) return mx::hip_check(e_, #expr); \
    } while (0)

namespace {

enum : uint32_t {
    T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
    T_STRING = 8, T_ARRAY = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12,
};

// (block size, type size) of the ggml types; {0, 0} if unknown
struct TypeGeom {
    int64_t block, size;
};
TypeGeom ggml_geom(uint32_t t) {
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
    case 24: return {1, 1};     // I8
    case 25: return {1, 2};     // I16
    case 26: return {1, 4};     // I32
    case 27: return {1, 8};     // I64
    case 28: return {1, 8};     // F64
    case 30: return {1, 2};     // BF16
    default: return {0, 0};
    }
}

int64_t scalar_size(uint32_t t) {
    switch (t) {
    case T_U8: case T_I8: case T_BOOL: return 1;
    case T_U16: case T_I16: return 2;
    case T_U32: case T_I32: case T_F32: return 4;
    case T_U64: case T_I64: case T_F64: return 8;
    default: return 0;
    }
}

struct Kv {
    uint32_t type;
    uint64_t pos;         // file offset of the value (after the type word)
    uint32_t elem_type;   // arrays
    uint64_t count;       // arrays
    std::string str;      // strings
};

}  // namespace

struct mx_gguf {
    int fd = -1;
    uint64_t file_size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_offset = 0;
    std::vector<std::string> names;
    std::vector<mx_gguf_tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
    std::unordered_map<std::string, Kv> kv;
    // pinned staging for mx_gguf_read (allocated on first use)
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    size_t stage_bytes = 0;
};

namespace {

// Bounded sequential reader over the file (pread; no mmap of multi-GB files).
struct Cursor {
    int fd;
    uint64_t pos, end;
    mx_status err = MX_OK;
    bool read(void *dst, uint64_t n) {
        if (err) return false;
        if (n > end - pos) {
            err = fail(MX_ERR_FORMAT, "gguf: truncated file (need %llu bytes at offset %llu, size %llu)",
                       (unsigned long long)n, (unsigned long long)pos, (unsigned long long)end);
            return false;
        }
        uint8_t *d = static_cast<uint8_t *>(dst);
        uint64_t done = 0;
        while (done < n) {
            const ssize_t r = pread(fd, d + done, n - done, (off_t)(pos + done));
            if (r <= 0) {
                err = fail(MX_ERR_IO, "gguf: read failed at offset %llu", (unsigned long long)(pos + done));
                return false;
            }
            done += (uint64_t)r;
        }
        pos += n;
        return true;
    }
    template <class T> bool get(T &v) { return read(&v, sizeof v); }
    bool skip(uint64_t n) {
        if (err) return false;
        if (n > end - pos) {
            err = fail(MX_ERR_FORMAT, "gguf: truncated file (skip %llu at %llu)", (unsigned long long)n,
                       (unsigned long long)pos);
            return false;
        }
        pos += n;
        return true;
    }
    bool string(std::string &s) {
        uint64_t n;
        if (!get(n)) return false;
        if (n > end - pos || n > (1u << 30)) {
            err = fail(MX_ERR_FORMAT, "gguf: string of %llu bytes at offset %llu runs past the file",
                       (unsigned long long)n, (unsigned long long)pos);
            return false;
        }
        s.resize(n);
        return n == 0 || read(&s[0], n);
    }
    // skips one value of `type` (arrays recursively, bounded depth)
    bool skip_value(uint32_t type, int depth = 0) {
        if (type == T_STRING) {
            uint64_t n;
            return get(n) && skip(n);
        }
        if (type == T_ARRAY) {
            uint32_t et;
            uint64_t cnt;
            if (!get(et) || !get(cnt)) return false;
            if (depth > 4) {
                err = fail(MX_ERR_FORMAT, "gguf: arrays nested too deeply");
                return false;
            }
            const int64_t es = scalar_size(et);
            if (es) {
                if (cnt > (end - pos) / (uint64_t)es) {
                    err = fail(MX_ERR_FORMAT, "gguf: array of %llu elements runs past the file",
                               (unsigned long long)cnt);
                    return false;
                }
                return skip(cnt * (uint64_t)es);
            }
            for (uint64_t i = 0; i < cnt; i++)
                if (!skip_value(et, depth + 1)) return false;
            return true;
        }
        const int64_t sz = scalar_size(type);
        if (!sz) {
            err = fail(MX_ERR_FORMAT, "gguf: unknown metadata value type %u", type);
            return false;
        }
        return skip((uint64_t)sz);
    }
};

mx_status parse(mx_gguf *g) {
    Cursor c{g->fd, 0, g->file_size};
    char magic[4];
    if (!c.read(magic, 4)) return c.err;
    if (memcmp(magic, "GGUF", 4) != 0) return fail(MX_ERR_FORMAT, "gguf: bad magic (not a GGUF file)");
    if (!c.get(g->version)) return c.err;
    if (g->version < 2 || g->version > 3)
        return fail(MX_ERR_FORMAT, "gguf: version %u not supported (2 or 3)", g->version);
    uint64_t n_tensors, n_kv;
    if (!c.get(n_tensors) || !c.get(n_kv)) return c.err;
    if (n_tensors > (1u << 24) || n_kv > (1u << 24))
        return fail(MX_ERR_FORMAT, "gguf: implausible counts (%llu tensors, %llu kv)",
                    (unsigned long long)n_tensors, (unsigned long long)n_kv);
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key;
        Kv v{};
        if (!c.string(key) || !c.get(v.type)) return c.err;
        v.pos = c.pos;
        if (v.type == T_STRING) {
            if (!c.string(v.str)) return c.err;
        } else if (v.type == T_ARRAY) {
            if (!c.get(v.elem_type) || !c.get(v.count)) return c.err;
            c.pos = v.pos;
            if (!c.skip_value(T_ARRAY)) return c.err;
        } else if (!c.skip_value(v.type)) {
            return c.err;
        }
        g->kv[key] = std::move(v);
    }
    auto al = g->kv.find("general.alignment");
    if (al != g->kv.end()) {
        if (al->second.type != T_U32) return fail(MX_ERR_FORMAT, "gguf: general.alignment is not a u32");
        uint32_t a;
        Cursor ac{g->fd, al->second.pos, g->file_size};
        if (!ac.get(a)) return ac.err;
        if (a == 0 || (a & (a - 1))) return fail(MX_ERR_FORMAT, "gguf: alignment %u is not a power of two", a);
        g->alignment = a;
    }
    g->names.resize(n_tensors);
    g->tensors.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        mx_gguf_tensor &t = g->tensors[i];
        memset(&t, 0, sizeof t);
        uint32_t nd;
        if (!c.string(g->names[i]) || !c.get(nd)) return c.err;
        if (nd == 0 || nd > 4) return fail(MX_ERR_FORMAT, "gguf: tensor %s has %u dims", g->names[i].c_str(), nd);
        t.n_dims = (int32_t)nd;
        for (int d = 0; d < 4; d++) t.ne[d] = 1;
        for (uint32_t d = 0; d < nd; d++) {
            uint64_t ne;
            if (!c.get(ne)) return c.err;
            if (ne == 0 || ne > ((uint64_t)1 << 40))
                return fail(MX_ERR_FORMAT, "gguf: tensor %s dim %u = %llu", g->names[i].c_str(), d,
                            (unsigned long long)ne);
            t.ne[d] = (int64_t)ne;
        }
        uint32_t type;
        uint64_t off;
        if (!c.get(type) || !c.get(off)) return c.err;
        t.ggml_type = (int32_t)type;
        t.offset = off;  // relative for now
        const TypeGeom tg = ggml_geom(type);
        // element count, dimension by dimension, rejected as soon as it passes 2^62
        // (four 2^40 dimensions would overflow even a 128-bit product)
        unsigned __int128 n = 1;
        for (int d = 0; d < 4; d++) {
            n *= (uint64_t)t.ne[d];
            if (n > ((unsigned __int128)1 << 62))
                return fail(MX_ERR_FORMAT, "gguf: tensor %s has more than 2^62 elements", g->names[i].c_str());
        }
        if (tg.block) {
            if (t.ne[0] % tg.block)
                return fail(MX_ERR_FORMAT, "gguf: tensor %s row of %lld is not a multiple of its block size %lld",
                            g->names[i].c_str(), (long long)t.ne[0], (long long)tg.block);
            const unsigned __int128 bytes = n / tg.block * tg.size;
            if (bytes > ((unsigned __int128)1 << 62)) return fail(MX_ERR_FORMAT, "gguf: tensor %s too large", g->names[i].c_str());
            t.nbytes = (uint64_t)bytes;
        }
        if (!g->by_name.emplace(g->names[i], i).second)
            return fail(MX_ERR_FORMAT, "gguf: duplicate tensor name %s", g->names[i].c_str());
    }
    g->data_offset = (c.pos + g->alignment - 1) / g->alignment * g->alignment;
    for (uint64_t i = 0; i < n_tensors; i++) {
        mx_gguf_tensor &t = g->tensors[i];
        if (t.offset % g->alignment)
            return fail(MX_ERR_FORMAT, "gguf: tensor %s offset %llu is not %llu-aligned", g->names[i].c_str(),
                        (unsigned long long)t.offset, (unsigned long long)g->alignment);
        if (t.offset > g->file_size || g->data_offset > g->file_size - t.offset ||
            t.nbytes > g->file_size - g->data_offset - t.offset)
            return fail(MX_ERR_FORMAT, "gguf: tensor %s data [%llu, +%llu) runs past the file (%llu bytes)",
                        g->names[i].c_str(), (unsigned long long)(g->data_offset + t.offset),
                        (unsigned long long)t.nbytes, (unsigned long long)g->file_size);
        t.offset += g->data_offset;
        t.name = g->names[i].c_str();
    }
    return MX_OK;
}

const Kv *find_kv(const mx_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    auto it = g->kv.find(key);
    return it == g->kv.end() ? nullptr : &it->second;
}

}  // namespace

extern "C" {

mx_status mx_gguf_open(const char *path, mx_gguf **out) {
    if (!path || !out) return fail(MX_ERR_NULL, "gguf_open: NULL argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(MX_ERR_IO, "gguf_open: cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return fail(MX_ERR_IO, "gguf_open: cannot stat %s", path);
    }
    mx_gguf *g = new (std::nothrow) mx_gguf;
    if (!g) {
        close(fd);
        return fail(MX_ERR_IO, "gguf_open: out of host memory");
    }
    g->fd = fd;
    g->file_size = (uint64_t)st.st_size;
    mx_status s;
    try {
        s = parse(g);
    } catch (...) {  // std::bad_alloc from a hostile table
        s = fail(MX_ERR_FORMAT, "gguf_open: out of host memory while parsing %s", path);
    }
    if (s != MX_OK) {
        mx_gguf_close(g);
        return s;
    }
    *out = g;
    return MX_OK;
}

void mx_gguf_close(mx_gguf *g) {
    if (!g) return;
    for (int i = 0; i < 2; i++) {
        if (g->done[i]) (void)hipEventDestroy(g->done[i]);
        if (g->stage[i]) (void)hipHostFree(g->stage[i]);
    }
    if (g->fd >= 0) close(g->fd);
    delete g;
}

uint32_t mx_gguf_version(const mx_gguf *g) { return g ? g->version : 0; }
uint64_t mx_gguf_alignment(const mx_gguf *g) { return g ? g->alignment : 0; }
uint64_t mx_gguf_data_offset(const mx_gguf *g) { return g ? g->data_offset : 0; }
int64_t mx_gguf_tensor_count(const mx_gguf *g) { return g ? (int64_t)g->tensors.size() : 0; }

mx_status mx_gguf_tensor_at(const mx_gguf *g, int64_t i, mx_gguf_tensor *out) {
    if (!g || !out) return fail(MX_ERR_NULL, "gguf_tensor_at: NULL argument");
    if (i < 0 || i >= (int64_t)g->tensors.size())
        return fail(MX_ERR_NOT_FOUND, "gguf_tensor_at: index %lld out of range", (long long)i);
    *out = g->tensors[(size_t)i];
    return MX_OK;
}

mx_status mx_gguf_find_tensor(const mx_gguf *g, const char *name, mx_gguf_tensor *out) {
    if (!g || !name || !out) return fail(MX_ERR_NULL, "gguf_find_tensor: NULL argument");
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) return fail(MX_ERR_NOT_FOUND, "tensor %s not found", name);
    *out = g->tensors[it->second];
    return MX_OK;
}

int32_t mx_gguf_kv_type(const mx_gguf *g, const char *key) {
    const Kv *v = find_kv(g, key);
    return v ? (int32_t)v->type : -1;
}

mx_status mx_gguf_get_int(const mx_gguf *g, const char *key, int64_t *out) {
    if (!g || !key || !out) return fail(MX_ERR_NULL, "gguf_get_int: NULL argument");
    const Kv *v = find_kv(g, key);
    if (!v) return fail(MX_ERR_NOT_FOUND, "metadata key %s not found", key);
    Cursor c{g->fd, v->pos, g->file_size};
    switch (v->type) {
#define MX_INT(T, CT)                      \
    case T: {                              \
        CT x;                              \
        if (!c.get(x)) return c.err;       \
        *out = (int64_t)x;                 \
        return MX_OK;                      \
    }
        MX_INT(T_U8, uint8_t) MX_INT(T_I8, int8_t) MX_INT(T_U16, uint16_t) MX_INT(T_I16, int16_t)
        MX_INT(T_U32, uint32_t) MX_INT(T_I32, int32_t) MX_INT(T_I64, int64_t) MX_INT(T_BOOL, uint8_t)
#undef MX_INT
    case T_U64: {
        uint64_t x;
        if (!c.get(x)) return c.err;
        if (x > (uint64_t)INT64_MAX) return fail(MX_ERR_FORMAT, "metadata %s does not fit int64", key);
        *out = (int64_t)x;
        return MX_OK;
    }
    default: return fail(MX_ERR_DTYPE, "metadata %s (type %u) is not an integer", key, v->type);
    }
}

mx_status mx_gguf_get_float(const mx_gguf *g, const char *key, double *out) {
    if (!g || !key || !out) return fail(MX_ERR_NULL, "gguf_get_float: NULL argument");
    const Kv *v = find_kv(g, key);
    if (!v) return fail(MX_ERR_NOT_FOUND, "metadata key %s not found", key);
    Cursor c{g->fd, v->pos, g->file_size};
    if (v->type == T_F32) {
        float x;
        if (!c.get(x)) return c.err;
        *out = x;
        return MX_OK;
    }
    if (v->type == T_F64) {
        double x;
        if (!c.get(x)) return c.err;
        *out = x;
        return MX_OK;
    }
    int64_t i;
    if (v->type != T_STRING && v->type != T_ARRAY && mx_gguf_get_int(g, key, &i) == MX_OK) {
        *out = (double)i;
        return MX_OK;
    }
    return fail(MX_ERR_DTYPE, "metadata %s (type %u) is not a number", key, v->type);
}

mx_status mx_gguf_get_string(const mx_gguf *g, const char *key, const char **out) {
    if (!g || !key || !out) return fail(MX_ERR_NULL, "gguf_get_string: NULL argument");
    const Kv *v = find_kv(g, key);
    if (!v) return fail(MX_ERR_NOT_FOUND, "metadata key %s not found", key);
    if (v->type != T_STRING) return fail(MX_ERR_DTYPE, "metadata %s (type %u) is not a string", key, v->type);
    *out = v->str.c_str();
    return MX_OK;
}

mx_status mx_gguf_get_array(const mx_gguf *g, const char *key, int32_t *elem_type, uint64_t *count) {
    if (!g || !key || !elem_type || !count) return fail(MX_ERR_NULL, "gguf_get_array: NULL argument");
    const Kv *v = find_kv(g, key);
    if (!v) return fail(MX_ERR_NOT_FOUND, "metadata key %s not found", key);
    if (v->type != T_ARRAY) return fail(MX_ERR_DTYPE, "metadata %s (type %u) is not an array", key, v->type);
    *elem_type = (int32_t)v->elem_type;
    *count = v->count;
    return MX_OK;
}

mx_status mx_gguf_read_host(const mx_gguf *g, const mx_gguf_tensor *t, void *dst, uint64_t dst_bytes) {
    if (!g || !t || !dst) return fail(MX_ERR_NULL, "gguf_read_host: NULL argument");
    if (t->nbytes == 0) return fail(MX_ERR_DTYPE, "gguf_read_host: tensor type %d has no known size", t->ggml_type);
    if (dst_bytes < t->nbytes) return fail(MX_ERR_SHAPE, "gguf_read_host: destination too small");
    Cursor c{g->fd, t->offset, g->file_size};
    return c.read(dst, t->nbytes) ? MX_OK : c.err;
}

mx_status mx_gguf_read(mx_gguf *g, const mx_gguf_tensor *t, void *dst, uint64_t dst_bytes, mx_stream_t stream) {
    if (!g || !t || !dst) return fail(MX_ERR_NULL, "gguf_read: NULL argument");
    if (t->nbytes == 0) return fail(MX_ERR_DTYPE, "gguf_read: tensor type %d has no known size", t->ggml_type);
    if (dst_bytes < t->nbytes) return fail(MX_ERR_SHAPE, "gguf_read: destination too small");
    const hipStream_t s = (hipStream_t)stream;
    constexpr size_t CHUNK = (size_t)32 << 20;
    if (!g->stage[0]) {
        for (int i = 0; i < 2; i++) {
            MX_HIP_G(hipHostMalloc(&g->stage[i], CHUNK, hipHostMallocDefault));
            MX_HIP_G(hipEventCreateWithFlags(&g->done[i], hipEventDisableTiming));
        }
        g->stage_bytes = CHUNK;
    }
    uint8_t *d = static_cast<uint8_t *>(dst);
    bool used[2] = {false, false};
    uint64_t off = 0;
    for (int i = 0; off < t->nbytes; i ^= 1) {
        const uint64_t n = t->nbytes - off < CHUNK ? t->nbytes - off : CHUNK;
        if (used[i]) MX_HIP_G(hipEventSynchronize(g->done[i]));  // the copy out of this buffer has finished
        Cursor c{g->fd, t->offset + off, g->file_size};
        if (!c.read(g->stage[i], n)) return c.err;
        MX_HIP_G(hipMemcpyAsync(d + off, g->stage[i], n, hipMemcpyHostToDevice, s));
        MX_HIP_G(hipEventRecord(g->done[i], s));
        used[i] = true;
        off += n;
    }
    for (int i = 0; i < 2; i++)
        if (used[i]) MX_HIP_G(hipEventSynchronize(g->done[i]));
    return MX_OK;
}

}  // extern "C"
