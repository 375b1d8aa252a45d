// lbq_gguf.cpp -- GGUF v3 container access (host side) and the direct GGUF ->
// device weight upload.
//
// Parsing follows the reference's Lightning parser (parse_gguf,
// /root/reference/src/gguf/parser.rs:136-213): magic 0x46554747, version 3 only,
// little-endian; metadata key/value pairs (types 0..12, arrays recursive);
// tensor infos (name, n_dims, dims[u64], ggml type u32, offset u64); the tensor
// data section starts at the end of the infos rounded up to general.alignment
// (a UInt32 key; default 32).  Tensor byte extents follow extract_tensor_bytes
// (src/quantization/gguf_ops.rs:19-59): ceil(numel / block_size) * type_size
// bytes from data_offset + offset, bounds-checked against the file.  Unlike the
// reference (whose UInt16/Int16 reads and alignment are unchecked), every read
// is bounds-checked and alignment 0 is rejected: malformed files give an error,
// never a fault.
//
// Upload: the file is mapped read-only; a weight's bytes go through two pinned
// staging buffers (hipHostMalloc) into device memory with asynchronous copies on
// a private stream, replacing candle's seek-and-read path (src/gguf/mod.rs:274-282).
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/lbq.h"

// from lbq_api.cpp
int lbq_fail_status(int status, const char *msg);
int lbq_make_owned_weight(lbq_ctx *ctx, uint32_t type, int64_t n, int64_t k, void *d_blocks, size_t nbytes,
                          lbq_weight **out);
int lbq_ctx_device(const lbq_ctx *ctx);

namespace {

int gfail(int status, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return lbq_fail_status(status, buf);
}

// GgmlDType table (/root/reference/src/quantization/mod.rs:58-127): block size,
// bytes per block; 0 for ids the table does not name.
void ggml_layout(uint32_t t, uint64_t *bs, uint64_t *ts) {
    static const uint64_t table[16][2] = {
        {1, 4}, {1, 2}, {32, 18}, {32, 20}, {0, 0}, {0, 0}, {32, 22}, {32, 24},
        {32, 34}, {32, 36}, {256, 82}, {256, 110}, {256, 144}, {256, 176}, {256, 210}, {256, 292}};
    *bs = *ts = 0;
    if (t < 16) {
        *bs = table[t][0];
        *ts = table[t][1];
    }
}

struct Meta {
    std::string key;
    uint32_t type;        // MetadataValueType
    uint64_t off;         // file offset of the value (after the type field)
    uint32_t elem_type;   // arrays: element type
    uint64_t len;         // arrays: element count
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type;
    uint64_t offset;  // relative to the data section
};

struct Reader {
    const uint8_t *p;
    uint64_t n, off = 0;
    int err = 0;
    bool need(uint64_t k, const char *what) {
        if (err) return false;
        if (k > n || off > n - k) {
            err = gfail(LBQ_ERR_FORMAT, "Unexpected EOF reading %s at offset %llu", what, (unsigned long long)off);
            return false;
        }
        return true;
    }
    uint8_t u8(const char *what) {
        if (!need(1, what)) return 0;
        return p[off++];
    }
    uint32_t u32(const char *what = "u32") {
        if (!need(4, what)) return 0;
        uint32_t v;
        memcpy(&v, p + off, 4);  // the host is little-endian, like the format
        off += 4;
        return v;
    }
    uint64_t u64(const char *what = "u64") {
        if (!need(8, what)) return 0;
        uint64_t v;
        memcpy(&v, p + off, 8);
        off += 8;
        return v;
    }
    std::string str() {
        const uint64_t len = u64("string length");
        if (!need(len, "string")) return std::string();
        std::string s(reinterpret_cast<const char *>(p + off), len);
        off += len;
        return s;
    }
};

const uint64_t kScalarSize[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};

// Skips one metadata value of type t (recursing into arrays), validating as it goes.
bool skip_value(Reader &r, uint32_t t, int depth) {
    if (t > 12) {
        r.err = gfail(LBQ_ERR_FORMAT, "Invalid metadata value type: %u", t);
        return false;
    }
    if (t == 8) {
        (void)r.str();
        return !r.err;
    }
    if (t == 9) {
        if (depth > 8) {
            r.err = gfail(LBQ_ERR_FORMAT, "metadata arrays nested too deeply");
            return false;
        }
        const uint32_t et = r.u32("array element type");
        const uint64_t len = r.u64("array length");
        if (r.err) return false;
        if (et > 12) {
            r.err = gfail(LBQ_ERR_FORMAT, "Invalid metadata value type: %u", et);
            return false;
        }
        if (et != 8 && et != 9) {  // fixed-size elements: one bounds check
            const uint64_t sz = kScalarSize[et];
            if (len > (r.n - r.off) / sz) return r.need(r.n - r.off + 1, "array");
            if (et == 7) {
                for (uint64_t i = 0; i < len; i++)
                    if (r.p[r.off + i] > 1) {
                        r.err = gfail(LBQ_ERR_FORMAT, "Invalid bool value: %u (must be 0 or 1)", r.p[r.off + i]);
                        return false;
                    }
            }
            r.off += len * sz;
            return true;
        }
        for (uint64_t i = 0; i < len; i++)
            if (!skip_value(r, et, depth + 1)) return false;
        return true;
    }
    const uint64_t sz = kScalarSize[t];
    if (!r.need(sz, "metadata value")) return false;
    if (t == 7 && r.p[r.off] > 1) {
        r.err = gfail(LBQ_ERR_FORMAT, "Invalid bool value: %u (must be 0 or 1)", r.p[r.off]);
        return false;
    }
    r.off += sz;
    return true;
}

}  // namespace

struct lbq_gguf {
    int fd = -1;
    const uint8_t *base = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_off = 0;
    std::vector<Meta> meta;
    std::unordered_map<std::string, size_t> meta_at;    // last occurrence wins (a map insert)
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> tensor_at;  // first occurrence wins (a linear find)
};

namespace {

int parse(lbq_gguf *g) {
    Reader r{g->base, g->size};
    const uint32_t magic = r.u32();
    if (r.err) return r.err;
    if (magic != 0x46554747u)
        return gfail(LBQ_ERR_FORMAT, "Invalid GGUF magic number: 0x%08X (expected 0x46554747)", magic);
    g->version = r.u32();
    if (r.err) return r.err;
    if (g->version != 3) return gfail(LBQ_ERR_FORMAT, "Unsupported GGUF version: %u (expected 3)", g->version);
    const uint64_t n_tensors = r.u64(), n_kv = r.u64();
    if (r.err) return r.err;
    for (uint64_t i = 0; i < n_kv; i++) {
        Meta m;
        m.key = r.str();
        m.type = r.u32("metadata value type");
        if (r.err) return r.err;
        if (m.type > 12) return gfail(LBQ_ERR_FORMAT, "Invalid metadata value type: %u", m.type);
        m.off = r.off;
        m.elem_type = 0;
        m.len = 0;
        if (m.type == 9) {
            Reader peek = r;
            m.elem_type = peek.u32("array element type");
            m.len = peek.u64("array length");
            if (peek.err) return peek.err;
        }
        if (!skip_value(r, m.type, 0)) return r.err;
        g->meta_at[m.key] = g->meta.size();
        g->meta.push_back(std::move(m));
    }
    auto al = g->meta_at.find("general.alignment");
    if (al != g->meta_at.end() && g->meta[al->second].type == 4) {
        uint32_t a;
        memcpy(&a, g->base + g->meta[al->second].off, 4);
        if (a == 0) return gfail(LBQ_ERR_FORMAT, "general.alignment is 0");
        g->alignment = a;
    }
    for (uint64_t i = 0; i < n_tensors; i++) {
        Tensor t;
        t.name = r.str();
        const uint32_t nd = r.u32("tensor dimension count");
        if (r.err) return r.err;
        if (nd > 8) return gfail(LBQ_ERR_FORMAT, "tensor '%s' has %u dimensions", t.name.c_str(), nd);
        for (uint32_t d = 0; d < nd; d++) t.dims.push_back(r.u64("tensor dimension"));
        t.type = r.u32("tensor type");
        t.offset = r.u64("tensor offset");
        if (r.err) return r.err;
        g->tensor_at.emplace(t.name, g->tensors.size());
        g->tensors.push_back(std::move(t));
    }
    g->data_off = r.off + (g->alignment - r.off % g->alignment) % g->alignment;
    return LBQ_OK;
}

const Meta *meta_of(const lbq_gguf *g, const char *key) {
    auto it = g->meta_at.find(key);
    return it == g->meta_at.end() ? nullptr : &g->meta[it->second];
}

// extract_tensor_bytes: the tensor's exact extent, bounds-checked
// The tensor's byte extent as extract_tensor_bytes computes it: ceil(numel / bs) *
// type_size from the GgmlDType table.  With `blocks`, type_size is instead the size
// of the block the kernels read (lbq_type_block_bytes): the two differ for Q2_K only,
// whose table entry (82) is shorter than its 84-byte block.
int tensor_span(const lbq_gguf *g, const char *name, const Tensor **t_out, uint64_t *start, uint64_t *nbytes,
                bool blocks_layout = false) {
    auto it = g->tensor_at.find(name);
    if (it == g->tensor_at.end()) return gfail(LBQ_ERR_NOT_FOUND, "Tensor not found: %s", name);
    const Tensor &t = g->tensors[it->second];
    uint64_t bs, ts;
    ggml_layout(t.type, &bs, &ts);
    // candle's reader (the device upload path) also takes BF16 tensors, which the
    // reference's own table -- and so extract_tensor_bytes -- does not know
    if (blocks_layout && t.type == LBQ_TYPE_BF16) bs = 1;
    if (!bs) return gfail(LBQ_ERR_UNSUPPORTED_TYPE, "Unknown quantization type: %u", t.type);
    if (blocks_layout && lbq_type_block_bytes(t.type) > 0) ts = (uint64_t)lbq_type_block_bytes(t.type);
    uint64_t numel = 1;
    for (uint64_t d : t.dims) {
        if (d && numel > UINT64_MAX / d) return gfail(LBQ_ERR_FORMAT, "tensor '%s' is too large", name);
        numel *= d;
    }
    const uint64_t blocks = numel / bs + (numel % bs ? 1 : 0);
    if (blocks > UINT64_MAX / ts) return gfail(LBQ_ERR_FORMAT, "tensor '%s' is too large", name);
    const uint64_t sz = blocks * ts;
    const uint64_t st = g->data_off + t.offset;
    if (t.offset > g->size || st > g->size || sz > g->size - st)
        return gfail(LBQ_ERR_FORMAT, "Tensor %s extends beyond file: start=%llu, end=%llu, file_size=%llu", name,
                     (unsigned long long)st, (unsigned long long)(st + sz), (unsigned long long)g->size);
    *t_out = &t;
    *start = st;
    *nbytes = sz;
    return LBQ_OK;
}

// host bytes -> device through two pinned staging buffers on a private stream
int stage_to_device(const uint8_t *src, uint64_t nbytes, void *d_dst) {
    constexpr size_t CH = 16u << 20;
    void *stg[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    hipStream_t st = nullptr;
    int status = LBQ_OK;
    hipError_t e = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
    for (int i = 0; i < 2 && e == hipSuccess; i++) {
        e = hipHostMalloc(&stg[i], CH, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming);
    }
    uint64_t done = 0;
    for (int i = 0; e == hipSuccess && done < nbytes; i ^= 1) {
        const size_t len = (size_t)std::min<uint64_t>(CH, nbytes - done);
        e = hipEventSynchronize(ev[i]);  // the buffer's previous copy has finished
        if (e != hipSuccess) break;
        memcpy(stg[i], src + done, len);
        e = hipMemcpyAsync(static_cast<uint8_t *>(d_dst) + done, stg[i], len, hipMemcpyHostToDevice, st);
        if (e == hipSuccess) e = hipEventRecord(ev[i], st);
        done += len;
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) status = gfail(LBQ_ERR_HIP, "GGUF upload: %s (%d)", hipGetErrorString(e), (int)e);
    if (st) (void)hipStreamSynchronize(st);
    for (int i = 0; i < 2; i++) {
        if (ev[i]) (void)hipEventDestroy(ev[i]);
        if (stg[i]) (void)hipHostFree(stg[i]);
    }
    if (st) (void)hipStreamDestroy(st);
    return status;
}

}  // namespace

extern "C" {

int lbq_gguf_open(const char *path, lbq_gguf **out) {
    if (!path || !out) return gfail(LBQ_ERR_INVALID_ARG, "null argument to lbq_gguf_open");
    *out = nullptr;
    lbq_gguf *g = new (std::nothrow) lbq_gguf;
    if (!g) return gfail(LBQ_ERR_OOM, "host allocation failed");
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (g->fd < 0) {
        delete g;
        return gfail(LBQ_ERR_IO, "Failed to open GGUF file: %s (%s)", path, strerror(errno));
    }
    struct stat sb;
    if (fstat(g->fd, &sb) != 0) {
        const int er = errno;
        lbq_gguf_close(g);
        return gfail(LBQ_ERR_IO, "Failed to stat GGUF file: %s (%s)", path, strerror(er));
    }
    g->size = (uint64_t)sb.st_size;
    if (g->size) {
        void *p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
        if (p == MAP_FAILED) {
            const int er = errno;
            lbq_gguf_close(g);
            return gfail(LBQ_ERR_IO, "Failed to mmap GGUF file: %s (%s)", path, strerror(er));
        }
        g->base = static_cast<const uint8_t *>(p);
    }
    const int s = parse(g);
    if (s) {
        lbq_gguf_close(g);
        return s;
    }
    *out = g;
    return LBQ_OK;
}

int lbq_gguf_close(lbq_gguf *g) {
    if (!g) return LBQ_OK;
    if (g->base) munmap(const_cast<uint8_t *>(g->base), g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
    return LBQ_OK;
}

int lbq_gguf_header(const lbq_gguf *g, uint32_t *version, int64_t *tensor_count, int64_t *metadata_count,
                    uint64_t *alignment, uint64_t *tensor_data_offset, uint64_t *file_size) {
    if (!g) return gfail(LBQ_ERR_INVALID_ARG, "null GGUF handle");
    if (version) *version = g->version;
    if (tensor_count) *tensor_count = (int64_t)g->tensors.size();
    if (metadata_count) *metadata_count = (int64_t)g->meta.size();
    if (alignment) *alignment = g->alignment;
    if (tensor_data_offset) *tensor_data_offset = g->data_off;
    if (file_size) *file_size = g->size;
    return LBQ_OK;
}

int lbq_gguf_tensor_info(const lbq_gguf *g, int64_t index, const char **name, uint32_t *ggml_type, uint32_t *n_dims,
                         uint64_t *dims, uint64_t *offset) {
    if (!g) return gfail(LBQ_ERR_INVALID_ARG, "null GGUF handle");
    if (index < 0 || index >= (int64_t)g->tensors.size())
        return gfail(LBQ_ERR_INVALID_ARG, "tensor index %lld out of range", (long long)index);
    const Tensor &t = g->tensors[(size_t)index];
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = t.type;
    if (n_dims) *n_dims = (uint32_t)t.dims.size();
    if (dims)
        for (size_t d = 0; d < t.dims.size(); d++) dims[d] = t.dims[d];
    if (offset) *offset = t.offset;
    return LBQ_OK;
}

int lbq_gguf_find_tensor(const lbq_gguf *g, const char *name, int64_t *index) {
    if (!g || !name || !index) return gfail(LBQ_ERR_INVALID_ARG, "null argument to lbq_gguf_find_tensor");
    auto it = g->tensor_at.find(name);
    if (it == g->tensor_at.end()) return gfail(LBQ_ERR_NOT_FOUND, "Tensor not found: %s", name);
    *index = (int64_t)it->second;
    return LBQ_OK;
}

int lbq_gguf_tensor_bytes(const lbq_gguf *g, const char *name, const void **data, size_t *nbytes) {
    if (!g || !name || !data || !nbytes) return gfail(LBQ_ERR_INVALID_ARG, "null argument to lbq_gguf_tensor_bytes");
    const Tensor *t;
    uint64_t st, sz;
    const int s = tensor_span(g, name, &t, &st, &sz);
    if (s) return s;
    *data = g->base + st;
    *nbytes = (size_t)sz;
    return LBQ_OK;
}

int lbq_gguf_meta_key(const lbq_gguf *g, int64_t index, const char **key, uint32_t *value_type) {
    if (!g) return gfail(LBQ_ERR_INVALID_ARG, "null GGUF handle");
    if (index < 0 || index >= (int64_t)g->meta.size())
        return gfail(LBQ_ERR_INVALID_ARG, "metadata index %lld out of range", (long long)index);
    if (key) *key = g->meta[(size_t)index].key.c_str();
    if (value_type) *value_type = g->meta[(size_t)index].type;
    return LBQ_OK;
}

int lbq_gguf_meta_int(const lbq_gguf *g, const char *key, int64_t *out) {
    if (!g || !key || !out) return gfail(LBQ_ERR_INVALID_ARG, "null argument to lbq_gguf_meta_int");
    const Meta *m = meta_of(g, key);
    if (!m) return gfail(LBQ_ERR_NOT_FOUND, "metadata key not found: %s", key);
    const uint8_t *p = g->base + m->off;
    switch (m->type) {
    case 0: *out = p[0]; return LBQ_OK;
    case 1: *out = (int8_t)p[0]; return LBQ_OK;
    case 2: { uint16_t v; memcpy(&v, p, 2); *out = v; return LBQ_OK; }
    case 3: { int16_t v; memcpy(&v, p, 2); *out = v; return LBQ_OK; }
    case 4: { uint32_t v; memcpy(&v, p, 4); *out = v; return LBQ_OK; }
    case 5: { int32_t v; memcpy(&v, p, 4); *out = v; return LBQ_OK; }
    case 7: *out = p[0]; return LBQ_OK;
    case 10: {
        uint64_t v;
        memcpy(&v, p, 8);
        if (v > (uint64_t)INT64_MAX) return gfail(LBQ_ERR_LIMIT, "metadata %s = %llu does not fit int64", key, (unsigned long long)v);
        *out = (int64_t)v;
        return LBQ_OK;
    }
    case 11: { int64_t v; memcpy(&v, p, 8); *out = v; return LBQ_OK; }
    default: return gfail(LBQ_ERR_FORMAT, "metadata %s has type %u, not an integer", key, m->type);
    }
}

int lbq_gguf_meta_float(const lbq_gguf *g, const char *key, double *out) {
    if (!g || !key || !out) return gfail(LBQ_ERR_INVALID_ARG, "null argument to lbq_gguf_meta_float");
    const Meta *m = meta_of(g, key);
    if (!m) return gfail(LBQ_ERR_NOT_FOUND, "metadata key not found: %s", key);
    const uint8_t *p = g->base + m->off;
    if (m->type == 6) {
        float v;
        memcpy(&v, p, 4);
        *out = v;
        return LBQ_OK;
    }
    if (m->type == 12) {
        memcpy(out, p, 8);
        return LBQ_OK;
    }
    return gfail(LBQ_ERR_FORMAT, "metadata %s has type %u, not a float", key, m->type);
}

int lbq_gguf_meta_string(const lbq_gguf *g, const char *key, const char **data, size_t *len) {
    if (!g || !key || !data || !len) return gfail(LBQ_ERR_INVALID_ARG, "null argument to lbq_gguf_meta_string");
    const Meta *m = meta_of(g, key);
    if (!m) return gfail(LBQ_ERR_NOT_FOUND, "metadata key not found: %s", key);
    if (m->type != 8) return gfail(LBQ_ERR_FORMAT, "metadata %s has type %u, not a string", key, m->type);
    uint64_t n;
    memcpy(&n, g->base + m->off, 8);
    *data = reinterpret_cast<const char *>(g->base + m->off + 8);
    *len = (size_t)n;
    return LBQ_OK;
}

int lbq_gguf_meta_array(const lbq_gguf *g, const char *key, uint32_t *elem_type, uint64_t *len) {
    if (!g || !key) return gfail(LBQ_ERR_INVALID_ARG, "null argument to lbq_gguf_meta_array");
    const Meta *m = meta_of(g, key);
    if (!m) return gfail(LBQ_ERR_NOT_FOUND, "metadata key not found: %s", key);
    if (m->type != 9) return gfail(LBQ_ERR_FORMAT, "metadata %s has type %u, not an array", key, m->type);
    if (elem_type) *elem_type = m->elem_type;
    if (len) *len = m->len;
    return LBQ_OK;
}

int lbq_gguf_copy_tensor(const lbq_gguf *g, const char *name, void *d_dst, size_t dst_bytes) {
    if (!g || !name || !d_dst) return gfail(LBQ_ERR_INVALID_ARG, "null argument to lbq_gguf_copy_tensor");
    const Tensor *t;
    uint64_t st, sz;
    int s = tensor_span(g, name, &t, &st, &sz, true);
    if (s) return s;
    if (dst_bytes < sz)
        return gfail(LBQ_ERR_SHAPE, "destination holds %zu bytes, tensor %s needs %llu", dst_bytes, name, (unsigned long long)sz);
    return stage_to_device(g->base + st, sz, d_dst);
}

int lbq_weight_from_gguf(lbq_ctx *ctx, const lbq_gguf *g, const char *name, lbq_weight **out_w) {
    if (!ctx || !g || !name || !out_w) return gfail(LBQ_ERR_INVALID_ARG, "null argument to lbq_weight_from_gguf");
    *out_w = nullptr;
    const Tensor *t;
    uint64_t st, sz;
    int s = tensor_span(g, name, &t, &st, &sz, true);
    if (s) return s;
    if (t->dims.size() != 2)
        return gfail(LBQ_ERR_SHAPE, "tensor %s has %zu dimensions; a weight has 2 (ne0 = k, ne1 = n)", name, t->dims.size());
    const int64_t k = (int64_t)t->dims[0], n = (int64_t)t->dims[1];
    int prev = -1;
    (void)hipGetDevice(&prev);
    hipError_t e = hipSetDevice(lbq_ctx_device(ctx));
    if (e != hipSuccess) return gfail(LBQ_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(e));
    void *d = nullptr;
    e = hipMalloc(&d, sz ? sz : 1);
    if (e != hipSuccess) {
        if (prev >= 0) (void)hipSetDevice(prev);
        return gfail(LBQ_ERR_OOM, "hipMalloc(%llu) for tensor %s: %s", (unsigned long long)sz, name, hipGetErrorString(e));
    }
    s = stage_to_device(g->base + st, sz, d);
    if (!s) s = lbq_make_owned_weight(ctx, t->type, n, k, d, (size_t)sz, out_w);
    if (s) (void)hipFree(d);
    if (prev >= 0) (void)hipSetDevice(prev);
    return s;
}

}  // extern "C"
