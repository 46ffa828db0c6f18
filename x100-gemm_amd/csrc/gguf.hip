// GGUF checkpoint reader (host code): the file is mapped read-only and parsed with a cursor that
// checks every read against the mapping's size.  Layout (GGUF v2/v3, as bench/gguf_dump.c:2-4
// summarises it):
//   "GGUF" | u32 version | u64 n_tensors | u64 n_kv |
//   n_kv x { str key | u32 type | value } |
//   n_tensors x { str name | u32 n_dims | u64 dims[n_dims] | u32 ggml_type | u64 offset } |
//   padding to general.alignment (default 32) | tensor data
// str = u64 length + bytes; an array value = u32 element type + u64 count + elements.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#pragma GCC visibility push(default)
#include "x100_gemm.h"
#include "x100_gguf.h"
#include "x100_qgemv.h"
#pragma GCC visibility pop

namespace {

// ggml type ids with the names bench/gguf_dump.c:12-14 prints and the block geometry of ggml's
// formats (bytes, elements).  Ids 4 and 5 are retired (empty names there too); the IQ formats
// are listed by name only.
struct TypeInfo {
    const char *name;
    uint32_t bytes;
    uint32_t elems;
};
const TypeInfo kTypes[] = {
    {"F32", 4, 1},      {"F16", 2, 1},       {"Q4_0", 18, 32},    {"Q4_1", 20, 32},   {"", 0, 0},
    {"", 0, 0},         {"Q5_0", 22, 32},    {"Q5_1", 24, 32},    {"Q8_0", 34, 32},   {"Q8_1", 36, 32},
    {"Q2_K", 84, 256},  {"Q3_K", 110, 256},  {"Q4_K", 144, 256},  {"Q5_K", 176, 256}, {"Q6_K", 210, 256},
    {"Q8_K", 292, 256}, {"IQ2_XXS", 0, 0},   {"IQ2_XS", 0, 0},    {"IQ3_XXS", 0, 0},  {"IQ1_S", 0, 0},
    {"IQ4_NL", 0, 0},   {"IQ3_S", 0, 0},     {"IQ2_S", 0, 0},     {"IQ4_XS", 0, 0},   {"I8", 1, 1},
    {"I16", 2, 1},      {"I32", 4, 1},       {"I64", 8, 1},       {"F64", 8, 1},      {"IQ1_M", 0, 0},
    {"BF16", 2, 1},
};
constexpr uint32_t kNTypes = sizeof(kTypes) / sizeof(kTypes[0]);

// Size of a fixed-size metadata value (0 for string / array / unknown).
uint64_t scalar_bytes(uint32_t t)
{
    switch (t) {
    case X100_GGUF_U8: case X100_GGUF_I8: case X100_GGUF_BOOL: return 1;
    case X100_GGUF_U16: case X100_GGUF_I16: return 2;
    case X100_GGUF_U32: case X100_GGUF_I32: case X100_GGUF_F32: return 4;
    case X100_GGUF_U64: case X100_GGUF_I64: case X100_GGUF_F64: return 8;
    }
    return 0;
}

struct Cursor {
    const uint8_t *p;
    uint64_t n, off = 0;
    bool ok = true;
    bool need(uint64_t k)
    {
        if (!ok || k > n - off) ok = false;
        return ok;
    }
    uint32_t u32()
    {
        uint32_t v = 0;
        if (need(4)) { memcpy(&v, p + off, 4); off += 4; }
        return v;
    }
    uint64_t u64()
    {
        uint64_t v = 0;
        if (need(8)) { memcpy(&v, p + off, 8); off += 8; }
        return v;
    }
    // A string: returns its offset and length, and moves past it.
    bool str(uint64_t &at, uint64_t &len)
    {
        len = u64();
        at = off;
        if (!need(len)) return false;
        off += len;
        return true;
    }
    // Skips one value of type t; arrays may nest (depth-limited).
    bool skip(uint32_t t, int depth = 0)
    {
        if (const uint64_t b = scalar_bytes(t)) return need(b) && (off += b, true);
        if (t == X100_GGUF_STRING) {
            uint64_t at, len;
            return str(at, len);
        }
        if (t == X100_GGUF_ARRAY && depth < 4) {
            const uint32_t et = u32();
            const uint64_t cnt = u64();
            if (!ok) return false;
            if (const uint64_t b = scalar_bytes(et)) {
                if (cnt > (n - off) / b) return ok = false;
                off += cnt * b;
                return true;
            }
            for (uint64_t i = 0; i < cnt && ok; i++) skip(et, depth + 1);
            return ok;
        }
        return ok = false;
    }
};

struct KV {
    std::string key;
    uint32_t type, elem_type = 0;
    uint64_t count = 0;
    uint64_t val;                     // file offset of the value (after the type field)
    std::vector<uint64_t> str_at;     // string arrays: offset of element j's length field
};

struct Tensor {
    std::string name;
    x100_gguf_tensor t;
};

int map_err(hipError_t e) { return e == hipErrorOutOfMemory ? X100_ENOMEM : X100_EHIP; }

}  // namespace

struct x100_gguf {
    const uint8_t *p = nullptr;
    uint64_t size = 0;
    uint32_t version = 0, alignment = 32;
    uint64_t data_off = 0;
    std::vector<KV> kv;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> kidx, tidx;
    ~x100_gguf()
    {
        if (p) munmap(const_cast<uint8_t *>(p), size);
    }
};

namespace {

int parse(x100_gguf *g)
{
    Cursor c{g->p, g->size};
    if (!c.need(4) || memcmp(g->p, "GGUF", 4) != 0) return X100_EFORMAT;
    c.off = 4;
    g->version = c.u32();
    if (g->version != 2 && g->version != 3) return X100_EFORMAT;
    const uint64_t nt = c.u64(), nkv = c.u64();
    // every key and tensor record takes at least 12 / 24 bytes: bounds the reservations
    if (!c.ok || nkv > g->size / 12 || nt > g->size / 24) return X100_EFORMAT;
    g->kv.reserve(nkv);
    for (uint64_t i = 0; i < nkv; i++) {
        KV e;
        uint64_t at, len;
        if (!c.str(at, len)) return X100_EFORMAT;
        e.key.assign((const char *)g->p + at, len);
        e.type = c.u32();
        e.val = c.off;
        if (e.type == X100_GGUF_ARRAY) {
            e.elem_type = c.u32();
            e.count = c.u64();
            c.off = e.val;
            if (c.ok && e.elem_type == X100_GGUF_STRING) {
                c.off += 12;
                if (e.count > (g->size - c.off) / 8) return X100_EFORMAT;
                e.str_at.reserve(e.count);
                for (uint64_t j = 0; j < e.count && c.ok; j++) {
                    e.str_at.push_back(c.off);
                    c.str(at, len);
                }
                if (!c.ok) return X100_EFORMAT;
                c.off = e.val;
            }
        }
        if (!c.skip(e.type)) return X100_EFORMAT;
        g->kidx.emplace(e.key, g->kv.size());
        g->kv.push_back(std::move(e));
    }
    int64_t al = 0;
    if (x100_gguf_get_int(g, "general.alignment", &al) == X100_OK) {
        if (al <= 0 || al > (1 << 20) || (al & (al - 1))) return X100_EFORMAT;
        g->alignment = (uint32_t)al;
    }
    g->tensors.reserve(nt);
    for (uint64_t i = 0; i < nt; i++) {
        Tensor e;
        uint64_t at, len;
        if (!c.str(at, len)) return X100_EFORMAT;
        e.name.assign((const char *)g->p + at, len);
        x100_gguf_tensor &t = e.t;
        memset(&t, 0, sizeof t);
        t.n_dims = c.u32();
        if (!c.ok || t.n_dims < 1 || t.n_dims > 4) return X100_EFORMAT;
        t.n_elems = 1;
        for (uint32_t d = 0; d < 4; d++) t.dims[d] = 1;
        for (uint32_t d = 0; d < t.n_dims; d++) {
            t.dims[d] = c.u64();
            if (t.dims[d] && t.n_elems > UINT64_MAX / t.dims[d]) return X100_EFORMAT;
            t.n_elems *= t.dims[d];
        }
        t.type = c.u32();
        t.offset = c.u64();
        if (!c.ok) return X100_EFORMAT;
        g->tensors.push_back(std::move(e));
    }
    g->data_off = (c.off + g->alignment - 1) / g->alignment * g->alignment;
    for (size_t i = 0; i < g->tensors.size(); i++) {
        Tensor &e = g->tensors[i];
        x100_gguf_tensor &t = e.t;
        t.name = e.name.c_str();
        const size_t bb = x100_gguf_block_bytes(t.type);
        const int be = x100_gguf_block_elems(t.type);
        if (bb && be) {
            if (t.n_elems % (uint64_t)be) return X100_EFORMAT;
            const uint64_t nblk = t.n_elems / (uint64_t)be;
            if (nblk > UINT64_MAX / bb) return X100_EFORMAT;
            t.n_bytes = nblk * bb;
            if (g->data_off > g->size || t.offset > g->size - g->data_off ||
                t.n_bytes > g->size - g->data_off - t.offset)
                return X100_EFORMAT;
            t.data = g->p + g->data_off + t.offset;
        }
        g->tidx.emplace(e.name, i);
    }
    return X100_OK;
}

const KV *find_kv(const x100_gguf *g, const char *key)
{
    if (!g || !key) return nullptr;
    auto it = g->kidx.find(key);
    return it == g->kidx.end() ? nullptr : &g->kv[it->second];
}

}  // namespace

extern "C" {

int x100_gguf_open(const char *path, x100_gguf **out)
{
    if (!out) return X100_EINVAL;
    *out = nullptr;
    if (!path) return X100_EINVAL;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return X100_EIO;
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return X100_EIO;
    }
    if (st.st_size <= 0) {   // empty (or not a regular file): nothing to map
        close(fd);
        return X100_EFORMAT;
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return X100_EIO;
    x100_gguf *g = new (std::nothrow) x100_gguf;
    if (!g) {
        munmap(m, (size_t)st.st_size);
        return X100_ENOMEM;
    }
    g->p = (const uint8_t *)m;
    g->size = (uint64_t)st.st_size;
    int rc;
    try {
        rc = parse(g);
    } catch (...) {   // std::bad_alloc from the tables
        rc = X100_ENOMEM;
    }
    if (rc != X100_OK) {
        delete g;
        return rc;
    }
    *out = g;
    return X100_OK;
}

void x100_gguf_close(x100_gguf *g) { delete g; }

uint32_t x100_gguf_version(const x100_gguf *g) { return g ? g->version : 0; }
int64_t x100_gguf_n_tensors(const x100_gguf *g) { return g ? (int64_t)g->tensors.size() : 0; }
int64_t x100_gguf_n_kv(const x100_gguf *g) { return g ? (int64_t)g->kv.size() : 0; }
uint32_t x100_gguf_alignment(const x100_gguf *g) { return g ? g->alignment : 0; }
uint64_t x100_gguf_data_offset(const x100_gguf *g) { return g ? g->data_off : 0; }

int x100_gguf_tensor_at(const x100_gguf *g, int64_t i, x100_gguf_tensor *t)
{
    if (!g || !t || i < 0 || i >= (int64_t)g->tensors.size()) return X100_EINVAL;
    *t = g->tensors[(size_t)i].t;
    return X100_OK;
}

int x100_gguf_find(const x100_gguf *g, const char *name, x100_gguf_tensor *t)
{
    if (!g || !name || !t) return X100_EINVAL;
    auto it = g->tidx.find(name);
    if (it == g->tidx.end()) return X100_ENOTFOUND;
    *t = g->tensors[it->second].t;
    return X100_OK;
}

int x100_gguf_kv_at(const x100_gguf *g, int64_t i, const char **key, uint32_t *type, uint32_t *elem_type,
                    uint64_t *count)
{
    if (!g || i < 0 || i >= (int64_t)g->kv.size()) return X100_EINVAL;
    const KV &e = g->kv[(size_t)i];
    if (key) *key = e.key.c_str();
    if (type) *type = e.type;
    if (elem_type) *elem_type = e.elem_type;
    if (count) *count = e.count;
    return X100_OK;
}

int x100_gguf_get_int(const x100_gguf *g, const char *key, int64_t *v)
{
    const KV *e = find_kv(g, key);
    if (!e || !v) return e ? X100_EINVAL : X100_ENOTFOUND;
    const uint8_t *q = g->p + e->val;   // in bounds: the parse skipped the whole value
    switch (e->type) {
    case X100_GGUF_U8: *v = *q; return X100_OK;
    case X100_GGUF_I8: *v = (int8_t)*q; return X100_OK;
    case X100_GGUF_U16: { uint16_t x; memcpy(&x, q, 2); *v = x; return X100_OK; }
    case X100_GGUF_I16: { int16_t x; memcpy(&x, q, 2); *v = x; return X100_OK; }
    case X100_GGUF_U32: { uint32_t x; memcpy(&x, q, 4); *v = x; return X100_OK; }
    case X100_GGUF_I32: { int32_t x; memcpy(&x, q, 4); *v = x; return X100_OK; }
    case X100_GGUF_I64: { int64_t x; memcpy(&x, q, 8); *v = x; return X100_OK; }
    case X100_GGUF_U64: {
        uint64_t x;
        memcpy(&x, q, 8);
        if (x > (uint64_t)INT64_MAX) return X100_ENOTFOUND;
        *v = (int64_t)x;
        return X100_OK;
    }
    }
    return X100_ENOTFOUND;
}

int x100_gguf_get_float(const x100_gguf *g, const char *key, double *v)
{
    const KV *e = find_kv(g, key);
    if (!e || !v) return e ? X100_EINVAL : X100_ENOTFOUND;
    const uint8_t *q = g->p + e->val;
    if (e->type == X100_GGUF_F32) { float x; memcpy(&x, q, 4); *v = x; return X100_OK; }
    if (e->type == X100_GGUF_F64) { double x; memcpy(&x, q, 8); *v = x; return X100_OK; }
    return X100_ENOTFOUND;
}

int x100_gguf_get_str(const x100_gguf *g, const char *key, const char **s, uint64_t *len)
{
    const KV *e = find_kv(g, key);
    if (!e || !s || !len) return e ? X100_EINVAL : X100_ENOTFOUND;
    if (e->type != X100_GGUF_STRING) return X100_ENOTFOUND;
    memcpy(len, g->p + e->val, 8);
    *s = (const char *)g->p + e->val + 8;
    return X100_OK;
}

int x100_gguf_get_arr_str(const x100_gguf *g, const char *key, uint64_t j, const char **s, uint64_t *len)
{
    const KV *e = find_kv(g, key);
    if (!e || !s || !len) return e ? X100_EINVAL : X100_ENOTFOUND;
    if (e->type != X100_GGUF_ARRAY || e->elem_type != X100_GGUF_STRING) return X100_ENOTFOUND;
    if (j >= e->str_at.size()) return X100_EINVAL;
    memcpy(len, g->p + e->str_at[j], 8);
    *s = (const char *)g->p + e->str_at[j] + 8;
    return X100_OK;
}

int x100_gguf_qwen3moe_params(const x100_gguf *g, x100_gguf_qwen3moe *p)
{
    if (!g || !p) return X100_EINVAL;
    memset(p, 0, sizeof *p);
    p->rope_base = 1e6f;
    p->n_act = 8;
    p->n_exp = 128;
    p->moe_ffn = 768;
    struct { const char *key; int *dst; } ints[] = {
        {"qwen3moe.block_count", &p->block_count},
        {"qwen3moe.embedding_length", &p->embd},
        {"qwen3moe.feed_forward_length", &p->ffn},
        {"qwen3moe.attention.head_count", &p->n_head},
        {"qwen3moe.attention.head_count_kv", &p->n_head_kv},
        {"qwen3moe.attention.key_length", &p->head_dim},
        {"qwen3moe.expert_count", &p->n_exp},
        {"qwen3moe.expert_used_count", &p->n_act},
        {"qwen3moe.expert_feed_forward_length", &p->moe_ffn},
    };
    for (auto &k : ints) {
        int64_t v;
        if (x100_gguf_get_int(g, k.key, &v) == X100_OK && v >= INT32_MIN && v <= INT32_MAX) *k.dst = (int)v;
    }
    double f;
    if (x100_gguf_get_float(g, "qwen3moe.rope.freq_base", &f) == X100_OK) p->rope_base = (float)f;
    const KV *tok = find_kv(g, "tokenizer.ggml.tokens");
    if (tok && tok->type == X100_GGUF_ARRAY && tok->count <= INT32_MAX) p->n_tokens = (int)tok->count;
    x100_gguf_tensor t;
    if (x100_gguf_find(g, "token_embd.weight", &t) == X100_OK && t.n_dims >= 2 && t.dims[1] <= INT32_MAX)
        p->vocab = (int)t.dims[1];
    return X100_OK;
}

const char *x100_gguf_type_name(uint32_t type) { return type < kNTypes ? kTypes[type].name : "?"; }
size_t x100_gguf_block_bytes(uint32_t type) { return type < kNTypes ? kTypes[type].bytes : 0; }
int x100_gguf_block_elems(uint32_t type) { return type < kNTypes ? (int)kTypes[type].elems : 0; }

int x100_gguf_upload(const x100_gguf *g, const x100_gguf_tensor *t, uint64_t byte0, uint64_t n, void *dst,
                     void *stream)
{
    if (!g || !t || !t->data || !dst) return X100_EINVAL;
    if (byte0 > t->n_bytes || n > t->n_bytes - byte0) return X100_EINVAL;
    if (n == 0) return X100_OK;
    hipError_t e = hipMemcpyAsync(dst, (const uint8_t *)t->data + byte0, n, hipMemcpyHostToDevice,
                                  (hipStream_t)stream);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
    return e == hipSuccess ? X100_OK : map_err(e);
}

int x100_gguf_pack_rows(const x100_gguf *g, const x100_gguf_tensor *t, uint64_t row0, uint64_t n_rows,
                        void *w_packed, void *stream)
{
    if (!g || !t || !t->data || !w_packed || n_rows == 0) return X100_EINVAL;
    const uint64_t K = t->dims[0];
    if (K == 0 || K > INT32_MAX || n_rows > INT32_MAX) return X100_EINVAL;
    const uint64_t rows = t->n_elems / K;
    if (row0 > rows || n_rows > rows - row0) return X100_EINVAL;
    const size_t rb = x100q_gguf_bytes((int)t->type, 1, (int)K);
    if (!rb) return X100_EINVAL;   // not a qgemv type, or K not a whole number of blocks
    void *tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, rb * n_rows);
    if (e != hipSuccess) return map_err(e);
    int rc = x100_gguf_upload(g, t, row0 * rb, n_rows * rb, tmp, stream);
    if (rc == X100_OK) rc = x100q_pack((int)t->type, (int)n_rows, (int)K, tmp, w_packed, stream);
    if (rc == X100_OK) {
        e = hipStreamSynchronize((hipStream_t)stream);
        if (e != hipSuccess) rc = map_err(e);
    }
    (void)hipFree(tmp);
    return rc;
}

}  // extern "C"
