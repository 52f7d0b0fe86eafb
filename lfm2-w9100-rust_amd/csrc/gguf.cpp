// gguf.cpp -- GGUF v3 model files for the LFM2 engine: a reader (header, typed
// metadata, tensor table, positioned reads of tensor bytes), a streaming writer,
// the lfm2moe hyper-parameter mapping and the loader that uploads a file's
// tensors through lfm_engine_upload_tensor.
//
// File layout, little-endian throughout, with the checks the reference applies
// (Amidwestnoob/lfm2-w9100-rust parser/src/gguf.rs:299-440):
//   "GGUF" | u32 version (== 3) | u64 tensor_count | u64 kv_count   (counts <= 100 000)
//   kv_count     x { string key | u32 value type | value }           (no duplicate keys)
//   tensor_count x { string name | u32 n_dims (<= 8) | u64 ne[n_dims] | u32 ggml type
//                    | u64 offset }                                  (no duplicate names)
//   zero padding up to `alignment` = metadata "general.alignment" when it is a U32
//   (a power of two), else 32; tensor data follows, tensor i at data_offset + offset_i,
//   and every tensor must end inside the file.
// Keys and tensor names are looked up through C strings, so one containing a NUL
// byte is rejected (the reference accepts it; no real model file has one).
// A string is a u64 byte length (<= 1 GiB) and UTF-8 bytes; an array is a u32
// element type, a u64 count (<= 10 000 000) and the elements' payloads.
#include <errno.h>
#include <fcntl.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <map>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/lfm_hip.h"
#include "host_err.h"

#define RC(call)                                                                              \
    do {                                                                                      \
        int _rc = (call);                                                                     \
        if (_rc != LFM_OK)                                                                    \
            return _rc;                                                                       \
    } while (0)

namespace {

constexpr uint32_t kVersion = 3;
constexpr uint64_t kMaxCount = 100000;       // tensors and metadata pairs
constexpr uint64_t kMaxString = 1ull << 30;  // bytes in one string
constexpr uint64_t kMaxArray = 10000000;     // elements in one array
constexpr uint32_t kMaxDims = 8;
constexpr uint32_t kDefaultAlign = 32;
// Arrays of arrays recurse; a corrupt file could nest them without bound.
constexpr int kMaxNesting = 64;

// One metadata value.  Scalars live in u (unsigned kinds and BOOL), i (signed
// kinds) or f (F32, F64); strings in s; arrays in a, all of type elem.
struct Value {
    uint32_t type = 0;
    uint32_t elem = 0;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string s;
    std::vector<Value> a;
};

// Elements per block and bytes per block of each ggml storage type the format
// accepts; other type ids are rejected.  The table is the reference parser's
// (gguf.rs:174-192), so a file is accepted, rejected and sized exactly as there.
// That includes its Q3_K and Q8_K entries, 112 and 288 bytes, where ggml's block
// structs take 110 and 292; no tensor of either type is uploaded to the engine.
bool block_info(uint32_t type, uint64_t *elems, uint64_t *bytes)
{
    static const struct {
        uint32_t type, elems, bytes;
    } table[] = {
        {0, 1, 4},      // F32
        {1, 1, 2},      // F16
        {2, 32, 18},    // Q4_0: f16 d, 16 B of nibbles
        {3, 32, 20},    // Q4_1: f16 d, m, 16 B
        {6, 32, 22},    // Q5_0: f16 d, 4 B high bits, 16 B
        {7, 32, 24},    // Q5_1: f16 d, m, 4 B, 16 B
        {8, 32, 34},    // Q8_0: f16 d, 32 int8
        {9, 32, 36},    // Q8_1: f16 d, s, 32 int8
        {10, 256, 84},  // Q2_K: 16 B scales, 64 B quants, f16 d, dmin
        {11, 256, 112}, // Q3_K (ggml's block: 110 B)
        {12, 256, 144}, // Q4_K: f16 d, dmin, 12 B scales, 128 B quants
        {13, 256, 176}, // Q5_K: f16 d, dmin, 12 B scales, 32 B high bits, 128 B
        {14, 256, 210}, // Q6_K: 128 B low bits, 64 B high bits, 16 int8 scales, f16 d
        {15, 256, 288}, // Q8_K (ggml's block: 292 B)
    };
    for (const auto &t : table)
        if (t.type == type) {
            *elems = t.elems;
            *bytes = t.bytes;
            return true;
        }
    return false;
}

// Bytes of a tensor.  A zero dimension makes an empty tensor (checked before the
// running product can overflow), quantized types need whole blocks.
int tensor_nbytes(uint32_t type, const uint64_t *ne, uint32_t nd, uint64_t *out)
{
    uint64_t per_block_elems, per_block_bytes;
    if (!block_info(type, &per_block_elems, &per_block_bytes))
        return fail(LFM_EINVAL, "unknown GGML type: %u", type);
    uint64_t n = 1;
    for (uint32_t k = 0; k < nd; ++k) {
        if (ne[k] == 0) {
            *out = 0;
            return LFM_OK;
        }
        if (__builtin_mul_overflow(n, ne[k], &n))
            return fail(LFM_EINVAL, "dimension product overflow");
    }
    if (n % per_block_elems)
        return fail(LFM_EINVAL, "tensor has %llu elements, not a multiple of block size %llu for "
                    "GGML type %u", (unsigned long long)n, (unsigned long long)per_block_elems,
                    type);
    if (__builtin_mul_overflow(n / per_block_elems, per_block_bytes, out))
        return fail(LFM_EINVAL, "tensor size overflow");
    return LFM_OK;
}

uint64_t align_up(uint64_t x, uint32_t a) { return (x + a - 1) & ~(uint64_t)(a - 1); }
bool power_of_two(uint32_t a) { return a && !(a & (a - 1)); }

// RFC 3629 UTF-8: no overlong forms, no surrogates, nothing above U+10FFFF.
bool valid_utf8(const uint8_t *p, size_t n)
{
    static const uint32_t min_cp[5] = {0, 0, 0x80, 0x800, 0x10000};
    size_t i = 0;
    while (i < n) {
        const uint8_t c = p[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        int len;
        uint32_t cp;
        if ((c & 0xE0) == 0xC0) {
            len = 2;
            cp = c & 0x1F;
        } else if ((c & 0xF0) == 0xE0) {
            len = 3;
            cp = c & 0x0F;
        } else if ((c & 0xF8) == 0xF0) {
            len = 4;
            cp = c & 0x07;
        } else {
            return false;
        }
        if (n - i < (size_t)len)
            return false;
        for (int k = 1; k < len; ++k) {
            if ((p[i + k] & 0xC0) != 0x80)
                return false;
            cp = cp << 6 | (p[i + k] & 0x3F);
        }
        if (cp < min_cp[len] || cp > 0x10FFFF || (cp >= 0xD800 && cp <= 0xDFFF))
            return false;
        i += len;
    }
    return true;
}

bool scalar_size(uint32_t type, size_t *size)
{
    switch (type) {
    case LFM_GGUF_TYPE_U8: case LFM_GGUF_TYPE_I8: case LFM_GGUF_TYPE_BOOL: *size = 1; return true;
    case LFM_GGUF_TYPE_U16: case LFM_GGUF_TYPE_I16: *size = 2; return true;
    case LFM_GGUF_TYPE_U32: case LFM_GGUF_TYPE_I32: case LFM_GGUF_TYPE_F32: *size = 4; return true;
    case LFM_GGUF_TYPE_U64: case LFM_GGUF_TYPE_I64: case LFM_GGUF_TYPE_F64: *size = 8; return true;
    default: return false;
    }
}

// Decodes a scalar of `type` from `size` little-endian bytes (the host is
// little-endian: x86-64 and the GPU hosts this library builds for).
int decode_scalar(uint32_t type, const uint8_t *p, Value *v)
{
    v->type = type;
    switch (type) {
    case LFM_GGUF_TYPE_U8: v->u = p[0]; break;
    case LFM_GGUF_TYPE_I8: v->i = (int8_t)p[0]; break;
    case LFM_GGUF_TYPE_BOOL:
        if (p[0] > 1)
            return fail(LFM_EINVAL, "invalid BOOL value: %u", p[0]);
        v->u = p[0];
        break;
    case LFM_GGUF_TYPE_U16: { uint16_t x; memcpy(&x, p, 2); v->u = x; break; }
    case LFM_GGUF_TYPE_I16: { int16_t x; memcpy(&x, p, 2); v->i = x; break; }
    case LFM_GGUF_TYPE_U32: { uint32_t x; memcpy(&x, p, 4); v->u = x; break; }
    case LFM_GGUF_TYPE_I32: { int32_t x; memcpy(&x, p, 4); v->i = x; break; }
    case LFM_GGUF_TYPE_F32: { float x; memcpy(&x, p, 4); v->f = x; break; }
    case LFM_GGUF_TYPE_U64: memcpy(&v->u, p, 8); break;
    case LFM_GGUF_TYPE_I64: memcpy(&v->i, p, 8); break;
    case LFM_GGUF_TYPE_F64: memcpy(&v->f, p, 8); break;
    default: return fail(LFM_EINTERNAL, "decode_scalar: type %u", type);
    }
    return LFM_OK;
}

// Bytes of a file, or of a caller's buffer copied in at parse time.
struct Source {
    int fd = -1;
    std::vector<uint8_t> mem;
    uint64_t len = 0;

    // Exactly n bytes at `off`; a short read is a truncated file.
    int read(void *dst, uint64_t n, uint64_t off) const
    {
        if (off > len || n > len - off)
            return fail(LFM_EINVAL, "unexpected end of file (truncated input)");
        if (fd < 0) {
            memcpy(dst, mem.data() + off, n);
            return LFM_OK;
        }
        uint8_t *d = (uint8_t *)dst;
        while (n) {
            const size_t chunk = (size_t)std::min<uint64_t>(n, 1u << 30);
            const ssize_t r = pread(fd, d, chunk, (off_t)off);
            if (r < 0 && errno == EINTR)
                continue;
            if (r < 0)
                return fail(LFM_EINVAL, "read error: %s", strerror(errno));
            if (r == 0)
                return fail(LFM_EINVAL, "unexpected end of file (truncated input)");
            d += r;
            off += (uint64_t)r;
            n -= (uint64_t)r;
        }
        return LFM_OK;
    }
};

// Sequential reads of the header through a 1 MiB window.
class Cursor {
  public:
    explicit Cursor(const Source &s) : src_(s), buf_(1u << 20) {}
    uint64_t pos() const { return pos_; }
    uint64_t left() const { return pos_ < src_.len ? src_.len - pos_ : 0; }

    int get(void *dst, uint64_t n)
    {
        uint8_t *d = (uint8_t *)dst;
        while (n) {
            if (pos_ >= base_ && pos_ < base_ + have_) {
                const uint64_t k = std::min(n, base_ + have_ - pos_);
                memcpy(d, buf_.data() + (pos_ - base_), k);
                d += k;
                pos_ += k;
                n -= k;
                continue;
            }
            if (pos_ >= src_.len)
                return fail(LFM_EINVAL, "unexpected end of file (truncated input)");
            const uint64_t want = std::min<uint64_t>(buf_.size(), src_.len - pos_);
            RC(src_.read(buf_.data(), want, pos_));
            base_ = pos_;
            have_ = want;
        }
        return LFM_OK;
    }
    int u32(uint32_t *v) { return get(v, 4); }
    int u64(uint64_t *v) { return get(v, 8); }
    int string(std::string *s)
    {
        uint64_t n;
        RC(u64(&n));
        if (n > kMaxString)
            return fail(LFM_EINVAL, "string length %llu exceeds maximum (1 GiB)",
                        (unsigned long long)n);
        if (n > left())
            return fail(LFM_EINVAL, "unexpected end of file (truncated input)");
        s->resize((size_t)n);
        RC(get(&(*s)[0], n));
        if (!valid_utf8((const uint8_t *)s->data(), s->size()))
            return fail(LFM_EINVAL, "invalid UTF-8 in string");
        return LFM_OK;
    }

  private:
    const Source &src_;
    std::vector<uint8_t> buf_;
    uint64_t pos_ = 0, base_ = 0, have_ = 0;
};

int read_value(Cursor &c, uint32_t type, Value *v, int depth)
{
    size_t size;
    if (scalar_size(type, &size)) {
        uint8_t b[8];
        RC(c.get(b, size));
        return decode_scalar(type, b, v);
    }
    v->type = type;
    if (type == LFM_GGUF_TYPE_STRING)
        return c.string(&v->s);
    if (type != LFM_GGUF_TYPE_ARRAY)
        return fail(LFM_EINVAL, "unknown metadata value type: %u", type);
    if (depth >= kMaxNesting)
        return fail(LFM_EINVAL, "arrays nested deeper than %d levels", kMaxNesting);
    uint64_t n;
    RC(c.u32(&v->elem));
    RC(c.u64(&n));
    if (n > kMaxArray)
        return fail(LFM_EINVAL, "array length %llu exceeds maximum (10 M)", (unsigned long long)n);
    // Elements of a known type take at least `least` bytes each: a count the rest
    // of the file cannot hold is the truncation it would end in, found before
    // building n values.
    size_t least = 0;
    if (!scalar_size(v->elem, &least))
        least = v->elem == LFM_GGUF_TYPE_STRING ? 8 : v->elem == LFM_GGUF_TYPE_ARRAY ? 12 : 0;
    if (least && n > c.left() / least)
        return fail(LFM_EINVAL, "unexpected end of file (truncated input)");
    v->a.reserve((size_t)std::min<uint64_t>(n, 4096));
    for (uint64_t k = 0; k < n; ++k) {
        v->a.emplace_back();
        RC(read_value(c, v->elem, &v->a.back(), depth + 1));
    }
    return LFM_OK;
}

struct TensorEntry {
    std::string name;
    std::vector<uint64_t> ne;
    uint32_t type = 0;
    uint64_t offset = 0; // relative to data_offset, as stored
    uint64_t nbytes = 0;
};

// ---- writer serialization
void put(std::vector<uint8_t> &b, const void *p, size_t n)
{
    b.insert(b.end(), (const uint8_t *)p, (const uint8_t *)p + n);
}
void put_u32(std::vector<uint8_t> &b, uint32_t v) { put(b, &v, 4); }
void put_u64(std::vector<uint8_t> &b, uint64_t v) { put(b, &v, 8); }
void put_string(std::vector<uint8_t> &b, const std::string &s)
{
    put_u64(b, s.size());
    put(b, s.data(), s.size());
}

// A value's payload (no type tag); array elements carry no tags of their own.
void put_payload(std::vector<uint8_t> &b, const Value &v)
{
    switch (v.type) {
    case LFM_GGUF_TYPE_U8: case LFM_GGUF_TYPE_BOOL: { uint8_t x = (uint8_t)v.u; put(b, &x, 1); break; }
    case LFM_GGUF_TYPE_I8: { int8_t x = (int8_t)v.i; put(b, &x, 1); break; }
    case LFM_GGUF_TYPE_U16: { uint16_t x = (uint16_t)v.u; put(b, &x, 2); break; }
    case LFM_GGUF_TYPE_I16: { int16_t x = (int16_t)v.i; put(b, &x, 2); break; }
    case LFM_GGUF_TYPE_U32: put_u32(b, (uint32_t)v.u); break;
    case LFM_GGUF_TYPE_I32: { int32_t x = (int32_t)v.i; put(b, &x, 4); break; }
    case LFM_GGUF_TYPE_F32: { float x = (float)v.f; put(b, &x, 4); break; }
    case LFM_GGUF_TYPE_U64: put_u64(b, v.u); break;
    case LFM_GGUF_TYPE_I64: put(b, &v.i, 8); break;
    case LFM_GGUF_TYPE_F64: put(b, &v.f, 8); break;
    case LFM_GGUF_TYPE_STRING: put_string(b, v.s); break;
    case LFM_GGUF_TYPE_ARRAY:
        put_u32(b, v.elem);
        put_u64(b, v.a.size());
        for (const Value &e : v.a)
            put_payload(b, e);
        break;
    }
}

int write_all(int fd, const void *p, uint64_t n, uint64_t off)
{
    const uint8_t *s = (const uint8_t *)p;
    while (n) {
        const size_t chunk = (size_t)std::min<uint64_t>(n, 1u << 30);
        const ssize_t r = pwrite(fd, s, chunk, (off_t)off);
        if (r < 0 && errno == EINTR)
            continue;
        if (r <= 0)
            return fail(LFM_EINVAL, "write error: %s", r < 0 ? strerror(errno) : "no progress");
        s += r;
        off += (uint64_t)r;
        n -= (uint64_t)r;
    }
    return LFM_OK;
}

void fill_value(const Value &v, lfm_gguf_value *out)
{
    memset(out, 0, sizeof(*out));
    out->type = v.type;
    out->elem_type = v.elem;
    out->u64 = v.u;
    out->i64 = v.i;
    out->f64 = v.f;
    if (v.type == LFM_GGUF_TYPE_STRING) {
        out->str = v.s.c_str();
        out->len = v.s.size();
    } else if (v.type == LFM_GGUF_TYPE_ARRAY) {
        out->len = v.a.size();
    }
}

} // namespace

struct lfm_gguf {
    Source src;
    uint32_t version = 0;
    uint32_t alignment = kDefaultAlign;
    uint64_t data_offset = 0;
    std::map<std::string, Value> meta; // byte-wise key order
    std::vector<const std::string *> keys;
    std::vector<TensorEntry> tensors;
    std::unordered_map<std::string, size_t> by_name;
};

struct lfm_gguf_writer {
    std::vector<std::pair<std::string, Value>> kv; // file order; a repeated key replaces
    std::vector<TensorEntry> tensors;
    std::vector<bool> written;
    std::unordered_map<std::string, size_t> by_name;
    int fd = -1;
    uint32_t alignment = kDefaultAlign;
    uint64_t data_offset = 0;
    uint64_t data_end = 0;
};

// ------------------------------------------------------------------ reader
// gguf.rs:299-440 (parse) + model_file.rs:30-58 (ModelFile::open).
static int parse(lfm_gguf *g)
{
    Cursor c(g->src);
    char magic[4];
    RC(c.get(magic, 4));
    if (memcmp(magic, "GGUF", 4))
        return fail(LFM_EINVAL, "invalid magic (expected \"GGUF\")");
    RC(c.u32(&g->version));
    if (g->version != kVersion)
        return fail(LFM_EINVAL, "unsupported GGUF version: %u (expected 3)", g->version);
    uint64_t n_tensors, n_kv;
    RC(c.u64(&n_tensors));
    RC(c.u64(&n_kv));
    if (n_tensors > kMaxCount)
        return fail(LFM_EINVAL, "tensor count %llu exceeds maximum (100000)",
                    (unsigned long long)n_tensors);
    if (n_kv > kMaxCount)
        return fail(LFM_EINVAL, "KV count %llu exceeds maximum (100000)", (unsigned long long)n_kv);

    for (uint64_t k = 0; k < n_kv; ++k) {
        std::string key;
        uint32_t type;
        Value v;
        RC(c.string(&key));
        if (key.find('\0') != std::string::npos)
            return fail(LFM_EINVAL, "metadata key contains a NUL byte (not addressable by name)");
        RC(c.u32(&type));
        RC(read_value(c, type, &v, 0));
        if (!g->meta.emplace(key, std::move(v)).second)
            return fail(LFM_EINVAL, "duplicate metadata key: %s", key.c_str());
    }
    auto al = g->meta.find("general.alignment");
    g->alignment = al != g->meta.end() && al->second.type == LFM_GGUF_TYPE_U32
                       ? (uint32_t)al->second.u
                       : kDefaultAlign;
    if (!power_of_two(g->alignment))
        return fail(LFM_EINVAL, "invalid alignment: %u (must be a power of two)", g->alignment);

    g->tensors.reserve((size_t)std::min<uint64_t>(n_tensors, 4096));
    for (uint64_t k = 0; k < n_tensors; ++k) {
        TensorEntry t;
        uint32_t nd;
        RC(c.string(&t.name));
        if (t.name.find('\0') != std::string::npos)
            return fail(LFM_EINVAL, "tensor name contains a NUL byte (not addressable by name)");
        RC(c.u32(&nd));
        if (nd > kMaxDims)
            return fail(LFM_EINVAL, "too many dimensions: %u (max 8)", nd);
        t.ne.resize(nd);
        for (uint32_t d = 0; d < nd; ++d)
            RC(c.u64(&t.ne[d]));
        RC(c.u32(&t.type));
        RC(c.u64(&t.offset));
        RC(tensor_nbytes(t.type, t.ne.data(), nd, &t.nbytes));
        if (!g->by_name.emplace(t.name, g->tensors.size()).second)
            return fail(LFM_EINVAL, "duplicate tensor name: %s", t.name.c_str());
        g->tensors.push_back(std::move(t));
    }

    g->data_offset = align_up(c.pos(), g->alignment);
    if (g->data_offset > g->src.len)
        return fail(LFM_EINVAL, "data offset %llu exceeds file length %llu",
                    (unsigned long long)g->data_offset, (unsigned long long)g->src.len);
    const uint64_t data_size = g->src.len - g->data_offset;
    for (const TensorEntry &t : g->tensors) {
        uint64_t end;
        if (t.offset > data_size)
            return fail(LFM_EINVAL, "tensor \"%s\" offset %llu exceeds data size %llu",
                        t.name.c_str(), (unsigned long long)t.offset,
                        (unsigned long long)data_size);
        if (__builtin_add_overflow(t.offset, t.nbytes, &end))
            return fail(LFM_EINVAL, "tensor \"%s\" offset+nbytes overflow", t.name.c_str());
        if (end > data_size)
            return fail(LFM_EINVAL, "tensor \"%s\" end %llu exceeds data size %llu",
                        t.name.c_str(), (unsigned long long)end, (unsigned long long)data_size);
    }
    for (const auto &kv : g->meta)
        g->keys.push_back(&kv.first);
    return LFM_OK;
}

static int finish_open(lfm_gguf *g, lfm_gguf **out)
{
    const int rc = parse(g);
    if (rc != LFM_OK) {
        lfm_gguf_close(g);
        return rc;
    }
    *out = g;
    return LFM_OK;
}

extern "C" int lfm_gguf_open(const char *path, lfm_gguf **out)
{
    if (!path || !out)
        return fail(LFM_EINVAL, "null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0)
        return fail(LFM_EINVAL, "open model file %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int err = errno;
        close(fd);
        return fail(LFM_EINVAL, "stat model file %s: %s", path, strerror(err));
    }
    lfm_gguf *g = new lfm_gguf();
    g->src.fd = fd;
    g->src.len = (uint64_t)st.st_size;
    return finish_open(g, out);
}

extern "C" int lfm_gguf_parse_memory(const void *data, size_t len, lfm_gguf **out)
{
    if ((!data && len) || !out)
        return fail(LFM_EINVAL, "null argument");
    *out = nullptr;
    lfm_gguf *g = new lfm_gguf();
    g->src.mem.assign((const uint8_t *)data, (const uint8_t *)data + len);
    g->src.len = len;
    return finish_open(g, out);
}

extern "C" void lfm_gguf_close(lfm_gguf *g)
{
    if (!g)
        return;
    if (g->src.fd >= 0)
        close(g->src.fd);
    delete g;
}

extern "C" int lfm_gguf_header(const lfm_gguf *g, uint32_t *version, uint32_t *alignment,
                               uint64_t *data_offset, uint64_t *n_kv, uint64_t *n_tensors)
{
    if (!g)
        return fail(LFM_EINVAL, "null gguf");
    if (version)
        *version = g->version;
    if (alignment)
        *alignment = g->alignment;
    if (data_offset)
        *data_offset = g->data_offset;
    if (n_kv)
        *n_kv = g->meta.size();
    if (n_tensors)
        *n_tensors = g->tensors.size();
    return LFM_OK;
}

extern "C" int lfm_gguf_meta_key(const lfm_gguf *g, uint64_t index, const char **key)
{
    if (!g || !key)
        return fail(LFM_EINVAL, "null argument");
    if (index >= g->keys.size())
        return fail(LFM_ERANGE, "metadata index %llu out of range (%zu keys)",
                    (unsigned long long)index, g->keys.size());
    *key = g->keys[index]->c_str();
    return LFM_OK;
}

static int find_meta(const lfm_gguf *g, const char *key, const Value **v)
{
    if (!g || !key)
        return fail(LFM_EINVAL, "null argument");
    auto it = g->meta.find(key);
    if (it == g->meta.end())
        return fail(LFM_ENOTFOUND, "metadata %s missing", key);
    *v = &it->second;
    return LFM_OK;
}

extern "C" int lfm_gguf_meta_get(const lfm_gguf *g, const char *key, lfm_gguf_value *out)
{
    const Value *v;
    RC(find_meta(g, key, &v));
    if (!out)
        return fail(LFM_EINVAL, "null argument");
    fill_value(*v, out);
    return LFM_OK;
}

extern "C" int lfm_gguf_meta_array_get(const lfm_gguf *g, const char *key, uint64_t index,
                                       lfm_gguf_value *out)
{
    const Value *v;
    RC(find_meta(g, key, &v));
    if (!out)
        return fail(LFM_EINVAL, "null argument");
    if (v->type != LFM_GGUF_TYPE_ARRAY)
        return fail(LFM_EINVAL, "metadata %s is not an array", key);
    if (index >= v->a.size())
        return fail(LFM_ERANGE, "metadata %s: index %llu out of range (%zu elements)", key,
                    (unsigned long long)index, v->a.size());
    fill_value(v->a[index], out);
    return LFM_OK;
}

// ModelFile::meta_u32 (model_file.rs:131-140): U32, U64, I32, I64 and U8 values,
// wider ones truncated to 32 bits.
extern "C" int lfm_gguf_meta_u32(const lfm_gguf *g, const char *key, uint32_t *out)
{
    const Value *v;
    RC(find_meta(g, key, &v));
    if (!out)
        return fail(LFM_EINVAL, "null argument");
    switch (v->type) {
    case LFM_GGUF_TYPE_U32: case LFM_GGUF_TYPE_U64: case LFM_GGUF_TYPE_U8:
        *out = (uint32_t)v->u;
        return LFM_OK;
    case LFM_GGUF_TYPE_I32: case LFM_GGUF_TYPE_I64:
        *out = (uint32_t)v->i;
        return LFM_OK;
    default:
        return fail(LFM_EINVAL, "metadata %s not a u32 (type %u)", key, v->type);
    }
}

// ModelFile::meta_f32 (model_file.rs:146-152): F32, or F64 rounded to f32.
extern "C" int lfm_gguf_meta_f32(const lfm_gguf *g, const char *key, float *out)
{
    const Value *v;
    RC(find_meta(g, key, &v));
    if (!out)
        return fail(LFM_EINVAL, "null argument");
    if (v->type != LFM_GGUF_TYPE_F32 && v->type != LFM_GGUF_TYPE_F64)
        return fail(LFM_EINVAL, "metadata %s not an f32 (type %u)", key, v->type);
    *out = (float)v->f;
    return LFM_OK;
}

// ModelFile::meta_str (model_file.rs:158-163).  *len is the byte length; the
// copy is NUL-terminated and needs cap >= len + 1.
extern "C" int lfm_gguf_meta_str(const lfm_gguf *g, const char *key, char *buf, size_t cap,
                                 size_t *len)
{
    const Value *v;
    RC(find_meta(g, key, &v));
    if (v->type != LFM_GGUF_TYPE_STRING)
        return fail(LFM_EINVAL, "metadata %s not a string (type %u)", key, v->type);
    if (len)
        *len = v->s.size();
    if (!buf || cap < v->s.size() + 1)
        return fail(LFM_ERANGE, "metadata %s: %zu bytes need a buffer of %zu", key, v->s.size(),
                    v->s.size() + 1);
    memcpy(buf, v->s.c_str(), v->s.size() + 1);
    return LFM_OK;
}

// ModelFile::meta_u32_array (model_file.rs:166-182): an array of U32, I32, U16,
// I16, U8 or I8 elements.  *len is the element count; cap may be 0 to query it.
extern "C" int lfm_gguf_meta_u32_array(const lfm_gguf *g, const char *key, uint32_t *out,
                                       size_t cap, size_t *len)
{
    const Value *v;
    RC(find_meta(g, key, &v));
    if (v->type != LFM_GGUF_TYPE_ARRAY)
        return fail(LFM_EINVAL, "metadata %s not an array (type %u)", key, v->type);
    for (const Value &e : v->a)
        if (e.type != LFM_GGUF_TYPE_U32 && e.type != LFM_GGUF_TYPE_I32 &&
            e.type != LFM_GGUF_TYPE_U16 && e.type != LFM_GGUF_TYPE_I16 &&
            e.type != LFM_GGUF_TYPE_U8 && e.type != LFM_GGUF_TYPE_I8)
            return fail(LFM_EINVAL, "metadata %s: array element not int (type %u)", key, e.type);
    if (len)
        *len = v->a.size();
    if (cap < v->a.size() || (!out && !v->a.empty()))
        return fail(LFM_ERANGE, "metadata %s: %zu elements, capacity %zu", key, v->a.size(), cap);
    for (size_t k = 0; k < v->a.size(); ++k) {
        const Value &e = v->a[k];
        const bool is_signed = e.type == LFM_GGUF_TYPE_I32 || e.type == LFM_GGUF_TYPE_I16 ||
                               e.type == LFM_GGUF_TYPE_I8;
        out[k] = is_signed ? (uint32_t)e.i : (uint32_t)e.u;
    }
    return LFM_OK;
}

extern "C" int lfm_gguf_tensor_info(const lfm_gguf *g, uint64_t index, lfm_gguf_tensor *out)
{
    if (!g || !out)
        return fail(LFM_EINVAL, "null argument");
    if (index >= g->tensors.size())
        return fail(LFM_ERANGE, "tensor index %llu out of range (%zu tensors)",
                    (unsigned long long)index, g->tensors.size());
    const TensorEntry &t = g->tensors[index];
    memset(out, 0, sizeof(*out));
    out->name = t.name.c_str();
    out->ggml_type = t.type;
    out->n_dims = (uint32_t)t.ne.size();
    for (size_t d = 0; d < t.ne.size(); ++d)
        out->ne[d] = t.ne[d];
    out->offset = t.offset;
    out->file_offset = g->data_offset + t.offset;
    out->nbytes = t.nbytes;
    return LFM_OK;
}

extern "C" int lfm_gguf_find_tensor(const lfm_gguf *g, const char *name, uint64_t *index)
{
    if (!g || !name || !index)
        return fail(LFM_EINVAL, "null argument");
    auto it = g->by_name.find(name);
    if (it == g->by_name.end())
        return fail(LFM_ENOTFOUND, "missing tensor %s", name);
    *index = it->second;
    return LFM_OK;
}

// ModelFile::read_tensor_range (model_file.rs:111-122).
extern "C" int lfm_gguf_read_tensor_range(const lfm_gguf *g, const char *name, uint64_t byte_off,
                                          void *dst, uint64_t len)
{
    uint64_t i, end;
    RC(lfm_gguf_find_tensor(g, name, &i));
    const TensorEntry &t = g->tensors[i];
    if (__builtin_add_overflow(byte_off, len, &end) || end > t.nbytes)
        return fail(LFM_ERANGE, "range exceeds tensor %s", name);
    if (!dst && len)
        return fail(LFM_EINVAL, "null destination");
    return g->src.read(dst, len, g->data_offset + t.offset + byte_off);
}

// ModelFile::read_tensor_into (model_file.rs:100-109): the destination holds
// exactly the tensor's bytes.
extern "C" int lfm_gguf_read_tensor(const lfm_gguf *g, const char *name, void *dst, size_t len)
{
    uint64_t i;
    RC(lfm_gguf_find_tensor(g, name, &i));
    if (len != g->tensors[i].nbytes)
        return fail(LFM_EINVAL, "tensor destination length: %zu given, %llu needed", len,
                    (unsigned long long)g->tensors[i].nbytes);
    return lfm_gguf_read_tensor_range(g, name, 0, dst, len);
}

// load_hyperparams (engine/src/lfm.rs:102-145): the same keys, defaults and order
// of checks.  `strict` applies the reference's fixed LFM2.5-8B-A1B geometry;
// without it any geometry the engine accepts may be read (reduced test models).
extern "C" int lfm_gguf_hparams(const lfm_gguf *g, int strict, lfm_hparams *out)
{
    if (!g || !out)
        return fail(LFM_EINVAL, "null argument");
    lfm_hparams hp;
    memset(&hp, 0, sizeof(hp));
    uint32_t kv[LFM_MAX_LAYERS];
    size_t n_kv = 0;
    RC(lfm_gguf_meta_u32(g, "lfm2moe.block_count", &hp.n_layers));
    RC(lfm_gguf_meta_u32(g, "lfm2moe.embedding_length", &hp.dim));
    RC(lfm_gguf_meta_u32(g, "lfm2moe.attention.head_count", &hp.heads));
    const int kv_rc = lfm_gguf_meta_u32_array(g, "lfm2moe.attention.head_count_kv", kv,
                                              LFM_MAX_LAYERS, &n_kv);
    if (kv_rc == LFM_ERANGE)
        return fail(LFM_EINVAL, "head_count_kv has %zu entries (at most %d layers)", n_kv,
                    LFM_MAX_LAYERS);
    RC(kv_rc);
    RC(lfm_gguf_meta_u32(g, "lfm2moe.vocab_size", &hp.vocab));
    RC(lfm_gguf_meta_u32(g, "lfm2moe.expert_count", &hp.n_expert));
    RC(lfm_gguf_meta_u32(g, "lfm2moe.expert_used_count", &hp.n_used));
    RC(lfm_gguf_meta_u32(g, "lfm2moe.expert_feed_forward_length", &hp.expert_ff));
    RC(lfm_gguf_meta_u32(g, "lfm2moe.feed_forward_length", &hp.n_ff));
    // meta_u32_default: any failure (missing or not an integer) takes the default.
    if (lfm_gguf_meta_u32(g, "lfm2moe.leading_dense_block_count", &hp.dense_lead) != LFM_OK)
        hp.dense_lead = 2;
    if (lfm_gguf_meta_u32(g, "lfm2moe.shortconv.l_cache", &hp.conv_l_cache) != LFM_OK)
        hp.conv_l_cache = 3;
    if (strict && (hp.dim != 2048 || hp.heads != 32 || hp.n_layers != 24 || hp.vocab != 128000 ||
                   hp.n_expert != 32 || hp.n_used != 4 || hp.expert_ff != 1792))
        return fail(LFM_EINVAL,
                    "unsupported geometry: dim=%u heads=%u layers=%u vocab=%u n_expert=%u "
                    "n_used=%u expert_ff=%u",
                    hp.dim, hp.heads, hp.n_layers, hp.vocab, hp.n_expert, hp.n_used, hp.expert_ff);
    if (hp.n_layers == 0 || hp.n_layers > LFM_MAX_LAYERS)
        return fail(LFM_EINVAL, "block_count %u outside 1..%d", hp.n_layers, LFM_MAX_LAYERS);
    if (n_kv != hp.n_layers)
        return fail(LFM_EINVAL, "head_count_kv has %zu entries for %u layers", n_kv, hp.n_layers);
    for (uint32_t l = 0; l < hp.n_layers; ++l)
        hp.kv_heads[l] = kv[l];
    hp.head_dim = 64;
    RC(lfm_gguf_meta_f32(g, "lfm2moe.attention.layer_norm_rms_epsilon", &hp.eps));
    RC(lfm_gguf_meta_f32(g, "lfm2moe.rope.freq_base", &hp.rope_theta));
    if (lfm_gguf_meta_u32(g, "tokenizer.ggml.eos_token_id", &hp.eos) != LFM_OK)
        hp.eos = 124900;
    *out = hp;
    return LFM_OK;
}

// ------------------------------------------------------------------ engine loading
// GpuEngine::load's staging loop (engine/src/gpu_lfm.rs:64-97): every F32 and
// Q6_K tensor, in file order, is read into one host staging buffer sized for the
// largest and uploaded; tensors of other types are skipped.
// Every F32 / Q6_K tensor of the file has a shape the engine takes (no zero
// dimension, whole Q6_K rows): checked on the host before any upload.
static int check_gguf_tensors(const lfm_gguf *g)
{
    for (const TensorEntry &t : g->tensors) {
        if (t.type != LFM_GGML_TYPE_F32 && t.type != LFM_GGML_TYPE_Q6_K)
            continue;
        if (t.ne.size() > 4)
            return fail(LFM_EINVAL, "%s: %zu dimensions (the engine takes 1..4)", t.name.c_str(),
                        t.ne.size());
        size_t want = 0;
        RC(lfm_check_tensor(t.name.c_str(), t.type, t.ne.data(), (uint32_t)t.ne.size(), &want));
        if (want != t.nbytes)
            return fail(LFM_EINTERNAL, "%s: %zu bytes by shape, %llu in the file table",
                        t.name.c_str(), want, (unsigned long long)t.nbytes);
    }
    return LFM_OK;
}

extern "C" int lfm_engine_load_gguf(lfm_engine *e, const lfm_gguf *g)
{
    if (!e || !g)
        return fail(LFM_EINVAL, "null argument");
    RC(check_gguf_tensors(g));
    uint64_t most = 0;
    for (const TensorEntry &t : g->tensors)
        if (t.type == LFM_GGML_TYPE_F32 || t.type == LFM_GGML_TYPE_Q6_K)
            most = std::max(most, t.nbytes);
    std::vector<uint8_t> staging((size_t)std::max<uint64_t>(most, 4));
    for (const TensorEntry &t : g->tensors) {
        if (t.type != LFM_GGML_TYPE_F32 && t.type != LFM_GGML_TYPE_Q6_K)
            continue;
        RC(g->src.read(staging.data(), t.nbytes, g->data_offset + t.offset));
        RC(lfm_engine_upload_tensor(e, t.name.c_str(), t.type, t.ne.data(),
                                    (uint32_t)t.ne.size(), staging.data(), (size_t)t.nbytes));
    }
    return LFM_OK;
}

// ModelFile::open + GpuEngine::load + set_ctx (gpu_lfm.rs:51-120): a finalized
// engine with the file's hyper-parameters and tensors.
extern "C" int lfm_engine_open_gguf(const char *path, int device, uint32_t ctx, int strict,
                                    lfm_engine **out)
{
    if (!out)
        return fail(LFM_EINVAL, "null argument");
    *out = nullptr;
    lfm_gguf *g = nullptr;
    RC(lfm_gguf_open(path, &g));
    lfm_hparams hp;
    lfm_engine *e = nullptr;
    int rc = check_gguf_tensors(g);
    if (rc == LFM_OK)
        rc = lfm_gguf_hparams(g, strict, &hp);
    if (rc == LFM_OK && (hp.n_expert < 4 || hp.n_expert > 64))
        rc = fail(LFM_EINVAL, "resident routing supports 4..=64 experts");
    if (rc == LFM_OK)
        rc = lfm_engine_create(&hp, device, &e);
    if (rc == LFM_OK && ctx)
        rc = lfm_engine_set_ctx(e, ctx);
    if (rc == LFM_OK)
        rc = lfm_engine_load_gguf(e, g);
    if (rc == LFM_OK)
        rc = lfm_engine_finalize(e);
    lfm_gguf_close(g);
    if (rc != LFM_OK) {
        lfm_engine_destroy(e);
        return rc;
    }
    *out = e;
    return LFM_OK;
}

// ------------------------------------------------------------------ writer
extern "C" int lfm_gguf_writer_create(lfm_gguf_writer **out)
{
    if (!out)
        return fail(LFM_EINVAL, "null argument");
    *out = new lfm_gguf_writer();
    return LFM_OK;
}

extern "C" void lfm_gguf_writer_free(lfm_gguf_writer *w)
{
    if (!w)
        return;
    if (w->fd >= 0)
        close(w->fd);
    delete w;
}

static int writer_set(lfm_gguf_writer *w, const char *key, Value &&v)
{
    if (!w || !key)
        return fail(LFM_EINVAL, "null argument");
    if (w->fd >= 0)
        return fail(LFM_ESTATE, "metadata must be set before lfm_gguf_writer_begin");
    if (!valid_utf8((const uint8_t *)key, strlen(key)))
        return fail(LFM_EINVAL, "key is not valid UTF-8");
    for (auto &kv : w->kv)
        if (kv.first == key) {
            kv.second = std::move(v);
            return LFM_OK;
        }
    if (w->kv.size() >= kMaxCount)
        return fail(LFM_ERANGE, "more than %llu metadata pairs", (unsigned long long)kMaxCount);
    w->kv.emplace_back(key, std::move(v));
    return LFM_OK;
}

extern "C" int lfm_gguf_writer_set_scalar(lfm_gguf_writer *w, const char *key, uint32_t type,
                                          const void *value)
{
    size_t size;
    if (!scalar_size(type, &size))
        return fail(LFM_EINVAL, "type %u is not a scalar type", type);
    if (!value)
        return fail(LFM_EINVAL, "null value");
    Value v;
    RC(decode_scalar(type, (const uint8_t *)value, &v));
    return writer_set(w, key, std::move(v));
}

static int string_value(const char *s, uint64_t len, Value *v)
{
    if (!s && len)
        return fail(LFM_EINVAL, "null string");
    if (len > kMaxString)
        return fail(LFM_EINVAL, "string length %llu exceeds maximum (1 GiB)",
                    (unsigned long long)len);
    if (!valid_utf8((const uint8_t *)s, (size_t)len))
        return fail(LFM_EINVAL, "string is not valid UTF-8");
    v->type = LFM_GGUF_TYPE_STRING;
    v->s.assign(s ? s : "", (size_t)len);
    return LFM_OK;
}

extern "C" int lfm_gguf_writer_set_string(lfm_gguf_writer *w, const char *key, const char *s,
                                          uint64_t len)
{
    Value v;
    RC(string_value(s, len, &v));
    return writer_set(w, key, std::move(v));
}

extern "C" int lfm_gguf_writer_set_array(lfm_gguf_writer *w, const char *key, uint32_t elem_type,
                                         const void *values, uint64_t count)
{
    size_t size;
    if (!scalar_size(elem_type, &size))
        return fail(LFM_EINVAL, "element type %u is not a scalar type", elem_type);
    if (count > kMaxArray)
        return fail(LFM_EINVAL, "array length %llu exceeds maximum (10 M)",
                    (unsigned long long)count);
    if (!values && count)
        return fail(LFM_EINVAL, "null values");
    Value v;
    v.type = LFM_GGUF_TYPE_ARRAY;
    v.elem = elem_type;
    v.a.resize((size_t)count);
    for (uint64_t k = 0; k < count; ++k)
        RC(decode_scalar(elem_type, (const uint8_t *)values + k * size, &v.a[k]));
    return writer_set(w, key, std::move(v));
}

extern "C" int lfm_gguf_writer_set_string_array(lfm_gguf_writer *w, const char *key,
                                                const char *const *strs, const uint64_t *lens,
                                                uint64_t count)
{
    if (count > kMaxArray)
        return fail(LFM_EINVAL, "array length %llu exceeds maximum (10 M)",
                    (unsigned long long)count);
    if (!strs && count)
        return fail(LFM_EINVAL, "null strings");
    Value v;
    v.type = LFM_GGUF_TYPE_ARRAY;
    v.elem = LFM_GGUF_TYPE_STRING;
    v.a.resize((size_t)count);
    for (uint64_t k = 0; k < count; ++k)
        RC(string_value(strs[k], lens ? lens[k] : (strs[k] ? strlen(strs[k]) : 0), &v.a[k]));
    return writer_set(w, key, std::move(v));
}

extern "C" int lfm_gguf_writer_add_tensor(lfm_gguf_writer *w, const char *name, uint32_t ggml_type,
                                          uint32_t n_dims, const uint64_t *ne, uint64_t *index)
{
    if (!w || !name || (!ne && n_dims))
        return fail(LFM_EINVAL, "null argument");
    if (w->fd >= 0)
        return fail(LFM_ESTATE, "tensors must be added before lfm_gguf_writer_begin");
    if (n_dims > kMaxDims)
        return fail(LFM_EINVAL, "too many dimensions: %u (max 8)", n_dims);
    if (!valid_utf8((const uint8_t *)name, strlen(name)))
        return fail(LFM_EINVAL, "tensor name is not valid UTF-8");
    if (w->tensors.size() >= kMaxCount)
        return fail(LFM_ERANGE, "more than %llu tensors", (unsigned long long)kMaxCount);
    TensorEntry t;
    t.name = name;
    t.type = ggml_type;
    t.ne.assign(ne, ne + n_dims);
    RC(tensor_nbytes(ggml_type, ne, n_dims, &t.nbytes));
    if (!w->by_name.emplace(t.name, w->tensors.size()).second)
        return fail(LFM_EINVAL, "duplicate tensor name: %s", name);
    if (index)
        *index = w->tensors.size();
    w->tensors.push_back(std::move(t));
    w->written.push_back(false);
    return LFM_OK;
}

// Lays out the data section (each tensor at the next multiple of the alignment)
// and writes everything before it: header, metadata, tensor table, padding.
extern "C" int lfm_gguf_writer_begin(lfm_gguf_writer *w, const char *path)
{
    if (!w || !path)
        return fail(LFM_EINVAL, "null argument");
    if (w->fd >= 0)
        return fail(LFM_ESTATE, "lfm_gguf_writer_begin called twice");
    w->alignment = kDefaultAlign;
    for (const auto &kv : w->kv)
        if (kv.first == "general.alignment" && kv.second.type == LFM_GGUF_TYPE_U32)
            w->alignment = (uint32_t)kv.second.u;
    if (!power_of_two(w->alignment))
        return fail(LFM_EINVAL, "invalid alignment: %u (must be a power of two)", w->alignment);
    uint64_t off = 0;
    for (TensorEntry &t : w->tensors) {
        off = align_up(off, w->alignment);
        t.offset = off;
        off += t.nbytes;
    }
    w->data_end = align_up(off, w->alignment);

    std::vector<uint8_t> head;
    put(head, "GGUF", 4);
    put_u32(head, kVersion);
    put_u64(head, w->tensors.size());
    put_u64(head, w->kv.size());
    for (const auto &kv : w->kv) {
        put_string(head, kv.first);
        put_u32(head, kv.second.type);
        put_payload(head, kv.second);
    }
    for (const TensorEntry &t : w->tensors) {
        put_string(head, t.name);
        put_u32(head, (uint32_t)t.ne.size());
        for (uint64_t d : t.ne)
            put_u64(head, d);
        put_u32(head, t.type);
        put_u64(head, t.offset);
    }
    w->data_offset = align_up(head.size(), w->alignment);
    head.resize((size_t)w->data_offset, 0);

    const int fd = open(path, O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    if (fd < 0)
        return fail(LFM_EINVAL, "create %s: %s", path, strerror(errno));
    w->fd = fd;
    return write_all(fd, head.data(), head.size(), 0);
}

extern "C" int lfm_gguf_writer_write_tensor(lfm_gguf_writer *w, uint64_t index, const void *data,
                                            uint64_t nbytes)
{
    if (!w)
        return fail(LFM_EINVAL, "null writer");
    if (w->fd < 0)
        return fail(LFM_ESTATE, "tensor data is written after lfm_gguf_writer_begin");
    if (index >= w->tensors.size())
        return fail(LFM_ERANGE, "tensor index %llu out of range", (unsigned long long)index);
    const TensorEntry &t = w->tensors[index];
    if (nbytes != t.nbytes)
        return fail(LFM_EINVAL, "%s: %llu bytes given, %llu expected", t.name.c_str(),
                    (unsigned long long)nbytes, (unsigned long long)t.nbytes);
    if (!data && nbytes)
        return fail(LFM_EINVAL, "null data");
    RC(write_all(w->fd, data, nbytes, w->data_offset + t.offset));
    w->written[index] = true;
    return LFM_OK;
}

// Checks that every tensor was written, extends the file to the padded end of
// the data section (gaps read as zeros) and closes it.
extern "C" int lfm_gguf_writer_finish(lfm_gguf_writer *w)
{
    if (!w)
        return fail(LFM_EINVAL, "null writer");
    if (w->fd < 0)
        return fail(LFM_ESTATE, "lfm_gguf_writer_finish before lfm_gguf_writer_begin");
    for (size_t k = 0; k < w->tensors.size(); ++k)
        if (!w->written[k] && w->tensors[k].nbytes)
            return fail(LFM_ESTATE, "tensor %s was not written", w->tensors[k].name.c_str());
    int rc = LFM_OK;
    if (ftruncate(w->fd, (off_t)(w->data_offset + w->data_end)) != 0)
        rc = fail(LFM_EINVAL, "ftruncate: %s", strerror(errno));
    if (close(w->fd) != 0 && rc == LFM_OK)
        rc = fail(LFM_EINVAL, "close: %s", strerror(errno));
    w->fd = -1;
    return rc;
}

// The lfm2moe metadata that load_hyperparams reads (engine/src/lfm.rs:102-145),
// with general.architecture; head_count_kv is written as an I32 array, one entry
// per layer.
extern "C" int lfm_gguf_writer_set_hparams(lfm_gguf_writer *w, const lfm_hparams *hp)
{
    if (!w || !hp)
        return fail(LFM_EINVAL, "null argument");
    if (hp->n_layers == 0 || hp->n_layers > LFM_MAX_LAYERS)
        return fail(LFM_EINVAL, "n_layers must be 1..%d", LFM_MAX_LAYERS);
    const char *arch = "lfm2moe";
    RC(lfm_gguf_writer_set_string(w, "general.architecture", arch, strlen(arch)));
    const struct {
        const char *key;
        uint32_t v;
    } u32s[] = {
        {"lfm2moe.block_count", hp->n_layers},
        {"lfm2moe.embedding_length", hp->dim},
        {"lfm2moe.attention.head_count", hp->heads},
        {"lfm2moe.vocab_size", hp->vocab},
        {"lfm2moe.expert_count", hp->n_expert},
        {"lfm2moe.expert_used_count", hp->n_used},
        {"lfm2moe.expert_feed_forward_length", hp->expert_ff},
        {"lfm2moe.feed_forward_length", hp->n_ff},
        {"lfm2moe.leading_dense_block_count", hp->dense_lead},
        {"lfm2moe.shortconv.l_cache", hp->conv_l_cache},
        {"tokenizer.ggml.eos_token_id", hp->eos},
    };
    for (const auto &kv : u32s)
        RC(lfm_gguf_writer_set_scalar(w, kv.key, LFM_GGUF_TYPE_U32, &kv.v));
    int32_t kv[LFM_MAX_LAYERS];
    for (uint32_t l = 0; l < hp->n_layers; ++l)
        kv[l] = (int32_t)hp->kv_heads[l];
    RC(lfm_gguf_writer_set_array(w, "lfm2moe.attention.head_count_kv", LFM_GGUF_TYPE_I32, kv,
                                 hp->n_layers));
    RC(lfm_gguf_writer_set_scalar(w, "lfm2moe.attention.layer_norm_rms_epsilon",
                                  LFM_GGUF_TYPE_F32, &hp->eps));
    RC(lfm_gguf_writer_set_scalar(w, "lfm2moe.rope.freq_base", LFM_GGUF_TYPE_F32,
                                  &hp->rope_theta));
    return LFM_OK;
}

// The seeded synthetic model (the tensors lfm_model_tensor_desc lists, with the
// bytes lfm_synth_tensor generates) as a GGUF file, one tensor in memory at a time.
extern "C" int lfm_gguf_write_synthetic(const char *path, const lfm_hparams *hp,
                                        const lfm_synth_opts *o, int threads)
{
    lfm_synth_opts def;
    if (!o) {
        lfm_synth_default_opts(&def);
        o = &def;
    }
    const int count = lfm_model_tensor_count(hp);
    if (count < 0)
        return fail(LFM_EINVAL, "bad hparams");
    lfm_gguf_writer *w = nullptr;
    RC(lfm_gguf_writer_create(&w));
    std::vector<lfm_tensor_desc> descs((size_t)count);
    const char *name = "lfm2 synthetic (seeded)";
    const uint32_t align = kDefaultAlign;
    int rc = lfm_gguf_writer_set_hparams(w, hp);
    if (rc == LFM_OK)
        rc = lfm_gguf_writer_set_string(w, "general.name", name, strlen(name));
    if (rc == LFM_OK)
        rc = lfm_gguf_writer_set_scalar(w, "general.alignment", LFM_GGUF_TYPE_U32, &align);
    if (rc == LFM_OK)
        rc = lfm_gguf_writer_set_scalar(w, "lfm.synthetic.seed", LFM_GGUF_TYPE_U64, &o->seed);
    for (int i = 0; rc == LFM_OK && i < count; ++i) {
        rc = lfm_model_tensor_desc(hp, o, i, &descs[i]);
        if (rc != LFM_OK)
            rc = fail(rc, "lfm_model_tensor_desc(%d) failed", i);
        else
            rc = lfm_gguf_writer_add_tensor(w, descs[i].name, descs[i].ggml_type, descs[i].n_dims,
                                            descs[i].ne, nullptr);
    }
    if (rc == LFM_OK)
        rc = lfm_gguf_writer_begin(w, path);
    std::vector<uint8_t> buf;
    for (int i = 0; rc == LFM_OK && i < count; ++i) {
        const size_t nb = lfm_tensor_nbytes(&descs[i]);
        buf.resize(nb);
        rc = lfm_synth_tensor(o, &descs[i], buf.data(), nb, threads);
        if (rc != LFM_OK)
            rc = fail(rc, "lfm_synth_tensor(%s) failed", descs[i].name);
        else
            rc = lfm_gguf_writer_write_tensor(w, (uint64_t)i, buf.data(), nb);
    }
    if (rc == LFM_OK)
        rc = lfm_gguf_writer_finish(w);
    lfm_gguf_writer_free(w);
    return rc;
}
