// GGUF reader and writer of the inferi_hip C ABI (host code, no device work).
//
// The reader follows Gguf::from_bytes (crates/inferi/src/gguf.rs:516-692):
// header (magic in either byte order, version, tensor and metadata counts),
// typed metadata (gguf.rs:388-511), tensor infos whose GGUF dimensions are
// reversed into [rows, cols, ...] order (gguf.rs:620-626), and tensor data at
// offsets relative to the aligned end of the infos, the alignment being
// `general.alignment` when it is a U32, else 32 (gguf.rs:519-529, 640).  The
// file is memory-mapped and every tensor's bytes are handed out in place.
// Where the reference panics (a read past the end, rank > 4) or returns an
// error (bad magic, unknown value or tensor type), these functions return
// IFR_EINVAL and ifr_last_error(NULL) says why.
//
// The writer produces the same layout: metadata in insertion order, tensor
// infos in insertion order, each tensor's data at the next multiple of the
// alignment, zero padding.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../include/inferi_hip.h"

std::string &ifr_free_error(); // host.cpp: the message ifr_last_error(NULL) returns

namespace {

#define g_err ifr_free_error()

ifr_status gfail(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return IFR_EINVAL;
}

constexpr uint32_t MAGIC_LE = 0x46554747u; // "GGUF" read as little-endian
constexpr uint32_t MAGIC_BE = 0x47475546u;

// Bytes of one value of a scalar metadata type (0 for string / array).
uint32_t scalar_size(int32_t t) {
    switch (t) {
    case IFR_GGUF_U8: case IFR_GGUF_I8: case IFR_GGUF_BOOL: return 1;
    case IFR_GGUF_U16: case IFR_GGUF_I16: return 2;
    case IFR_GGUF_U32: case IFR_GGUF_I32: case IFR_GGUF_F32: return 4;
    case IFR_GGUF_U64: case IFR_GGUF_I64: case IFR_GGUF_F64: return 8;
    default: return 0;
    }
}

// Tensor types the reference reads (gguf.rs:74-104, 644-692) with their
// block size in elements and bytes; the others are listed with no data.
bool tensor_block(int32_t t, uint32_t &elems, uint32_t &bytes, bool &known) {
    known = true;
    switch (t) {
    case 0: elems = 1; bytes = 4; return true;        // F32
    case 1: elems = 1; bytes = 2; return true;        // F16
    case 2: elems = 32; bytes = 18; return true;      // Q4_0
    case 3: elems = 32; bytes = 20; return true;      // Q4_1
    case 6: elems = 32; bytes = 22; return true;      // Q5_0
    case 7: elems = 32; bytes = 24; return true;      // Q5_1
    case 8: elems = 32; bytes = 34; return true;      // Q8_0
    case 12: elems = 256; bytes = 144; return true;   // Q4_K
    case 13: elems = 256; bytes = 176; return true;   // Q5_K
    case 14: elems = 256; bytes = 210; return true;   // Q6_K
    case 15: elems = 256; bytes = 292; return true;   // Q8_K
    case 9: case 10: case 11: case 16: case 17: case 18: case 19: case 20: case 21: case 22: case 23: case 24:
    case 25: case 26: case 27: case 28: case 29:
        known = false; // a type of the format whose data the reference does not read
        elems = 1;
        bytes = 0;
        return true;
    default: return false;
    }
}

struct Value {
    int32_t type = -1;
    uint64_t raw = 0;         // scalar bits (little-endian, zero-extended)
    std::string str;          // STRING
    int32_t elem_type = -1;   // ARRAY
    uint64_t len = 0;         // ARRAY
    const uint8_t *data = nullptr; // ARRAY of scalars: the elements in the file
    std::vector<std::string> strs; // ARRAY of STRING
};

struct Tensor {
    std::string name;
    int32_t dtype = 0;
    uint32_t rank = 0;
    uint64_t dims[4] = {1, 1, 1, 1}; // reference order: GGUF's reversed
    uint64_t offset = 0;             // from the start of the file
    uint64_t bytes = 0;
    bool has_data = false;
};

struct Reader {
    const uint8_t *p;
    size_t n, off = 0;
    bool ok = true;
    bool take(void *dst, size_t k) {
        if (!ok || k > n - off) return ok = false;
        memcpy(dst, p + off, k);
        off += k;
        return true;
    }
    template <class T>
    bool get(T &v) { return take(&v, sizeof v); }
    bool skip(uint64_t k) {
        if (!ok || k > n - off) return ok = false;
        off += k;
        return true;
    }
    bool str(std::string &s) {
        uint64_t len;
        if (!get(len) || len > n - off) return ok = false;
        s.assign((const char *)p + off, (size_t)len);
        off += len;
        return true;
    }
};

} // namespace

struct ifr_gguf {
    void *map = nullptr;
    size_t map_len = 0;
    std::vector<uint8_t> own; // ifr_gguf_from_bytes copies here
    const uint8_t *base = nullptr;
    size_t len = 0;
    uint32_t version = 0, alignment = 32;
    std::vector<std::pair<std::string, Value>> meta;
    std::map<std::string, size_t> meta_ix;
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> tensor_ix;
    ~ifr_gguf() {
        if (map) munmap(map, map_len);
    }
};

namespace {

bool read_array(Reader &r, Value &v, int depth);

bool read_value(Reader &r, int32_t type, Value &v, int depth) {
    v.type = type;
    if (uint32_t sz = scalar_size(type)) {
        v.raw = 0;
        return r.take(&v.raw, sz);
    }
    if (type == IFR_GGUF_STRING) return r.str(v.str);
    if (type == IFR_GGUF_ARRAY) return read_array(r, v, depth);
    gfail("gguf: metadata value type %d is not part of the supported gguf version", type);
    return r.ok = false;
}

bool read_array(Reader &r, Value &v, int depth) {
    uint32_t et;
    uint64_t len;
    if (!r.get(et) || !r.get(len)) return false;
    if (depth > 8) {
        gfail("gguf: arrays nested deeper than 8");
        return r.ok = false;
    }
    v.elem_type = (int32_t)et;
    v.len = len;
    if (uint32_t sz = scalar_size((int32_t)et)) {
        if (len > (r.n - r.off) / sz) return r.ok = false;
        v.data = r.p + r.off;
        return r.skip(len * sz);
    }
    if (et == IFR_GGUF_STRING) {
        if (len > (r.n - r.off) / 8) return r.ok = false; // each string has an 8-byte length
        v.strs.resize((size_t)len);
        for (uint64_t i = 0; i < len; i++)
            if (!r.str(v.strs[(size_t)i])) return false;
        return true;
    }
    if (et == IFR_GGUF_ARRAY) { // nested arrays are walked (the reference keeps them) but not exposed
        for (uint64_t i = 0; i < len; i++) {
            Value sub;
            if (!read_array(r, sub, depth + 1)) return false;
        }
        return true;
    }
    gfail("gguf: metadata value type %u is not part of the supported gguf version", et);
    return r.ok = false;
}

ifr_status parse(ifr_gguf *g) {
    Reader r{g->base, g->len};
    uint32_t magic = 0;
    uint64_t n_tensors = 0, n_meta = 0;
    if (!r.get(magic)) return gfail("gguf: file shorter than its magic number");
    if (magic != MAGIC_LE && magic != MAGIC_BE)
        return gfail("gguf: the input isn't a ggml binary file (magic %#x instead of 0x46554747 or 0x47475546)", magic);
    if (!r.get(g->version) || !r.get(n_tensors) || !r.get(n_meta)) return gfail("gguf: truncated header");
    for (uint64_t i = 0; i < n_meta; i++) {
        std::string key;
        uint32_t type;
        Value v;
        g_err.clear();
        if (!r.str(key) || !r.get(type) || !read_value(r, (int32_t)type, v, 0))
            return g_err.empty() ? gfail("gguf: truncated in metadata entry %llu", (unsigned long long)i) : IFR_EINVAL;
        auto it = g->meta_ix.find(key);
        if (it != g->meta_ix.end()) { // the reference's map keeps the last value of a repeated key
            g->meta[it->second].second = std::move(v);
        } else {
            g->meta_ix[key] = g->meta.size();
            g->meta.emplace_back(std::move(key), std::move(v));
        }
    }
    auto al = g->meta_ix.find("general.alignment");
    if (al != g->meta_ix.end() && g->meta[al->second].second.type == IFR_GGUF_U32) {
        g->alignment = (uint32_t)g->meta[al->second].second.raw;
        if (g->alignment == 0) return gfail("gguf: general.alignment is 0");
    }
    for (uint64_t i = 0; i < n_tensors; i++) {
        Tensor t;
        uint32_t rank, type;
        uint64_t off;
        if (!r.str(t.name) || !r.get(rank)) return gfail("gguf: truncated in tensor info %llu", (unsigned long long)i);
        if (rank > 4) return gfail("gguf: tensor %s has rank %u (at most 4)", t.name.c_str(), rank);
        t.rank = rank;
        for (uint32_t d = 0; d < rank; d++)
            if (!r.get(t.dims[rank - 1 - d])) return gfail("gguf: truncated in tensor info %llu", (unsigned long long)i);
        if (!r.get(type) || !r.get(off)) return gfail("gguf: truncated in tensor info %llu", (unsigned long long)i);
        uint32_t be, bb;
        bool known;
        if (!tensor_block((int32_t)type, be, bb, known))
            return gfail("gguf: tensor %s of type %u is not part of the supported gguf version", t.name.c_str(), type);
        t.dtype = (int32_t)type;
        t.offset = off;
        // element count, multiplied step by step with an overflow check
        uint64_t elems = 1;
        for (int d = 0; d < 4; d++)
            if (__builtin_mul_overflow(elems, t.dims[d], &elems) || (elems >> 62))
                return gfail("gguf: tensor %s is too large", t.name.c_str());
        if (known && elems % be)
            return gfail("gguf: tensor %s has %llu elements, not a multiple of its block of %u", t.name.c_str(),
                         (unsigned long long)elems, be);
        uint64_t bytes = 0;
        if (known && __builtin_mul_overflow(elems / be, (uint64_t)bb, &bytes))
            return gfail("gguf: tensor %s is too large", t.name.c_str());
        t.bytes = bytes;
        t.has_data = known;
        g->tensor_ix[t.name] = g->tensors.size(); // a repeated name keeps the last info, as a map insert does
        g->tensors.push_back(std::move(t));
    }
    const uint64_t start = ((uint64_t)r.off + g->alignment - 1) / g->alignment * g->alignment;
    for (Tensor &t : g->tensors) {
        if (t.offset > g->len || start > g->len - t.offset) return gfail("gguf: tensor %s starts past the end", t.name.c_str());
        t.offset += start;
        if (t.has_data && t.bytes > g->len - t.offset)
            return gfail("gguf: tensor %s (%llu bytes at %llu) runs past the end of the file (%zu bytes)",
                         t.name.c_str(), (unsigned long long)t.bytes, (unsigned long long)t.offset, g->len);
    }
    return IFR_OK;
}

const Value *find(const ifr_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    auto it = g->meta_ix.find(key);
    return it == g->meta_ix.end() ? nullptr : &g->meta[it->second].second;
}

} // namespace

// ------------------------------------------------------------------ writer

struct ifr_gguf_writer {
    struct Kv {
        std::string key;
        int32_t type;
        std::vector<uint8_t> enc; // encoded value (after the type field)
    };
    std::vector<Kv> kv;
    struct T {
        std::string name;
        int32_t dtype;
        uint32_t rank;
        uint64_t dims[4];
        std::vector<uint8_t> data;
    };
    std::vector<T> tensors;
};

namespace {

void put(std::vector<uint8_t> &b, const void *p, size_t n) {
    const uint8_t *q = (const uint8_t *)p;
    b.insert(b.end(), q, q + n);
}
template <class V>
void put(std::vector<uint8_t> &b, V v) { put(b, &v, sizeof v); }
void put_str(std::vector<uint8_t> &b, const char *s, size_t n) {
    put(b, (uint64_t)n);
    put(b, s, n);
}

ifr_status writer_kv(ifr_gguf_writer *w, const char *key, int32_t type, std::vector<uint8_t> enc) {
    for (auto &e : w->kv)
        if (e.key == key) {
            e.type = type;
            e.enc = std::move(enc);
            return IFR_OK;
        }
    w->kv.push_back({key, type, std::move(enc)});
    return IFR_OK;
}

} // namespace

extern "C" {

IFR_API ifr_status ifr_gguf_open(const char *path, ifr_gguf **out) {
    if (!path || !out) return gfail("gguf: null argument");
    *out = nullptr;
    int fd = open(path, O_RDONLY);
    if (fd < 0) return gfail("gguf: cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return gfail("gguf: cannot stat %s", path);
    }
    ifr_gguf *g = new ifr_gguf();
    g->len = (size_t)st.st_size;
    if (g->len) {
        g->map = mmap(nullptr, g->len, PROT_READ, MAP_PRIVATE, fd, 0);
        if (g->map == MAP_FAILED) {
            g->map = nullptr;
            close(fd);
            delete g;
            return gfail("gguf: cannot map %s", path);
        }
        g->map_len = g->len;
    }
    close(fd);
    g->base = (const uint8_t *)g->map;
    ifr_status s = parse(g);
    if (s) {
        delete g;
        return s;
    }
    *out = g;
    return IFR_OK;
}

IFR_API ifr_status ifr_gguf_from_bytes(const void *bytes, size_t len, ifr_gguf **out) {
    if ((!bytes && len) || !out) return gfail("gguf: null argument");
    *out = nullptr;
    ifr_gguf *g = new ifr_gguf();
    g->own.assign((const uint8_t *)bytes, (const uint8_t *)bytes + len);
    g->base = g->own.data();
    g->len = len;
    ifr_status s = parse(g);
    if (s) {
        delete g;
        return s;
    }
    *out = g;
    return IFR_OK;
}

IFR_API void ifr_gguf_close(ifr_gguf *g) { delete g; }

IFR_API uint32_t ifr_gguf_version(const ifr_gguf *g) { return g ? g->version : 0; }
IFR_API uint32_t ifr_gguf_alignment(const ifr_gguf *g) { return g ? g->alignment : 0; }
IFR_API uint64_t ifr_gguf_metadata_count(const ifr_gguf *g) { return g ? g->meta.size() : 0; }
IFR_API const char *ifr_gguf_metadata_key(const ifr_gguf *g, uint64_t i) {
    return g && i < g->meta.size() ? g->meta[(size_t)i].first.c_str() : nullptr;
}

IFR_API int32_t ifr_gguf_metadata_type(const ifr_gguf *g, const char *key, int32_t *elem_type, uint64_t *len) {
    const Value *v = find(g, key);
    if (!v) return -1;
    if (elem_type) *elem_type = v->type == IFR_GGUF_ARRAY ? v->elem_type : -1;
    if (len) *len = v->type == IFR_GGUF_ARRAY ? v->len : v->type == IFR_GGUF_STRING ? v->str.size() : 1;
    return v->type;
}

IFR_API ifr_status ifr_gguf_get_scalar(const ifr_gguf *g, const char *key, int32_t type, void *out) {
    const Value *v = find(g, key);
    if (!v || !out) return gfail("gguf: no metadata key %s", key ? key : "(null)");
    if (v->type != type || !scalar_size(type))
        return gfail("gguf: metadata %s has type %d, not %d", key, v->type, type);
    memcpy(out, &v->raw, scalar_size(type));
    return IFR_OK;
}

IFR_API ifr_status ifr_gguf_get_string(const ifr_gguf *g, const char *key, const char **s, uint64_t *len) {
    const Value *v = find(g, key);
    if (!v || !s) return gfail("gguf: no metadata key %s", key ? key : "(null)");
    if (v->type != IFR_GGUF_STRING) return gfail("gguf: metadata %s has type %d, not a string", key, v->type);
    *s = v->str.c_str();
    if (len) *len = v->str.size();
    return IFR_OK;
}

IFR_API ifr_status ifr_gguf_get_array(const ifr_gguf *g, const char *key, int32_t *elem_type, uint64_t *len,
                                      const void **data) {
    const Value *v = find(g, key);
    if (!v) return gfail("gguf: no metadata key %s", key ? key : "(null)");
    if (v->type != IFR_GGUF_ARRAY) return gfail("gguf: metadata %s has type %d, not an array", key, v->type);
    if (elem_type) *elem_type = v->elem_type;
    if (len) *len = v->len;
    if (data) *data = v->data;
    return IFR_OK;
}

IFR_API ifr_status ifr_gguf_get_array_string(const ifr_gguf *g, const char *key, uint64_t i, const char **s,
                                             uint64_t *len) {
    const Value *v = find(g, key);
    if (!v || !s) return gfail("gguf: no metadata key %s", key ? key : "(null)");
    if (v->type != IFR_GGUF_ARRAY || v->elem_type != IFR_GGUF_STRING)
        return gfail("gguf: metadata %s is not an array of strings", key);
    if (i >= v->strs.size()) return gfail("gguf: index %llu past the %zu strings of %s", (unsigned long long)i, v->strs.size(), key);
    *s = v->strs[(size_t)i].c_str();
    if (len) *len = v->strs[(size_t)i].size();
    return IFR_OK;
}

IFR_API uint64_t ifr_gguf_tensor_count(const ifr_gguf *g) { return g ? g->tensors.size() : 0; }
IFR_API const char *ifr_gguf_tensor_name(const ifr_gguf *g, uint64_t i) {
    return g && i < g->tensors.size() ? g->tensors[(size_t)i].name.c_str() : nullptr;
}

IFR_API ifr_status ifr_gguf_tensor_info(const ifr_gguf *g, const char *name, int32_t *dtype, uint64_t dims[4],
                                        uint32_t *rank, const void **data, uint64_t *bytes) {
    if (!g || !name) return gfail("gguf: null argument");
    auto it = g->tensor_ix.find(name);
    if (it == g->tensor_ix.end()) return gfail("gguf: no tensor %s", name);
    const Tensor &t = g->tensors[it->second];
    if (dtype) *dtype = t.dtype;
    if (dims)
        for (int d = 0; d < 4; d++) dims[d] = t.dims[d];
    if (rank) *rank = t.rank;
    if (data) *data = t.has_data ? g->base + t.offset : nullptr;
    if (bytes) *bytes = t.bytes;
    return IFR_OK;
}

IFR_API ifr_status ifr_gguf_writer_create(ifr_gguf_writer **out) {
    if (!out) return gfail("gguf: null argument");
    *out = new ifr_gguf_writer();
    return IFR_OK;
}

IFR_API void ifr_gguf_writer_destroy(ifr_gguf_writer *w) { delete w; }

IFR_API ifr_status ifr_gguf_writer_set(ifr_gguf_writer *w, const char *key, int32_t type, const void *value) {
    if (!w || !key || !value) return gfail("gguf: null argument");
    std::vector<uint8_t> enc;
    if (uint32_t sz = scalar_size(type)) {
        put(enc, value, sz);
    } else if (type == IFR_GGUF_STRING) {
        const char *s = (const char *)value;
        put_str(enc, s, strlen(s));
    } else {
        return gfail("gguf: ifr_gguf_writer_set takes a scalar or string type, not %d", type);
    }
    return writer_kv(w, key, type, std::move(enc));
}

IFR_API ifr_status ifr_gguf_writer_set_array(ifr_gguf_writer *w, const char *key, int32_t elem_type, const void *data,
                                             uint64_t len) {
    if (!w || !key || (!data && len)) return gfail("gguf: null argument");
    std::vector<uint8_t> enc;
    put(enc, (uint32_t)elem_type);
    put(enc, len);
    if (uint32_t sz = scalar_size(elem_type)) {
        put(enc, data, (size_t)(sz * len));
    } else if (elem_type == IFR_GGUF_STRING) {
        const char *const *s = (const char *const *)data;
        for (uint64_t i = 0; i < len; i++) {
            if (!s[i]) return gfail("gguf: null string %llu in array %s", (unsigned long long)i, key);
            put_str(enc, s[i], strlen(s[i]));
        }
    } else {
        return gfail("gguf: arrays of type %d cannot be written", elem_type);
    }
    return writer_kv(w, key, IFR_GGUF_ARRAY, std::move(enc));
}

IFR_API ifr_status ifr_gguf_writer_add_tensor(ifr_gguf_writer *w, const char *name, int32_t dtype, uint32_t rank,
                                              const uint64_t *dims, const void *data, uint64_t bytes) {
    if (!w || !name || !dims || (!data && bytes)) return gfail("gguf: null argument");
    if (rank < 1 || rank > 4) return gfail("gguf: tensor %s has rank %u (1 to 4)", name, rank);
    uint32_t be, bb;
    bool known;
    if (!tensor_block(dtype, be, bb, known) || !known) return gfail("gguf: tensor type %d cannot be written", dtype);
    uint64_t elems = 1;
    for (uint32_t d = 0; d < rank; d++) elems *= dims[d];
    if (elems % be || elems / be * bb != bytes)
        return gfail("gguf: tensor %s: %llu elements of type %d take %llu bytes, not %llu", name,
                     (unsigned long long)elems, dtype, (unsigned long long)(elems / be * bb), (unsigned long long)bytes);
    for (auto &t : w->tensors)
        if (t.name == name) return gfail("gguf: tensor %s added twice", name);
    ifr_gguf_writer::T t;
    t.name = name;
    t.dtype = dtype;
    t.rank = rank;
    for (int d = 0; d < 4; d++) t.dims[d] = d < (int)rank ? dims[d] : 1;
    t.data.assign((const uint8_t *)data, (const uint8_t *)data + bytes);
    w->tensors.push_back(std::move(t));
    return IFR_OK;
}

IFR_API ifr_status ifr_gguf_writer_save(ifr_gguf_writer *w, const char *path) {
    if (!w || !path) return gfail("gguf: null argument");
    uint32_t alignment = 32;
    for (auto &e : w->kv)
        if (e.key == "general.alignment" && e.type == IFR_GGUF_U32) memcpy(&alignment, e.enc.data(), 4);
    if (!alignment) return gfail("gguf: general.alignment is 0");
    std::vector<uint8_t> b;
    put(b, MAGIC_LE);
    put(b, (uint32_t)3);
    put(b, (uint64_t)w->tensors.size());
    put(b, (uint64_t)w->kv.size());
    for (auto &e : w->kv) {
        put_str(b, e.key.data(), e.key.size());
        put(b, (uint32_t)e.type);
        put(b, e.enc.data(), e.enc.size());
    }
    uint64_t off = 0;
    std::vector<uint64_t> offs;
    for (auto &t : w->tensors) {
        put_str(b, t.name.data(), t.name.size());
        put(b, t.rank);
        for (uint32_t d = 0; d < t.rank; d++) put(b, t.dims[t.rank - 1 - d]); // GGUF order: reversed
        put(b, (uint32_t)t.dtype);
        put(b, off);
        offs.push_back(off);
        off = (off + t.data.size() + alignment - 1) / alignment * alignment;
    }
    b.resize((b.size() + alignment - 1) / alignment * alignment, 0);
    const size_t start = b.size();
    for (size_t i = 0; i < w->tensors.size(); i++) {
        b.resize(start + offs[i], 0);
        put(b, w->tensors[i].data.data(), w->tensors[i].data.size());
    }
    if (!w->tensors.empty()) b.resize(start + off, 0);
    FILE *f = fopen(path, "wb");
    if (!f) return gfail("gguf: cannot create %s", path);
    const size_t n = fwrite(b.data(), 1, b.size(), f);
    const int c = fclose(f);
    if (n != b.size() || c != 0) return gfail("gguf: short write to %s", path);
    return IFR_OK;
}

} // extern "C"
