// GGUF reader and device residency: the checkpoint seam that feeds real
// tensors to the matrix path.  Follows src/gguf.rs of the reference:
//  * open (gguf.rs:108-150): memory-map the file, check the v3 header, scan
//    every metadata value structurally (bounded: 100,000 entries, 10,000,000
//    values in all, nesting below depth 4) and index only the requested keys;
//  * directory (gguf.rs:156-237): tensor entries, the data section start at
//    general.alignment (default 32, a power of two <= 4096), offsets aligned,
//    strictly increasing when sorted, inside the file; each entry's extent
//    runs to the next tensor (or the end of the file);
//  * select (gguf.rs:40-87): the format's own alignment (F32 4, MXFP4 1,
//    others 2), a whole number of blocks in the first dimension, at most
//    2^32 - 1 elements, and bytes within the extent;
//  * typed metadata reads (gguf.rs:239-348).
// Residency: the reference registers the mapped pages with Metal (zero copy,
// buffer.rs:145-297); here a selected tensor is copied once into device
// memory (oco_gguf_upload) and read from HBM by every kernel after that.
#include <fcntl.h>
#include <hip/hip_runtime_api.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/oco_hip.h"

namespace oco {
int fail(int code, const char *fmt, ...);
int hip_check(hipError_t e, const char *what);
}  // namespace oco
using oco::fail;

#define OCO_TRY_C(expr)                   \
    do {                                  \
        int _rc = (expr);                 \
        if (_rc != OCO_OK) return _rc;    \
    } while (0)

namespace {

constexpr uint64_t MAX_ENTRIES = 100000;
constexpr uint64_t MAX_VALUES = 10000000;

struct Field {
    uint32_t kind;
    size_t begin, end;  // the value's bytes in the map
};

// Bounded little-endian reads over [pos, end); every failure is a
// checkpoint error with a message.
struct Reader {
    const uint8_t *base;
    size_t pos, end;
    uint64_t budget = MAX_VALUES;
    const char *err = nullptr;

    bool take(size_t n, const uint8_t **out) {
        if (n > end - pos) return bad("truncated GGUF value");
        if (out) *out = base + pos;
        pos += n;
        return true;
    }
    bool bad(const char *m) {
        if (!err) err = m;
        return false;
    }
    bool u32(uint32_t *v) {
        const uint8_t *p;
        if (!take(4, &p)) return false;
        memcpy(v, p, 4);
        return true;
    }
    bool u64(uint64_t *v) {
        const uint8_t *p;
        if (!take(8, &p)) return false;
        memcpy(v, p, 8);
        return true;
    }
    bool string(const char **s, size_t *n) {
        uint64_t len;
        if (!u64(&len)) return false;
        if (len > end - pos) return bad("truncated GGUF value");
        const uint8_t *p;
        take((size_t)len, &p);
        if (s) *s = (const char *)p;
        if (n) *n = (size_t)len;
        return true;
    }
    static int scalar_bytes(uint32_t kind) {
        switch (kind) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        }
        return 0;
    }
    bool array_header(uint32_t *kind, uint64_t *n) {
        if (!u32(kind) || !u64(n)) return false;
        const int minimum = *kind == 8 ? 8 : *kind == 9 ? 12 : scalar_bytes(*kind);
        if (!minimum) return bad("unknown metadata type");
        if (*n > MAX_VALUES || *n > (end - pos) / (uint64_t)minimum) return bad("excessive or truncated metadata array");
        return true;
    }
    bool skip_value(uint32_t kind, int depth) {
        if (depth >= 4) return bad("nested metadata is too deep");
        if (budget == 0) return bad("metadata exceeds aggregate value budget");
        budget--;
        if (kind == 8) return string(nullptr, nullptr);
        if (kind == 9) {
            uint32_t k;
            uint64_t n;
            if (!array_header(&k, &n)) return false;
            return skip_array(k, n, depth);
        }
        const int b = scalar_bytes(kind);
        if (!b) return bad("unknown metadata type");
        return take((size_t)b, nullptr);
    }
    bool skip_array(uint32_t kind, uint64_t n, int depth) {
        if (n > budget) return bad("metadata exceeds aggregate value budget");
        if (kind != 8 && kind != 9) {
            if (depth + 1 >= 4) return bad("nested metadata is too deep");
            budget -= n;
            const uint64_t bytes = (uint64_t)scalar_bytes(kind) * n;
            if (bytes > end - pos) return bad("truncated GGUF value");
            return take((size_t)bytes, nullptr);
        }
        for (uint64_t i = 0; i < n; i++)
            if (!skip_value(kind, depth + 1)) return false;
        return true;
    }
};

}  // namespace

struct oco_gguf {
    const uint8_t *map = nullptr;
    size_t size = 0;
    std::unordered_map<std::string, Field> meta;
    uint64_t tensor_count = 0;
    size_t tensor_offset = 0;
    bool have_directory = false;
    std::vector<std::string> names;
    std::vector<oco_gguf_entry> entries;
    std::unordered_map<std::string, size_t> index;
};

static int checkpoint(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return fail(OCO_ERR_CHECKPOINT, "%s", buf);
}

static void unmap(oco_gguf *g) {
    if (g->map && g->size) munmap((void *)g->map, g->size);
    g->map = nullptr;
}

extern "C" int oco_gguf_open(const char *path, const char *const *keep, uint32_t nkeep, oco_gguf **out) {
    if (!path || !out) return fail(OCO_ERR_INVALID, "oco_gguf_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(OCO_ERR_INVALID, "oco_gguf_open: cannot open %s", path);
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return fail(OCO_ERR_INVALID, "oco_gguf_open: cannot stat %s", path);
    }
    oco_gguf *g = new oco_gguf();
    g->size = (size_t)st.st_size;
    if (g->size) {
        void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            close(fd);
            delete g;
            return fail(OCO_ERR_INVALID, "oco_gguf_open: cannot map %s", path);
        }
        g->map = (const uint8_t *)m;
    }
    close(fd);
    std::unordered_set<std::string> wanted;
    for (uint32_t i = 0; i < nkeep; i++)
        if (keep && keep[i]) wanted.insert(keep[i]);

    Reader r{g->map, 0, g->size};
    uint32_t magic = 0, version = 0;
    uint64_t nt = 0, nm = 0;
    int rc = OCO_OK;
    auto finish = [&](int code) {
        if (code != OCO_OK) {
            unmap(g);
            delete g;
        } else {
            *out = g;
        }
        return code;
    };
    if (!r.u32(&magic)) return finish(checkpoint("%s", r.err));
    if (magic != 0x46554747u) return finish(checkpoint("not a GGUF file"));
    if (!r.u32(&version)) return finish(checkpoint("%s", r.err));
    if (version != 3) return finish(checkpoint("only GGUF version 3 is supported"));
    if (!r.u64(&nt) || !r.u64(&nm)) return finish(checkpoint("%s", r.err));
    if (nm > MAX_ENTRIES) return finish(checkpoint("excessive GGUF metadata count"));
    if (nm > (r.end - r.pos) / 12) return finish(checkpoint("truncated GGUF metadata directory"));
    std::unordered_set<std::string> keys;
    for (uint64_t i = 0; i < nm; i++) {
        const char *k;
        size_t kn;
        uint32_t kind;
        if (!r.string(&k, &kn) || !r.u32(&kind)) return finish(checkpoint("%s", r.err));
        std::string key(k, kn);
        if (!keys.insert(key).second) return finish(checkpoint("duplicate GGUF metadata key"));
        const size_t start = r.pos;
        if (!r.skip_value(kind, 0)) return finish(checkpoint("%s", r.err));
        if (wanted.count(key)) g->meta[key] = Field{kind, start, r.pos};
    }
    g->tensor_count = nt;
    g->tensor_offset = r.pos;
    return finish(rc);
}

extern "C" int oco_gguf_close(oco_gguf *g) {
    if (!g) return OCO_OK;
    unmap(g);
    delete g;
    return OCO_OK;
}

// ---- metadata --------------------------------------------------------------------

namespace {
struct Value {
    enum { U, S, F, B, STR } tag;
    uint64_t u;
    int64_t s;
    double f;
    const char *str;
    size_t len;
};

bool read_value(Reader &r, uint32_t kind, Value &v) {
    const uint8_t *p;
    switch (kind) {
    case 0: if (!r.take(1, &p)) return false; v.tag = Value::U; v.u = p[0]; return true;
    case 1: if (!r.take(1, &p)) return false; v.tag = Value::S; v.s = (int8_t)p[0]; return true;
    case 2: { if (!r.take(2, &p)) return false; uint16_t x; memcpy(&x, p, 2); v.tag = Value::U; v.u = x; return true; }
    case 3: { if (!r.take(2, &p)) return false; int16_t x; memcpy(&x, p, 2); v.tag = Value::S; v.s = x; return true; }
    case 4: { if (!r.take(4, &p)) return false; uint32_t x; memcpy(&x, p, 4); v.tag = Value::U; v.u = x; return true; }
    case 5: { if (!r.take(4, &p)) return false; int32_t x; memcpy(&x, p, 4); v.tag = Value::S; v.s = x; return true; }
    case 6: { if (!r.take(4, &p)) return false; float x; memcpy(&x, p, 4); v.tag = Value::F; v.f = x; return true; }
    case 7:
        if (!r.take(1, &p)) return false;
        if (p[0] > 1) return r.bad("invalid GGUF boolean");
        v.tag = Value::B;
        v.u = p[0];
        return true;
    case 8: v.tag = Value::STR; return r.string(&v.str, &v.len);
    case 10: { if (!r.take(8, &p)) return false; uint64_t x; memcpy(&x, p, 8); v.tag = Value::U; v.u = x; return true; }
    case 11: { if (!r.take(8, &p)) return false; int64_t x; memcpy(&x, p, 8); v.tag = Value::S; v.s = x; return true; }
    case 12: { if (!r.take(8, &p)) return false; double x; memcpy(&x, p, 8); v.tag = Value::F; v.f = x; return true; }
    }
    return r.bad("unknown metadata type");
}
}  // namespace

static int scalar(const oco_gguf *g, const char *key, Value &v) {
    if (!g || !key) return fail(OCO_ERR_INVALID, "oco_gguf: null argument");
    auto it = g->meta.find(key);
    if (it == g->meta.end()) return checkpoint("missing metadata %s", key);
    if (it->second.kind == 9) return checkpoint("expected scalar metadata %s", key);
    Reader r{g->map, it->second.begin, it->second.end};
    if (!read_value(r, it->second.kind, v)) return checkpoint("%s", r.err);
    return OCO_OK;
}

extern "C" int oco_gguf_has(const oco_gguf *g, const char *key) { return g && key && g->meta.count(key) ? 1 : 0; }

extern "C" int oco_gguf_text(const oco_gguf *g, const char *key, const char **text, size_t *len) {
    Value v;
    OCO_TRY_C(scalar(g, key, v));
    if (v.tag != Value::STR) return checkpoint("expected string %s", key);
    if (text) *text = v.str;
    if (len) *len = v.len;
    return OCO_OK;
}

extern "C" int oco_gguf_number(const oco_gguf *g, const char *key, double *out) {
    Value v;
    OCO_TRY_C(scalar(g, key, v));
    double d;
    if (v.tag == Value::U) d = (double)v.u;
    else if (v.tag == Value::S) d = (double)v.s;
    else if (v.tag == Value::F) d = v.f;
    else return checkpoint("expected number %s", key);
    if (!(d - d == 0)) return checkpoint("non-finite number %s", key);
    if (out) *out = d;
    return OCO_OK;
}

extern "C" int oco_gguf_boolean(const oco_gguf *g, const char *key, int *out) {
    Value v;
    OCO_TRY_C(scalar(g, key, v));
    if (v.tag == Value::B || (v.tag == Value::U && v.u <= 1)) {
        if (out) *out = (int)v.u;
        return OCO_OK;
    }
    return checkpoint("expected boolean %s", key);
}

extern "C" int oco_gguf_unsigned(const oco_gguf *g, const char *key, uint64_t *out) {
    Value v;
    OCO_TRY_C(scalar(g, key, v));
    if (v.tag == Value::U) {
        if (out) *out = v.u;
        return OCO_OK;
    }
    if (v.tag == Value::S && v.s >= 0) {
        if (out) *out = (uint64_t)v.s;
        return OCO_OK;
    }
    return checkpoint("expected unsigned integer %s", key);
}

// Arrays: element kind, count, and element i read as a string or an integer.
static int array_at(const oco_gguf *g, const char *key, uint32_t *kind, uint64_t *count, Reader &r) {
    if (!g || !key) return fail(OCO_ERR_INVALID, "oco_gguf: null argument");
    auto it = g->meta.find(key);
    if (it == g->meta.end()) return checkpoint("missing metadata %s", key);
    if (it->second.kind != 9) return checkpoint("expected array metadata %s", key);
    r = Reader{g->map, it->second.begin, it->second.end};
    if (!r.array_header(kind, count)) return checkpoint("%s", r.err);
    return OCO_OK;
}

extern "C" int oco_gguf_array(const oco_gguf *g, const char *key, uint32_t *kind, uint64_t *count) {
    Reader r{nullptr, 0, 0};
    return array_at(g, key, kind, count, r);
}

extern "C" int oco_gguf_array_string(const oco_gguf *g, const char *key, uint64_t i, const char **text, size_t *len) {
    uint32_t kind;
    uint64_t count;
    Reader r{nullptr, 0, 0};
    OCO_TRY_C(array_at(g, key, &kind, &count, r));
    if (kind != 8) return checkpoint("unexpected array element type for %s", key);
    if (i >= count) return fail(OCO_ERR_INVALID, "oco_gguf_array_string: index %llu of %llu", (unsigned long long)i,
                                (unsigned long long)count);
    for (uint64_t j = 0; j <= i; j++)
        if (!r.string(j == i ? text : nullptr, j == i ? len : nullptr)) return checkpoint("%s", r.err);
    return OCO_OK;
}

// Every element of an integer array as a non-negative integer
// (unsigned_integers, gguf.rs:313-333); `out` holds `capacity` values.
extern "C" int oco_gguf_array_unsigned(const oco_gguf *g, const char *key, uint64_t *out, uint64_t capacity) {
    uint32_t kind;
    uint64_t count;
    Reader r{nullptr, 0, 0};
    OCO_TRY_C(array_at(g, key, &kind, &count, r));
    if (count > capacity) return fail(OCO_ERR_INVALID, "oco_gguf_array_unsigned: %llu values, room for %llu",
                                      (unsigned long long)count, (unsigned long long)capacity);
    for (uint64_t j = 0; j < count; j++) {
        Value v;
        if (!read_value(r, kind, v)) return checkpoint("%s", r.err);
        if (v.tag == Value::U) out[j] = v.u;
        else if (v.tag == Value::S && v.s >= 0) out[j] = (uint64_t)v.s;
        else return checkpoint("expected unsigned integer array %s", key);
    }
    return OCO_OK;
}

// ---- tensor directory ------------------------------------------------------------

extern "C" int oco_gguf_directory(oco_gguf *g, uint64_t *count) {
    if (!g) return fail(OCO_ERR_INVALID, "oco_gguf_directory: null handle");
    if (g->have_directory) {
        if (count) *count = g->entries.size();
        return OCO_OK;
    }
    if (g->tensor_count > MAX_ENTRIES) return checkpoint("excessive GGUF tensor count");
    Reader r{g->map, g->tensor_offset, g->size};
    if (g->tensor_count > (r.end - r.pos) / 32) return checkpoint("truncated GGUF tensor directory");
    std::vector<std::string> names;
    std::vector<oco_gguf_entry> entries;
    std::unordered_map<std::string, size_t> index;
    for (uint64_t t = 0; t < g->tensor_count; t++) {
        const char *s;
        size_t sn;
        uint32_t dims;
        if (!r.string(&s, &sn) || !r.u32(&dims)) return checkpoint("%s", r.err);
        std::string name(s, sn);
        if (dims < 1 || dims > 4) return checkpoint("invalid dimensions for %s", name.c_str());
        oco_gguf_entry e;
        memset(&e, 0, sizeof e);
        e.rank = dims;
        for (uint32_t d = 0; d < dims; d++) {
            if (!r.u64(&e.shape[d])) return checkpoint("%s", r.err);
            if (e.shape[d] == 0) return checkpoint("zero tensor dimension");
        }
        if (!r.u32(&e.code) || !r.u64(&e.offset)) return checkpoint("%s", r.err);
        if (!index.emplace(name, entries.size()).second) return checkpoint("duplicate tensor name");
        names.push_back(std::move(name));
        entries.push_back(e);
    }
    uint64_t alignment = 32;
    if (g->meta.count("general.alignment")) OCO_TRY_C(oco_gguf_unsigned(g, "general.alignment", &alignment));
    if (alignment == 0 || (alignment & (alignment - 1)) || alignment > 4096) return checkpoint("invalid GGUF alignment");
    const uint64_t start = (r.pos + alignment - 1) / alignment * alignment;
    std::vector<size_t> order(entries.size());
    for (size_t i = 0; i < order.size(); i++) order[i] = i;
    std::sort(order.begin(), order.end(), [&](size_t a, size_t b) { return entries[a].offset < entries[b].offset; });
    for (size_t i = 0; i < order.size(); i++) {
        oco_gguf_entry &e = entries[order[i]];
        if (e.offset % alignment) return checkpoint("unaligned tensor");
        if (e.offset > UINT64_MAX - start) return checkpoint("tensor offset overflow");
        const uint64_t absolute = start + e.offset;
        if (absolute >= g->size) return checkpoint("tensor offset outside file");
        uint64_t end = g->size;
        if (i + 1 < order.size()) {
            const uint64_t next = entries[order[i + 1]].offset;
            if (e.offset >= next) return checkpoint("overlapping tensor offsets");
            if (next > UINT64_MAX - start) return checkpoint("tensor offset overflow");
            end = start + next;
        }
        if (end > g->size) return checkpoint("tensor offset outside file");
        e.offset = absolute;
        e.extent = end - absolute;
    }
    g->names = std::move(names);
    g->entries = std::move(entries);
    g->index = std::move(index);
    g->have_directory = true;
    if (count) *count = g->entries.size();
    return OCO_OK;
}

extern "C" int oco_gguf_entry_at(const oco_gguf *g, uint64_t i, const char **name, oco_gguf_entry *out) {
    if (!g || !g->have_directory) return fail(OCO_ERR_INVALID, "oco_gguf_entry_at: no directory (oco_gguf_directory)");
    if (i >= g->entries.size()) return fail(OCO_ERR_INVALID, "oco_gguf_entry_at: index %llu", (unsigned long long)i);
    if (name) *name = g->names[i].c_str();
    if (out) *out = g->entries[i];
    return OCO_OK;
}

extern "C" int oco_gguf_find(const oco_gguf *g, const char *name, oco_gguf_entry *out) {
    if (!g || !name) return fail(OCO_ERR_INVALID, "oco_gguf_find: null argument");
    if (!g->have_directory) return fail(OCO_ERR_INVALID, "oco_gguf_find: no directory (oco_gguf_directory)");
    auto it = g->index.find(name);
    if (it == g->index.end()) return checkpoint("missing tensor %s", name);
    if (out) *out = g->entries[it->second];
    return OCO_OK;
}

extern "C" int oco_gguf_select(const oco_gguf_entry *e, oco_gguf_tensor *out) {
    if (!e || !out) return fail(OCO_ERR_INVALID, "oco_gguf_select: null argument");
    uint32_t block, size;
    if (oco_block_layout(e->code, &block, &size) != OCO_OK) return checkpoint("unsupported GGUF tensor type %u", e->code);
    const uint64_t alignment = e->code == OCO_F32 ? 4 : e->code == OCO_MXFP4 ? 1 : 2;
    if (e->offset % alignment) return checkpoint("unaligned tensor data");
    if (e->shape[0] % block) return checkpoint("invalid tensor block alignment");
    uint64_t elements = 1;
    for (uint32_t d = 0; d < e->rank; d++) {
        if (e->shape[d] && elements > UINT64_MAX / e->shape[d]) return checkpoint("tensor size overflow");
        elements *= e->shape[d];
    }
    if (elements > 0xffffffffull) return checkpoint("tensor exceeds the supported index range");
    const uint64_t bytes = elements / block * size;
    if (bytes > e->extent) return checkpoint("truncated or overlapping selected tensor");
    memset(out, 0, sizeof *out);
    out->format = e->code;
    out->rank = e->rank;
    for (uint32_t d = 0; d < 4; d++) out->shape[d] = e->shape[d];
    out->offset = e->offset;
    out->bytes = bytes;
    return OCO_OK;
}

extern "C" const void *oco_gguf_data(const oco_gguf *g, const oco_gguf_tensor *t) {
    if (!g || !t || t->offset + t->bytes > g->size) return nullptr;
    return g->map + t->offset;
}

// Copy a selected tensor into device memory `dst` (at least t->bytes),
// ordered on `stream` and complete on return (the file pages are read once).
extern "C" int oco_gguf_upload(const oco_gguf *g, const oco_gguf_tensor *t, void *dst, oco_stream stream) {
    if (!g || !t || !dst) return fail(OCO_ERR_INVALID, "oco_gguf_upload: null argument");
    if (t->offset > g->size || t->bytes > g->size - t->offset)
        return checkpoint("tensor outside the mapped file");
    if (!t->bytes) return OCO_OK;
    OCO_TRY_C(oco::hip_check(hipMemcpyAsync(dst, g->map + t->offset, t->bytes, hipMemcpyHostToDevice,
                                            (hipStream_t)stream),
                             "oco_gguf_upload: hipMemcpyAsync"));
    return oco::hip_check(hipStreamSynchronize((hipStream_t)stream), "oco_gguf_upload: hipStreamSynchronize");
}
