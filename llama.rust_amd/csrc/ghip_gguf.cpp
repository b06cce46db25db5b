// ghip_gguf.cpp -- GGUF container reader and device upload (the C ABI's
// ghip_gguf_* entry points).
//
// Follows the reference's reader (crates/ggml/src/gguf.rs, a port of
// ggml/src/gguf.cpp gguf_init_from_file): magic "GGUF", u32 version (<= 3),
// u64 tensor count, u64 kv count, the kv pairs, the tensor infos, then the
// data section at the next multiple of general.alignment (default 32; only
// when tensors exist).  Little-endian throughout.  The same checks and the
// same error texts (gguf.rs:278-300).  Gguf::open's split pass
// (gguf.rs:388-480: split.count / split.no / split.tensors.count, part files
// named {prefix}-{no+1:05}-of-{count:05}.gguf) is followed when asked.
//
// The file is memory-mapped; ghip_gguf_upload copies one tensor's bytes to
// device memory through pinned staging buffers (double-buffered against the
// copy engine) and can register the uploaded weight (ghip_weight_register),
// which builds its device-side repacked copy: the load-time repack of the
// reference's CPU_REPACK buffer, done on the device.
#include "../../include/ghip.h"
#include "ghip_internal.h"

#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

namespace {

constexpr uint32_t kGgufVersion = 3;
constexpr uint64_t kDefaultAlignment = 32;
constexpr size_t kMaxName = 64;  // GGML_MAX_NAME (types.rs:7)

// block size and bytes per block of every ggml type id (types.rs:72-112)
bool ggml_type_size(uint32_t t, int64_t &blck, int64_t &bytes) {
    struct Row { uint32_t id; int64_t blck, bytes; };
    static const Row rows[] = {
        {0, 1, 4},     {1, 1, 2},      {2, 32, 18},    {3, 32, 20},    {6, 32, 22},    {7, 32, 24},
        {8, 32, 34},   {9, 32, 36},    {10, 256, 84},  {11, 256, 110}, {12, 256, 144}, {13, 256, 176},
        {14, 256, 210}, {15, 256, 292}, {16, 256, 66}, {17, 256, 74},  {18, 256, 98},  {19, 256, 50},
        {20, 32, 18},  {21, 256, 110}, {22, 256, 82},  {23, 256, 136}, {24, 1, 1},     {25, 1, 2},
        {26, 1, 4},    {27, 1, 8},     {28, 1, 8},     {29, 256, 56},  {30, 1, 2},     {34, 256, 54},
        {35, 256, 66}, {39, 32, 17},   {40, 64, 36},   {41, 128, 18},  {42, 64, 18},
    };
    for (const Row &r : rows)
        if (r.id == t) {
            blck = r.blck;
            bytes = r.bytes;
            return true;
        }
    return false;
}

enum : uint32_t {
    T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
    T_STR = 8, T_ARR = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12,
};
const char *type_name(uint32_t t) {
    static const char *n[] = {"uint8", "int8",  "uint16", "int16",  "uint32", "int32", "float32",
                              "bool",  "string", "array", "uint64", "int64",  "float64"};
    return t <= 12 ? n[t] : "?";
}

// One scalar (or string) value; arrays hold their elements.
struct Value {
    uint32_t type = 0;
    uint64_t u = 0;   // unsigned integers and bool
    int64_t i = 0;    // signed integers
    double f = 0.0;   // floats
    std::string s;
    uint32_t arr_type = 0;
    std::vector<Value> arr;
};

struct Tensor {
    std::string name;
    uint32_t type;
    int64_t ne[4];
    uint64_t nb[4];
    uint64_t offset;
    int part;
    uint64_t size() const { return nb[3] * (uint64_t)ne[3]; }
};

struct Part {
    void *map = nullptr;
    size_t len = 0;
    uint64_t data_offset = 0;
};

struct ParseError {
    std::string msg;
};

[[noreturn]] void fail(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    throw ParseError{buf};
}

struct Cursor {
    const uint8_t *buf;
    size_t len, pos = 0;
    const uint8_t *take(size_t n, const char *what) {
        if (n > len - pos) fail("truncated file while reading %s", what);
        const uint8_t *p = buf + pos;
        pos += n;
        return p;
    }
    template <typename T>
    T get(const char *what) {
        T v;
        memcpy(&v, take(sizeof(T), what), sizeof(T));
        return v;
    }
    std::string str(const char *what) {
        const uint64_t n = get<uint64_t>(what);
        if (n > len - pos) fail("truncated file while reading %s", what);
        const uint8_t *p = take((size_t)n, what);
        return std::string((const char *)p, (size_t)n);
    }
    Value value(uint32_t ty, const char *what) {
        Value v;
        v.type = ty;
        switch (ty) {
        case T_U8: v.u = get<uint8_t>(what); break;
        case T_I8: v.i = get<int8_t>(what); break;
        case T_U16: v.u = get<uint16_t>(what); break;
        case T_I16: v.i = get<int16_t>(what); break;
        case T_U32: v.u = get<uint32_t>(what); break;
        case T_I32: v.i = get<int32_t>(what); break;
        case T_F32: v.f = get<float>(what); break;
        case T_BOOL: v.u = get<uint8_t>(what) != 0; break;
        case T_STR: v.s = str(what); break;
        case T_U64: v.u = get<uint64_t>(what); break;
        case T_I64: v.i = get<int64_t>(what); break;
        case T_F64: v.f = get<double>(what); break;
        case T_ARR: {
            const uint32_t et = get<uint32_t>(what);
            if (et > 12 || et == T_ARR) fail("invalid gguf array element type %u", et);
            const uint64_t n = get<uint64_t>(what);
            // every element takes at least one byte of the file: a count the
            // rest of the file cannot hold is a truncated file, refused before
            // any element is built (each Value costs ~100 bytes of host memory)
            if (n > len - pos) fail("truncated file while reading %s", what);
            v.arr_type = et;
            v.arr.reserve((size_t)std::min<uint64_t>(n, 1u << 20));
            for (uint64_t k = 0; k < n; k++) v.arr.push_back(value(et, what));
            break;
        }
        default: fail("invalid gguf metadata type %u", ty);
        }
        return v;
    }
};

}  // namespace

struct ghip_gguf {
    uint32_t version = 0;
    std::vector<std::pair<std::string, Value>> kv;
    std::vector<Tensor> tensors;
    uint64_t alignment = kDefaultAlignment;
    uint64_t data_offset = 0;
    std::vector<Part> parts;
    ~ghip_gguf() {
        for (Part &p : parts)
            if (p.map && p.map != MAP_FAILED) munmap(p.map, p.len);
    }
    int64_t find_key(const char *k) const {
        for (size_t i = 0; i < kv.size(); i++)
            if (kv[i].first == k) return (int64_t)i;
        return -1;
    }
};

namespace {

// one file: gguf_init_from_file (gguf.rs:488-600)
ghip_gguf *open_single(const std::string &path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) fail("io error: cannot open %s: %s", path.c_str(), strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        fail("io error: cannot stat %s", path.c_str());
    }
    Part part;
    part.len = (size_t)st.st_size;
    part.map = part.len ? mmap(nullptr, part.len, PROT_READ, MAP_PRIVATE, fd, 0) : nullptr;
    ::close(fd);
    if (part.len && part.map == MAP_FAILED) fail("io error: cannot map %s", path.c_str());
    ghip_gguf *g = new ghip_gguf();
    g->parts.push_back(part);
    try {
        Cursor c{(const uint8_t *)part.map, part.len};
        const uint8_t *magic = c.take(4, "magic");
        if (memcmp(magic, "GGUF", 4) != 0) fail("not a GGUF file (bad magic)");
        g->version = c.get<uint32_t>("version");
        if (g->version > kGgufVersion) fail("unsupported GGUF version %u (max %u)", g->version, kGgufVersion);
        const uint64_t n_tensors = c.get<uint64_t>("tensor count");
        const uint64_t n_kv = c.get<uint64_t>("kv count");
        for (uint64_t i = 0; i < n_kv; i++) {
            std::string key = c.str("kv pair");
            if (key.empty()) fail("truncated file while reading empty kv key");
            if (g->find_key(key.c_str()) >= 0) fail("duplicate key '%s'", key.c_str());
            const uint32_t ty = c.get<uint32_t>("kv type");
            if (ty > 12) fail("invalid gguf metadata type %u", ty);
            g->kv.emplace_back(std::move(key), c.value(ty, "kv value"));
        }
        const int64_t ai = g->find_key("general.alignment");
        if (ai >= 0) {
            uint32_t a;
            if (!ghip_gguf_get_u32(g, ai, -1, &a))
                fail("key 'general.alignment' is %s, expected uint32", type_name(g->kv[ai].second.type));
            if (a == 0 || (a & (a - 1)) != 0) fail("alignment %u not a power of 2", a);
            g->alignment = a;
        }
        for (uint64_t i = 0; i < n_tensors; i++) {
            Tensor t;
            t.name = c.str("tensor info");
            if (t.name.size() >= kMaxName) fail("tensor name too long: '%s'", t.name.c_str());
            for (const Tensor &o : g->tensors)
                if (o.name == t.name) fail("duplicate tensor name '%s'", t.name.c_str());
            const uint32_t n_dims = c.get<uint32_t>("tensor n_dims");
            if (n_dims > 4) fail("tensor '%s' has invalid shape/type", t.name.c_str());
            for (int j = 0; j < 4; j++) {
                t.ne[j] = 1;
                if ((uint32_t)j < n_dims) {
                    t.ne[j] = c.get<int64_t>("tensor ne");
                    if (t.ne[j] < 0) fail("tensor '%s' has invalid shape/type", t.name.c_str());
                }
            }
            t.type = c.get<uint32_t>("tensor type");
            int64_t blck, bytes;
            if (!ggml_type_size(t.type, blck, bytes) || t.ne[0] % blck != 0)
                fail("tensor '%s' has invalid shape/type", t.name.c_str());
            // strides and the element count in checked arithmetic: a shape
            // whose byte size does not fit 64 bits is refused (gguf.rs:561-568
            // forms the same products), so size() and every later bounds
            // check see the true extent
            int64_t nel = 1;
            uint64_t nb1, nb2, nb3, total;
            bool ovf = false;
            for (int j = 0; j < 4; j++) ovf |= __builtin_mul_overflow(nel, t.ne[j], &nel);
            ovf |= __builtin_mul_overflow((uint64_t)bytes, (uint64_t)(t.ne[0] / blck), &nb1);
            ovf |= __builtin_mul_overflow(nb1, (uint64_t)t.ne[1], &nb2);
            ovf |= __builtin_mul_overflow(nb2, (uint64_t)t.ne[2], &nb3);
            ovf |= __builtin_mul_overflow(nb3, (uint64_t)t.ne[3], &total);
            if (ovf) fail("tensor '%s' has invalid shape/type", t.name.c_str());
            t.nb[0] = (uint64_t)bytes;
            t.nb[1] = nb1;
            t.nb[2] = nb2;
            t.nb[3] = nb3;
            t.offset = c.get<uint64_t>("tensor offset");
            t.part = 0;
            g->tensors.push_back(std::move(t));
        }
        // the data section is padded to the alignment (only when tensors exist)
        g->data_offset = n_tensors > 0 ? (c.pos + g->alignment - 1) / g->alignment * g->alignment : c.pos;
        g->parts[0].data_offset = g->data_offset;
    } catch (...) {
        delete g;
        throw;
    }
    return g;
}

// exact u16 (gguf_get_val_u16, gguf.rs:168-174)
bool exact_u16(const ghip_gguf *g, int64_t i, uint16_t &out) {
    if (i < 0) return false;
    const Value &v = g->kv[(size_t)i].second;
    if (v.type != T_U16) return false;
    out = (uint16_t)v.u;
    return true;
}

std::string split_path(const std::string &prefix, int no, int count) {
    char buf[64];
    snprintf(buf, sizeof buf, "-%05d-of-%05d.gguf", no + 1, count);
    return prefix + buf;
}

// Gguf::open (gguf.rs:388-480): part 0's kv is the metadata; every part's
// tensors are appended in order, each reading its own file
ghip_gguf *open_splits(const std::string &path) {
    ghip_gguf *g = open_single(path);
    const int64_t ci = g->find_key("split.count");
    if (ci < 0) return g;
    try {
        uint16_t n_split;
        if (!exact_u16(g, ci, n_split))
            fail("key 'split.count' is %s, expected uint16", type_name(g->kv[ci].second.type));
        if (n_split <= 1) return g;
        uint16_t idx;
        if (!exact_u16(g, g->find_key("split.no"), idx)) fail("key not found: 'split.no'");
        if (idx != 0)
            fail("tensor '%s' has invalid shape/type",
                 ("illegal split file idx: " + std::to_string(idx) + " (file: " + path +
                  "), model must be loaded with the first split").c_str());
        const std::string post = split_path("", 0, n_split);
        if (path.size() <= post.size() || path.compare(path.size() - post.size(), post.size(), post) != 0)
            fail("tensor '%s' has invalid shape/type", ("invalid split file name: " + path).c_str());
        const std::string prefix = path.substr(0, path.size() - post.size());
        for (int k = 1; k < n_split; k++) {
            const std::string fn = split_path(prefix, k, n_split);
            ghip_gguf *p;
            try {
                p = open_single(fn);
            } catch (const ParseError &) {
                fail("tensor '%s' has invalid shape/type",
                     ("llama_model_loader: failed to load GGUF split from " + fn).c_str());
            }
            uint16_t pno;
            if (!exact_u16(p, p->find_key("split.no"), pno)) {
                delete p;
                fail("tensor '%s' has invalid shape/type", ("missing key split.no in GGUF split " + fn).c_str());
            }
            if (pno != k) {
                delete p;
                fail("tensor '%s' has invalid shape/type",
                     ("invalid split file idx: " + std::to_string(pno) + " (file: " + fn + "), expected " +
                      std::to_string(k)).c_str());
            }
            const int part_no = (int)g->parts.size();
            g->parts.push_back(p->parts[0]);
            p->parts.clear();  // the mapping now belongs to g
            for (Tensor &t : p->tensors) {
                for (const Tensor &o : g->tensors)
                    if (o.name == t.name) {
                        const std::string dup = t.name;  // t lives in p
                        delete p;
                        fail("duplicate tensor name '%s'", dup.c_str());
                    }
                t.part = part_no;
                g->tensors.push_back(t);
            }
            delete p;
        }
        uint32_t nt;
        const int64_t ti = g->find_key("split.tensors.count");
        if (ti < 0 || !ghip_gguf_get_u32(g, ti, -1, &nt)) fail("key not found: 'split.tensors.count'");
        if (nt != g->tensors.size())
            fail("tensor '%s' has invalid shape/type",
                 ("corrupted model: " + std::to_string(nt) + " tensors expected but " +
                  std::to_string(g->tensors.size()) + " found").c_str());
    } catch (...) {
        delete g;
        throw;
    }
    return g;
}

const Value *elem(const ghip_gguf *g, int64_t i, int64_t j) {
    if (!g || i < 0 || (size_t)i >= g->kv.size()) return nullptr;
    const Value &v = g->kv[(size_t)i].second;
    if (j < 0) return &v;
    if (v.type != T_ARR || (size_t)j >= v.arr.size()) return nullptr;
    return &v.arr[(size_t)j];
}

}  // namespace

extern "C" {

ghip_status ghip_gguf_open(const char *path, int follow_splits, ghip_gguf **out, char *err, size_t err_len) {
    if (!out || !path) return GHIP_STATUS_BACKEND_ERROR;
    *out = nullptr;
    try {
        *out = follow_splits ? open_splits(path) : open_single(path);
        if (err && err_len) err[0] = 0;
        return GHIP_STATUS_SUCCESS;
    } catch (const ParseError &e) {
        if (err && err_len) snprintf(err, err_len, "%s", e.msg.c_str());
        return GHIP_STATUS_BACKEND_ERROR;
    }
}

void ghip_gguf_close(ghip_gguf *g) { delete g; }

uint32_t ghip_gguf_version(const ghip_gguf *g) { return g ? g->version : 0; }
uint64_t ghip_gguf_alignment(const ghip_gguf *g) { return g ? g->alignment : 0; }
uint64_t ghip_gguf_data_offset(const ghip_gguf *g) { return g ? g->data_offset : 0; }
int64_t ghip_gguf_n_kv(const ghip_gguf *g) { return g ? (int64_t)g->kv.size() : 0; }
int64_t ghip_gguf_n_parts(const ghip_gguf *g) { return g ? (int64_t)g->parts.size() : 0; }

const char *ghip_gguf_key(const ghip_gguf *g, int64_t i) {
    return g && i >= 0 && (size_t)i < g->kv.size() ? g->kv[(size_t)i].first.c_str() : nullptr;
}
int64_t ghip_gguf_find_key(const ghip_gguf *g, const char *key) { return g && key ? g->find_key(key) : -1; }

int32_t ghip_gguf_kv_type(const ghip_gguf *g, int64_t i) {
    const Value *v = elem(g, i, -1);
    return v ? (int32_t)v->type : -1;
}
int32_t ghip_gguf_arr_type(const ghip_gguf *g, int64_t i) {
    const Value *v = elem(g, i, -1);
    return v && v->type == T_ARR ? (int32_t)v->arr_type : -1;
}
int64_t ghip_gguf_arr_n(const ghip_gguf *g, int64_t i) {
    const Value *v = elem(g, i, -1);
    return v && v->type == T_ARR ? (int64_t)v->arr.size() : -1;
}

// Value::as_u32 (gguf.rs:156-168): unsigned and signed integers that fit
int ghip_gguf_get_u32(const ghip_gguf *g, int64_t i, int64_t j, uint32_t *out) {
    const Value *v = elem(g, i, j);
    if (!v || !out) return 0;
    switch (v->type) {
    case T_U8: case T_U16: case T_U32: *out = (uint32_t)v->u; return 1;
    case T_I8: case T_I16: *out = (uint32_t)v->i; return 1;  // `as u32` wraps, as the reference's cast
    case T_I32: case T_I64:
        if (v->i < 0 || v->i > (int64_t)UINT32_MAX) return 0;
        *out = (uint32_t)v->i;
        return 1;
    case T_U64:
        if (v->u > UINT32_MAX) return 0;
        *out = (uint32_t)v->u;
        return 1;
    default: return 0;
    }
}
// Value::as_u16: the exact type only
int ghip_gguf_get_u16(const ghip_gguf *g, int64_t i, int64_t j, uint16_t *out) {
    const Value *v = elem(g, i, j);
    if (!v || !out || v->type != T_U16) return 0;
    *out = (uint16_t)v->u;
    return 1;
}
// Value::as_f32 (gguf.rs:141-155): floats and every integer type
int ghip_gguf_get_f32(const ghip_gguf *g, int64_t i, int64_t j, float *out) {
    const Value *v = elem(g, i, j);
    if (!v || !out) return 0;
    switch (v->type) {
    case T_F32: case T_F64: *out = (float)v->f; return 1;
    case T_U8: case T_U16: case T_U32: case T_U64: *out = (float)v->u; return 1;
    case T_I8: case T_I16: case T_I32: case T_I64: *out = (float)v->i; return 1;
    default: return 0;
    }
}
// the stored integer, widened (any integer type; no cast rules)
int ghip_gguf_get_i64(const ghip_gguf *g, int64_t i, int64_t j, int64_t *out) {
    const Value *v = elem(g, i, j);
    if (!v || !out) return 0;
    switch (v->type) {
    case T_U8: case T_U16: case T_U32: case T_U64: *out = (int64_t)v->u; return 1;
    case T_I8: case T_I16: case T_I32: case T_I64: *out = v->i; return 1;
    default: return 0;
    }
}
int ghip_gguf_get_f64(const ghip_gguf *g, int64_t i, int64_t j, double *out) {
    const Value *v = elem(g, i, j);
    if (!v || !out || (v->type != T_F32 && v->type != T_F64)) return 0;
    *out = v->f;
    return 1;
}
int ghip_gguf_get_bool(const ghip_gguf *g, int64_t i, int64_t j, int *out) {
    const Value *v = elem(g, i, j);
    if (!v || !out || v->type != T_BOOL) return 0;
    *out = (int)v->u;
    return 1;
}
int ghip_gguf_get_str(const ghip_gguf *g, int64_t i, int64_t j, const char **s, size_t *n) {
    const Value *v = elem(g, i, j);
    if (!v || !s || v->type != T_STR) return 0;
    *s = v->s.data();
    if (n) *n = v->s.size();
    return 1;
}

int64_t ghip_gguf_n_tensors(const ghip_gguf *g) { return g ? (int64_t)g->tensors.size() : 0; }

int64_t ghip_gguf_find_tensor(const ghip_gguf *g, const char *name) {
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->tensors.size(); i++)
        if (g->tensors[i].name == name) return (int64_t)i;
    return -1;
}

ghip_status ghip_gguf_tensor(const ghip_gguf *g, int64_t i, ghip_gguf_tensor_info *out) {
    if (!g || !out || i < 0 || (size_t)i >= g->tensors.size()) return GHIP_STATUS_BACKEND_ERROR;
    const Tensor &t = g->tensors[(size_t)i];
    memset(out, 0, sizeof *out);
    snprintf(out->name, sizeof out->name, "%s", t.name.c_str());
    out->type = (int32_t)t.type;
    for (int j = 0; j < 4; j++) {
        out->ne[j] = t.ne[j];
        out->nb[j] = t.nb[j];
    }
    out->offset = t.offset;
    out->size = t.size();
    out->part = t.part;
    return GHIP_STATUS_SUCCESS;
}

// tensor_data (gguf.rs:632-640): the bytes in the part that declares it, or
// NULL when they lie outside that file
const void *ghip_gguf_tensor_data(const ghip_gguf *g, int64_t i) {
    if (!g || i < 0 || (size_t)i >= g->tensors.size()) return nullptr;
    const Tensor &t = g->tensors[(size_t)i];
    const Part &p = g->parts[(size_t)t.part];
    const uint64_t start = p.data_offset + t.offset, n = t.size();
    if (start > p.len || n > p.len - start) return nullptr;
    return (const uint8_t *)p.map + start;
}

ghip_status ghip_gguf_upload(ghip_context *ctx, const ghip_gguf *g, int64_t i, void *dst, int register_weight,
                             void *stream) {
    if (!ctx) return GHIP_STATUS_BACKEND_ERROR;
    const void *src = ghip_gguf_tensor_data(g, i);
    if (!src) return ghip_context_fail(ctx, GHIP_STATUS_BACKEND_ERROR, "gguf_upload: no such tensor, or its bytes lie outside the file");
    if (!dst) return ghip_context_fail(ctx, GHIP_STATUS_BACKEND_ERROR, "gguf_upload: null destination");
    const Tensor &t = g->tensors[(size_t)i];
    ghip_status st = ghip_context_upload(ctx, dst, src, t.size(), stream);
    if (st != GHIP_STATUS_SUCCESS || !register_weight) return st;
    ghip_tensor w;
    memset(&w, 0, sizeof w);
    w.type = (int32_t)t.type;
    for (int j = 0; j < 4; j++) {
        w.ne[j] = t.ne[j];
        w.nb[j] = t.nb[j];
    }
    w.data = dst;
    st = ghip_weight_register(ctx, &w, stream);
    if (st != GHIP_STATUS_SUCCESS) return st;
    return ghip_synchronize(ctx, stream);
}

}  // extern "C"
