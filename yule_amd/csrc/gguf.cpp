// gguf.cpp — GGUF v3 reader (yule-core/src/gguf.rs:271-432) and a decode
// runner built straight from a GGUF file (yule-infer weight_loader.rs:
// 78-199 tensor names, model_runner.rs:384-465 configuration defaults).
//
// The file is memory-mapped read-only; every read goes through a
// bounds-checked cursor with the reference's limits (strings <= 1 MiB,
// <= 100k tensors and metadata pairs, arrays <= 10M elements, <= 8 dims),
// then tensor extents are checked against the file size and against each
// other (no overlaps), as gguf.rs does.  Tensor offsets are relative to the
// data section, which starts at the header end rounded up to
// general.alignment (default 32).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "internal.h"

namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;   // "GGUF"
constexpr uint32_t kGgufVersion = 3;
constexpr uint64_t kMaxStringLen = 1024 * 1024;
constexpr uint64_t kMaxTensorCount = 100000;
constexpr uint64_t kMaxKvCount = 100000;
constexpr uint64_t kMaxArrayLen = 10000000;
constexpr uint32_t kMaxDims = 8;
constexpr size_t kHeaderMinSize = 4 + 4 + 8 + 8;

// metadata value types (gguf.rs:19-32)
enum : uint32_t {
    T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
    T_STRING = 8, T_ARRAY = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12
};

struct Value {
    uint32_t type = 0;
    uint64_t u = 0;     // unsigned integer types and bool
    int64_t i = 0;      // signed integer types
    double f = 0.0;     // f32 / f64
    std::string s;
    uint64_t array_len = 0;
    uint32_t array_type = 0;
};

struct Tensor {
    std::string name;
    uint32_t dtype = 0;
    uint32_t n_dims = 0;
    uint64_t dims[kMaxDims] = {};
    uint64_t offset = 0, size = 0;
};

// (weights per block, bytes per block) of every GGUF type id Yule knows
// (dtype.rs:62-118, 155-190); false for unknown ids
bool type_geometry(uint32_t id, uint64_t *bs, uint64_t *bb, bool *quantized) {
    static const std::map<uint32_t, std::pair<uint32_t, uint32_t>> g = {
        {0, {1, 4}},     {1, {1, 2}},      {2, {32, 18}},    {3, {32, 20}},   {6, {32, 22}},   {7, {32, 24}},
        {8, {32, 34}},   {9, {32, 36}},    {10, {256, 84}},  {11, {256, 110}}, {12, {256, 144}}, {13, {256, 176}},
        {14, {256, 210}}, {15, {256, 292}}, {16, {256, 66}},  {17, {256, 74}},  {18, {256, 98}},  {19, {256, 50}},
        {20, {32, 18}},  {21, {256, 110}}, {22, {256, 82}},  {23, {256, 136}}, {24, {1, 1}},     {25, {1, 2}},
        {26, {1, 4}},    {27, {1, 8}},     {28, {1, 8}},     {29, {256, 56}},  {30, {1, 2}},     {34, {256, 54}},
        {35, {256, 66}}};
    auto it = g.find(id);
    if (it == g.end()) return false;
    *bs = it->second.first;
    *bb = it->second.second;
    *quantized = !(id <= 1 || (id >= 24 && id <= 28) || id == 30);
    return true;
}

// Well-formed UTF-8 as Rust's String::from_utf8 accepts it (gguf.rs:226-243
// rejects anything else): no overlong forms, no surrogates, nothing above
// U+10FFFF.
bool valid_utf8(const uint8_t *p, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = p[i];
        if (c < 0x80) { i++; continue; }
        size_t len;
        uint8_t lo = 0x80, hi = 0xBF;   // bounds of the first continuation byte
        if (c >= 0xC2 && c <= 0xDF) len = 2;
        else if (c == 0xE0) { len = 3; lo = 0xA0; }
        else if ((c >= 0xE1 && c <= 0xEC) || c == 0xEE || c == 0xEF) len = 3;
        else if (c == 0xED) { len = 3; hi = 0x9F; }
        else if (c == 0xF0) { len = 4; lo = 0x90; }
        else if (c >= 0xF1 && c <= 0xF3) len = 4;
        else if (c == 0xF4) { len = 4; hi = 0x8F; }
        else return false;
        if (n - i < len || p[i + 1] < lo || p[i + 1] > hi) return false;
        for (size_t k = 2; k < len; k++)
            if (p[i + k] < 0x80 || p[i + k] > 0xBF) return false;
        i += len;
    }
    return true;
}

struct Cursor {
    const uint8_t *p;
    size_t n, pos = 0;
    std::string err;
    bool need(size_t k) {
        if (n - pos < k) {
            if (err.empty())
                err = "unexpected EOF at offset " + std::to_string(pos) + ": need " + std::to_string(k) +
                      " bytes, have " + std::to_string(n - pos);
            return false;
        }
        return true;
    }
    template <class T>
    bool rd(T *v) {
        if (!need(sizeof(T))) return false;
        std::memcpy(v, p + pos, sizeof(T));
        pos += sizeof(T);
        return true;
    }
    bool str(std::string *s) {
        uint64_t len;
        if (!rd(&len)) return false;
        if (len > kMaxStringLen) {
            err = "string length " + std::to_string(len) + " exceeds maximum " + std::to_string(kMaxStringLen);
            return false;
        }
        if (!need((size_t)len)) return false;
        if (!valid_utf8(p + pos, (size_t)len)) {
            err = "invalid UTF-8 in string at offset " + std::to_string(pos);
            return false;
        }
        s->assign(reinterpret_cast<const char *>(p + pos), (size_t)len);
        pos += (size_t)len;
        return true;
    }
    // one value of `type`; arrays keep their length and element type (elements are skipped)
    bool value(uint32_t type, Value *v, int depth = 0) {
        v->type = type;
        switch (type) {
        case T_U8: { uint8_t x; if (!rd(&x)) return false; v->u = x; return true; }
        case T_I8: { int8_t x; if (!rd(&x)) return false; v->i = x; return true; }
        case T_U16: { uint16_t x; if (!rd(&x)) return false; v->u = x; return true; }
        case T_I16: { int16_t x; if (!rd(&x)) return false; v->i = x; return true; }
        case T_U32: { uint32_t x; if (!rd(&x)) return false; v->u = x; return true; }
        case T_I32: { int32_t x; if (!rd(&x)) return false; v->i = x; return true; }
        case T_F32: { float x; if (!rd(&x)) return false; v->f = x; return true; }
        case T_BOOL: { uint8_t x; if (!rd(&x)) return false; v->u = x != 0; return true; }
        case T_STRING: return str(&v->s);
        case T_U64: { uint64_t x; if (!rd(&x)) return false; v->u = x; return true; }
        case T_I64: { int64_t x; if (!rd(&x)) return false; v->i = x; return true; }
        case T_F64: { double x; if (!rd(&x)) return false; v->f = x; return true; }
        case T_ARRAY: {
            uint32_t et;
            uint64_t len;
            if (!rd(&et) || !rd(&len)) return false;
            if (len > kMaxArrayLen) {
                err = "array length " + std::to_string(len) + " exceeds maximum " + std::to_string(kMaxArrayLen);
                return false;
            }
            if (depth > 8) {
                err = "nested arrays too deep";
                return false;
            }
            v->array_len = len;
            v->array_type = et;
            Value tmp;
            for (uint64_t k = 0; k < len; k++)
                if (!value(et, &tmp, depth + 1)) return false;
            return true;
        }
        default:
            err = "unknown GGUF value type: " + std::to_string(type);
            return false;
        }
    }
};

}  // namespace

struct yule_gguf {
    void *map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_offset = 0;
    std::map<std::string, Value> kv;
    std::vector<Tensor> tensors;
    ~yule_gguf() {
        if (map) munmap(map, size);
    }
};

using namespace yule;

namespace {

int parse_error(const std::string &m) { return set_error(YULE_ERR_PARSE, "gguf: " + m); }

// GgufParser::parse_bytes (gguf.rs:271-432)
int parse(yule_gguf *g) {
    const uint8_t *p = static_cast<const uint8_t *>(g->map);
    Cursor c{p, g->size};
    uint32_t magic, version;
    uint64_t n_tensors, n_kv;
    if (!c.rd(&magic)) return parse_error(c.err);
    if (magic != kGgufMagic) return parse_error("invalid magic 0x" + [&] {
        char b[16];
        snprintf(b, sizeof b, "%08x", magic);
        return std::string(b);
    }());
    if (!c.rd(&version)) return parse_error(c.err);
    if (version != kGgufVersion) return parse_error("unsupported version " + std::to_string(version));
    g->version = version;
    if (!c.rd(&n_tensors)) return parse_error(c.err);
    if (n_tensors > kMaxTensorCount)
        return parse_error("tensor count " + std::to_string(n_tensors) + " exceeds maximum");
    if (!c.rd(&n_kv)) return parse_error(c.err);
    if (n_kv > kMaxKvCount) return parse_error("KV count " + std::to_string(n_kv) + " exceeds maximum");
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key;
        uint32_t type;
        Value v;
        if (!c.str(&key)) return parse_error("failed to read KV key " + std::to_string(i) + ": " + c.err);
        if (!c.rd(&type) || !c.value(type, &v)) return parse_error("failed to read KV value for '" + key + "': " + c.err);
        g->kv[key] = v;
    }
    g->tensors.resize((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        Tensor &t = g->tensors[(size_t)i];
        if (!c.str(&t.name)) return parse_error("failed to read tensor " + std::to_string(i) + " name: " + c.err);
        if (!c.rd(&t.n_dims)) return parse_error(c.err);
        if (t.n_dims > kMaxDims)
            return parse_error("tensor '" + t.name + "' has " + std::to_string(t.n_dims) + " dimensions, max is 8");
        for (uint32_t d = 0; d < t.n_dims; d++)
            if (!c.rd(&t.dims[d])) return parse_error(c.err);
        if (!c.rd(&t.dtype) || !c.rd(&t.offset)) return parse_error(c.err);
        uint64_t bs, bb;
        bool quant;
        if (!type_geometry(t.dtype, &bs, &bb, &quant)) return parse_error("unknown GGUF dtype: " + std::to_string(t.dtype));
        uint64_t n = 1;
        for (uint32_t d = 0; d < t.n_dims; d++) {
            if (t.dims[d] && n > UINT64_MAX / t.dims[d]) return parse_error("tensor '" + t.name + "': shape overflow");
            n *= t.dims[d];
        }
        const uint64_t units = quant ? (n + bs - 1) / bs : n;
        if (units && bb > UINT64_MAX / units) return parse_error("tensor '" + t.name + "': size overflow");
        t.size = units * bb;
    }
    // data section: header end rounded up to general.alignment (as_u32)
    auto it = g->kv.find("general.alignment");
    if (it != g->kv.end()) {
        const Value &v = it->second;
        if (v.type == T_U32 || v.type == T_U8 || v.type == T_U16) g->alignment = v.u;
        else if (v.type == T_I32 && v.i >= 0) g->alignment = (uint64_t)v.i;
    }
    if (g->alignment == 0) return parse_error("general.alignment is 0");
    g->data_offset = ((uint64_t)c.pos + g->alignment - 1) / g->alignment * g->alignment;
    for (const Tensor &t : g->tensors) {
        const uint64_t a = g->data_offset + t.offset;
        if (a < t.offset || a + t.size < a || a + t.size > g->size)
            return parse_error("tensor '" + t.name + "' out of bounds (offset " + std::to_string(a) + ", file size " +
                               std::to_string(g->size) + ")");
    }
    std::vector<const Tensor *> order;
    for (const Tensor &t : g->tensors) order.push_back(&t);
    std::sort(order.begin(), order.end(), [](const Tensor *a, const Tensor *b) { return a->offset < b->offset; });
    for (size_t i = 1; i < order.size(); i++)
        if (order[i - 1]->offset + order[i - 1]->size > order[i]->offset)
            return parse_error("overlapping tensors: '" + order[i - 1]->name + "' overlaps '" + order[i]->name + "'");
    return YULE_OK;
}

void fill(const yule_gguf *g, const Tensor &t, yule_gguf_tensor *out) {
    out->name = t.name.c_str();
    out->dtype = t.dtype;
    out->n_dims = t.n_dims;
    for (uint32_t d = 0; d < kMaxDims; d++) out->dims[d] = d < t.n_dims ? t.dims[d] : 1;
    out->offset = t.offset;
    out->size_bytes = t.size;
    out->data = static_cast<const uint8_t *>(g->map) + g->data_offset + t.offset;
}

const Tensor *find(const yule_gguf *g, const std::string &name) {
    for (const Tensor &t : g->tensors)
        if (t.name == name) return &t;
    return nullptr;
}

}  // namespace

extern "C" {

int yule_hip_gguf_open(const char *path, yule_gguf **out) {
    if (!path || !out) return set_error(YULE_ERR_INVALID, "gguf_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return set_error(YULE_ERR_IO, std::string("gguf_open: cannot open ") + path + ": " + strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return set_error(YULE_ERR_IO, std::string("gguf_open: cannot stat ") + path);
    }
    if ((size_t)st.st_size < kHeaderMinSize) {
        close(fd);
        return set_error(YULE_ERR_PARSE, "gguf: file too small to be valid GGUF");
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return set_error(YULE_ERR_IO, std::string("gguf_open: mmap failed for ") + path);
    auto *g = new yule_gguf();
    g->map = m;
    g->size = (size_t)st.st_size;
    const int rc = parse(g);
    if (rc) {
        delete g;
        return rc;
    }
    *out = g;
    return YULE_OK;
}

int yule_hip_gguf_close(yule_gguf *g) {
    delete g;
    return YULE_OK;
}

int yule_hip_gguf_header(const yule_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_offset,
                         uint64_t *n_tensors, uint64_t *n_kv) {
    if (!g) return set_error(YULE_ERR_INVALID, "gguf_header: null handle");
    if (version) *version = g->version;
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    if (n_tensors) *n_tensors = g->tensors.size();
    if (n_kv) *n_kv = g->kv.size();
    return YULE_OK;
}

int yule_hip_gguf_tensor(const yule_gguf *g, uint64_t index, yule_gguf_tensor *out) {
    if (!g || !out) return set_error(YULE_ERR_INVALID, "gguf_tensor: null argument");
    if (index >= g->tensors.size()) return set_error(YULE_ERR_INVALID, "gguf_tensor: index out of range");
    fill(g, g->tensors[(size_t)index], out);
    return YULE_OK;
}

int yule_hip_gguf_find(const yule_gguf *g, const char *name, yule_gguf_tensor *out) {
    if (!g || !name || !out) return set_error(YULE_ERR_INVALID, "gguf_find: null argument");
    const Tensor *t = find(g, name);
    if (!t) return set_error(YULE_ERR_INVALID, std::string("gguf: tensor not found: ") + name);
    fill(g, *t, out);
    return YULE_OK;
}

// GgufValue::as_u32 (gguf.rs:50-58)
int yule_hip_gguf_get_u32(const yule_gguf *g, const char *key, uint32_t *out) {
    if (!g || !key || !out) return set_error(YULE_ERR_INVALID, "gguf_get_u32: null argument");
    auto it = g->kv.find(key);
    if (it != g->kv.end()) {
        const Value &v = it->second;
        if (v.type == T_U32 || v.type == T_U8 || v.type == T_U16) { *out = (uint32_t)v.u; return YULE_OK; }
        if (v.type == T_I32 && v.i >= 0) { *out = (uint32_t)v.i; return YULE_OK; }
    }
    return set_error(YULE_ERR_INVALID, std::string("gguf: no u32 metadata ") + key);
}

// GgufValue::as_f64 (gguf.rs:71-77)
int yule_hip_gguf_get_f64(const yule_gguf *g, const char *key, double *out) {
    if (!g || !key || !out) return set_error(YULE_ERR_INVALID, "gguf_get_f64: null argument");
    auto it = g->kv.find(key);
    if (it != g->kv.end() && (it->second.type == T_F32 || it->second.type == T_F64)) {
        *out = it->second.f;
        return YULE_OK;
    }
    return set_error(YULE_ERR_INVALID, std::string("gguf: no float metadata ") + key);
}

int yule_hip_gguf_get_str(const yule_gguf *g, const char *key, const char **out) {
    if (!g || !key || !out) return set_error(YULE_ERR_INVALID, "gguf_get_str: null argument");
    auto it = g->kv.find(key);
    if (it != g->kv.end() && it->second.type == T_STRING) {
        *out = it->second.s.c_str();
        return YULE_OK;
    }
    return set_error(YULE_ERR_INVALID, std::string("gguf: no string metadata ") + key);
}

// Length of an array-valued key (tokenizer.ggml.tokens gives the vocabulary
// size when tokenizer.ggml.vocab_size is absent, gguf.rs:531-543).
int yule_hip_gguf_get_array_len(const yule_gguf *g, const char *key, uint64_t *out) {
    if (!g || !key || !out) return set_error(YULE_ERR_INVALID, "gguf_get_array_len: null argument");
    auto it = g->kv.find(key);
    if (it != g->kv.end() && it->second.type == T_ARRAY) {
        *out = it->second.array_len;
        return YULE_OK;
    }
    return set_error(YULE_ERR_INVALID, std::string("gguf: no array metadata ") + key);
}

// TransformerRunner::new over a GGUF file: GgufFile::to_loaded_model's keys
// (gguf.rs:493-599) and RunnerConfig's defaults (model_runner.rs:384-465:
// norm eps 1e-5 for Llama, rope base 10000, ff_dim from ffn_gate's rows,
// output.weight falling back to token_embd.weight, weight_loader.rs:166-170).
int yule_hip_runner_create_from_gguf(yule_hip_backend *be, const char *path, uint32_t max_seq,
                                     yule_hip_runner **out) {
    if (!be || !path || !out) return set_error(YULE_ERR_INVALID, "runner_create_from_gguf: null argument");
    *out = nullptr;
    yule_gguf *g = nullptr;
    int rc = yule_hip_gguf_open(path, &g);
    if (rc) return rc;
    struct Closer {
        yule_gguf *g;
        ~Closer() { yule_hip_gguf_close(g); }
    } closer{g};
    const char *arch = "unknown";
    yule_hip_gguf_get_str(g, "general.architecture", &arch);
    const std::string a = arch;
    if (a != "llama" && a != "mistral")
        return set_error(YULE_ERR_UNSUPPORTED, "runner_create_from_gguf: architecture '" + a +
                                                   "' (this runner is the dense Llama branch)");
    auto u32 = [&](const std::string &key, uint32_t dflt) {
        uint32_t v;
        return yule_hip_gguf_get_u32(g, key.c_str(), &v) == YULE_OK ? v : dflt;
    };
    auto f64 = [&](const std::string &key, double dflt) {
        double v;
        return yule_hip_gguf_get_f64(g, key.c_str(), &v) == YULE_OK ? v : dflt;
    };
    yule_model_desc d{};
    d.dim = u32(a + ".embedding_length", 0);
    d.n_heads = u32(a + ".attention.head_count", 0);
    d.n_kv_heads = u32(a + ".attention.head_count_kv", d.n_heads);
    d.n_layers = u32(a + ".block_count", 0);
    uint64_t n_tok = 0;
    d.vocab = u32("tokenizer.ggml.vocab_size",
                  yule_hip_gguf_get_array_len(g, "tokenizer.ggml.tokens", &n_tok) == YULE_OK ? (uint32_t)n_tok : 0);
    d.max_seq = max_seq ? max_seq : u32(a + ".context_length", 4096);
    d.norm_eps = (float)f64(a + ".attention.layer_norm_rms_epsilon", 1e-5);
    d.rope_base = (float)f64(a + ".rope.freq_base", 10000.0);
    set_error(YULE_OK, "");
    if (!d.dim || !d.n_heads || !d.n_layers || !d.vocab)
        return set_error(YULE_ERR_INVALID, "runner_create_from_gguf: missing model dimensions in metadata");
    const uint32_t hd = d.dim / d.n_heads, qd = d.n_heads * hd, kvd = d.n_kv_heads * hd;

    // a tensor with the expected [cols, rows] shape (GGUF order) and dtype geometry
    auto tensor = [&](const std::string &name, uint64_t cols, uint64_t rows, const void **ptr, uint32_t *dtype) {
        const Tensor *t = find(g, name);
        if (!t) return set_error(YULE_ERR_INVALID, "runner_create_from_gguf: tensor not found: " + name);
        uint64_t n = 1;
        for (uint32_t k = 0; k < t->n_dims; k++) n *= t->dims[k];
        if (t->dims[0] != cols || n != cols * rows)
            return set_error(YULE_ERR_INVALID, "runner_create_from_gguf: " + name + " has shape [" +
                                                   std::to_string(t->dims[0]) + ", ...] for [" + std::to_string(cols) +
                                                   ", " + std::to_string(rows) + "]");
        yule_gguf_tensor info;
        fill(g, *t, &info);
        *ptr = info.data;
        *dtype = t->dtype;
        return YULE_OK;
    };
    const Tensor *gate0 = find(g, "blk.0.ffn_gate.weight");
    if (!gate0 || gate0->n_dims < 2) return set_error(YULE_ERR_INVALID, "runner_create_from_gguf: no blk.0.ffn_gate.weight");
    d.ff_dim = (uint32_t)gate0->dims[1];
    std::vector<yule_layer_desc> layers(d.n_layers);
    if ((rc = tensor("token_embd.weight", d.dim, d.vocab, &d.token_embd, &d.token_embd_dtype)) ||
        (rc = tensor("output_norm.weight", d.dim, 1, &d.output_norm, &d.output_norm_dtype)))
        return rc;
    if (find(g, "output.weight")) {
        if ((rc = tensor("output.weight", d.dim, d.vocab, &d.output, &d.output_dtype))) return rc;
    } else {
        d.output = d.token_embd;
        d.output_dtype = d.token_embd_dtype;
    }
    for (uint32_t l = 0; l < d.n_layers; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        yule_layer_desc &L = layers[l];
        if ((rc = tensor(p + "attn_norm.weight", d.dim, 1, &L.attn_norm, &L.attn_norm_dtype)) ||
            (rc = tensor(p + "attn_q.weight", d.dim, qd, &L.wq, &L.wq_dtype)) ||
            (rc = tensor(p + "attn_k.weight", d.dim, kvd, &L.wk, &L.wk_dtype)) ||
            (rc = tensor(p + "attn_v.weight", d.dim, kvd, &L.wv, &L.wv_dtype)) ||
            (rc = tensor(p + "attn_output.weight", qd, d.dim, &L.wo, &L.wo_dtype)) ||
            (rc = tensor(p + "ffn_norm.weight", d.dim, 1, &L.ffn_norm, &L.ffn_norm_dtype)) ||
            (rc = tensor(p + "ffn_gate.weight", d.dim, d.ff_dim, &L.w_gate, &L.w_gate_dtype)) ||
            (rc = tensor(p + "ffn_up.weight", d.dim, d.ff_dim, &L.w_up, &L.w_up_dtype)) ||
            (rc = tensor(p + "ffn_down.weight", d.ff_dim, d.dim, &L.w_down, &L.w_down_dtype)))
            return rc;
    }
    d.layers = layers.data();
    return yule_hip_runner_create(be, &d, out);   // uploads every tensor; the mapping closes after
}

}  // extern "C"
