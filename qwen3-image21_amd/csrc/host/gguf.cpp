// GGUF v2/v3 reader behind the C ABI (qimm_gguf_*): memory-maps the file and
// validates every field against the file size before anything points into it.
//
// Stands in for candle's gguf_file::Content::read / Content::tensor as the
// reference's quantized VarBuilder uses them (src/service.rs:246-258,
// src/gguf_loader.rs:15-40); the name set follows src/gguf_mapping.rs:13-60
// and the fused gate_up of src/quantized_transformer.rs:173-188.
//
// Layout (GGUF spec, little-endian): magic "GGUF", u32 version, u64 tensor
// count, u64 metadata count; metadata entries (string key, u32 value type,
// value); tensor infos (string name, u32 n_dims, u64 ne[n_dims], u32 ggml
// type, u64 offset); padding to general.alignment (default 32); tensor data,
// each tensor at data_start + offset. Strings are u64 length + bytes.
#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "qimm.h"

namespace {

struct Meta {
    std::string key;
    int type = 0;
    int elem_type = -1;
    uint64_t count = 1;
    uint64_t value_off = 0;  // file offset of the value (after the type field)
};

struct Tensor {
    std::string name;
    int type = 0;
    int32_t n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t rel_off = 0;
    uint64_t abs_off = 0;
    uint64_t nbytes = 0;  // 0 = size unknown for this type
};

// (values per block, bytes per block) of the GGML types with a fixed layout.
bool type_size(int t, int64_t &blk, int64_t &bytes) {
    switch (t) {
    case 0: blk = 1; bytes = 4; return true;     // F32
    case 1: blk = 1; bytes = 2; return true;     // F16
    case 2: blk = 32; bytes = 18; return true;   // Q4_0
    case 3: blk = 32; bytes = 20; return true;   // Q4_1
    case 6: blk = 32; bytes = 22; return true;   // Q5_0
    case 7: blk = 32; bytes = 24; return true;   // Q5_1
    case 8: blk = 32; bytes = 34; return true;   // Q8_0
    case 9: blk = 32; bytes = 36; return true;   // Q8_1
    case 10: blk = 256; bytes = 84; return true;  // Q2_K
    case 11: blk = 256; bytes = 110; return true; // Q3_K
    case 12: blk = 256; bytes = 144; return true; // Q4_K
    case 13: blk = 256; bytes = 176; return true; // Q5_K
    case 14: blk = 256; bytes = 210; return true; // Q6_K
    case 15: blk = 256; bytes = 292; return true; // Q8_K
    case 24: blk = 1; bytes = 1; return true;    // I8
    case 25: blk = 1; bytes = 2; return true;    // I16
    case 26: blk = 1; bytes = 4; return true;    // I32
    case 27: blk = 1; bytes = 8; return true;    // I64
    case 28: blk = 1; bytes = 8; return true;    // F64
    case 30: blk = 1; bytes = 2; return true;    // BF16
    default: return false;
    }
}

// Fixed byte size of a scalar metadata type, 0 for string/array/unknown.
uint64_t scalar_size(int t) {
    switch (t) {
    case QIMM_GGUF_U8: case QIMM_GGUF_I8: case QIMM_GGUF_BOOL: return 1;
    case QIMM_GGUF_U16: case QIMM_GGUF_I16: return 2;
    case QIMM_GGUF_U32: case QIMM_GGUF_I32: case QIMM_GGUF_F32: return 4;
    case QIMM_GGUF_U64: case QIMM_GGUF_I64: case QIMM_GGUF_F64: return 8;
    default: return 0;
    }
}

const char *const kPrefix = "model.diffusion_model.";

void put_err(char *err, size_t len, const std::string &m) {
    if (err && len) {
        size_t n = m.size() < len - 1 ? m.size() : len - 1;
        memcpy(err, m.data(), n);
        err[n] = 0;
    }
}

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
    const uint8_t *base;
    uint64_t size, pos = 0;
    bool ok = true;
    std::string why;
    bool need(uint64_t n, const char *what) {
        if (!ok) return false;
        if (n > size || pos > size - n) {
            ok = false;
            why = std::string("truncated while reading ") + what + " at byte " + std::to_string(pos);
            return false;
        }
        return true;
    }
    template <class T>
    T get(const char *what) {
        T v{};
        if (need(sizeof(T), what)) {
            memcpy(&v, base + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    bool str(std::string &out, const char *what) {
        const uint64_t n = get<uint64_t>(what);
        if (!need(n, what)) return false;
        out.assign((const char *)base + pos, (size_t)n);
        pos += n;
        return true;
    }
    bool skip_str(const char *what) {
        const uint64_t n = get<uint64_t>(what);
        if (!need(n, what)) return false;
        pos += n;
        return true;
    }
    void fail(const std::string &m) {
        if (ok) {
            ok = false;
            why = m;
        }
    }
};

}  // namespace

struct qimm_gguf {
    int fd = -1;
    const uint8_t *map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint32_t alignment = 32;
    uint64_t data_off = 0;
    std::vector<Meta> meta;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name, meta_by_key;

    ~qimm_gguf() {
        if (map) munmap((void *)map, size);
        if (fd >= 0) close(fd);
    }
    const Meta *find_meta(const char *key) const {
        auto it = meta_by_key.find(key);
        return it == meta_by_key.end() ? nullptr : &meta[it->second];
    }
    const Tensor *find_tensor(const std::string &name) const {
        auto it = by_name.find(name);
        if (it != by_name.end()) return &tensors[it->second];
        it = by_name.find(kPrefix + name);
        return it == by_name.end() ? nullptr : &tensors[it->second];
    }
};

namespace {

bool parse(qimm_gguf *g, std::string &why) {
    Cursor c{g->map, g->size};
    const uint32_t magic = c.get<uint32_t>("magic");
    if (c.ok && magic != 0x46554747u) c.fail("bad magic (not a GGUF file)");
    g->version = c.get<uint32_t>("version");
    if (c.ok && g->version != 2 && g->version != 3)
        c.fail("unsupported GGUF version " + std::to_string(g->version));
    const uint64_t nt = c.get<uint64_t>("tensor count");
    const uint64_t nkv = c.get<uint64_t>("metadata count");
    // every entry takes at least 12 bytes (tensor info 28): reject counts the file cannot hold
    if (c.ok && (nkv > g->size / 12 || nt > g->size / 28)) c.fail("entry counts exceed the file size");
    for (uint64_t i = 0; c.ok && i < nkv; i++) {
        Meta m;
        c.str(m.key, "metadata key");
        m.type = (int)c.get<uint32_t>("metadata type");
        if (!c.ok) break;
        m.value_off = c.pos;
        if (m.type == QIMM_GGUF_STRING) {
            c.skip_str("metadata string");
        } else if (m.type == QIMM_GGUF_ARRAY) {
            m.elem_type = (int)c.get<uint32_t>("array type");
            m.count = c.get<uint64_t>("array count");
            if (!c.ok) break;
            if (m.elem_type == QIMM_GGUF_STRING) {
                for (uint64_t k = 0; c.ok && k < m.count; k++) c.skip_str("array string");
            } else {
                const uint64_t es = scalar_size(m.elem_type);
                if (!es) c.fail("array of unsupported element type " + std::to_string(m.elem_type) + " in " + m.key);
                else if (m.count > (g->size / es)) c.fail("array " + m.key + " longer than the file");
                else if (c.need(m.count * es, "array data")) c.pos += m.count * es;
            }
        } else {
            const uint64_t s = scalar_size(m.type);
            if (!s) c.fail("unknown metadata value type " + std::to_string(m.type) + " for " + m.key);
            else if (c.need(s, "metadata value")) c.pos += s;
        }
        if (!c.ok) break;
        if (g->meta_by_key.count(m.key)) {
            c.fail("duplicate metadata key " + m.key);
            break;
        }
        g->meta_by_key[m.key] = g->meta.size();
        g->meta.push_back(std::move(m));
    }
    if (c.ok) {
        if (const Meta *a = g->find_meta("general.alignment")) {
            if (a->type != QIMM_GGUF_U32) {
                c.fail("general.alignment is not u32");
            } else {
                uint32_t al;
                memcpy(&al, g->map + a->value_off, 4);
                if (al == 0 || (al & (al - 1))) c.fail("general.alignment " + std::to_string(al) + " is not a power of two");
                g->alignment = al;
            }
        }
    }
    for (uint64_t i = 0; c.ok && i < nt; i++) {
        Tensor t;
        c.str(t.name, "tensor name");
        const uint32_t nd = c.get<uint32_t>("tensor n_dims");
        if (c.ok && (nd < 1 || nd > 4)) c.fail("tensor " + t.name + " has " + std::to_string(nd) + " dims");
        t.n_dims = (int32_t)nd;
        for (uint32_t d = 0; c.ok && d < nd; d++) {
            const uint64_t v = c.get<uint64_t>("tensor dim");
            if (c.ok && (v == 0 || v > ((uint64_t)1 << 40))) c.fail("tensor " + t.name + " has a bad dimension");
            t.ne[d] = (int64_t)v;
        }
        t.type = (int)c.get<uint32_t>("tensor type");
        t.rel_off = c.get<uint64_t>("tensor offset");
        if (!c.ok) break;
        if (g->by_name.count(t.name)) {
            c.fail("duplicate tensor name " + t.name);
            break;
        }
        g->by_name[t.name] = g->tensors.size();
        g->tensors.push_back(std::move(t));
    }
    if (c.ok) {
        const uint64_t a = g->alignment;
        g->data_off = (c.pos + a - 1) / a * a;
        if (g->data_off > g->size && !g->tensors.empty()) c.fail("data section starts past the end of the file");
    }
    for (size_t i = 0; c.ok && i < g->tensors.size(); i++) {
        Tensor &t = g->tensors[i];
        if (t.rel_off % g->alignment) {
            c.fail("tensor " + t.name + " offset is not aligned");
            break;
        }
        t.abs_off = g->data_off + t.rel_off;
        int64_t blk, bytes;
        if (!type_size(t.type, blk, bytes)) continue;  // listed, data not addressable
        if (t.ne[0] % blk) {
            c.fail("tensor " + t.name + " row length " + std::to_string(t.ne[0]) + " is not a multiple of its block");
            break;
        }
        // nb = ne1 * ne2 * ne3 * (ne0 / blk) * bytes, each product checked for
        // overflow: a wrapped size could pass the bounds check below
        uint64_t nb = (uint64_t)(t.ne[0] / blk);
        bool wrap = __builtin_mul_overflow(nb, (uint64_t)bytes, &nb);
        for (int d = 1; d < 4 && !wrap; d++) wrap = __builtin_mul_overflow(nb, (uint64_t)t.ne[d], &nb);
        if (wrap || t.rel_off > g->size || nb > g->size || t.abs_off > g->size || nb > g->size - t.abs_off) {
            c.fail("tensor " + t.name + " data lies outside the file");
            break;
        }
        t.nbytes = nb;
    }
    why = c.why;
    return c.ok;
}

void fill(const qimm_gguf *g, const Tensor &t, qimm_gguf_tensor_info *info) {
    info->name = t.name.c_str();
    info->ggml_type = t.type;
    info->n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) info->ne[d] = t.ne[d];
    info->data = t.nbytes ? (const void *)(g->map + t.abs_off) : nullptr;
    info->nbytes = (size_t)t.nbytes;
    info->offset = t.abs_off;
}

// The known block submodules (src/gguf_mapping.rs:43-59) plus the fused gate_up.
bool known_block_sub(const std::string &s) {
    static const char *const subs[] = {"attn.to_q.weight",        "attn.to_k.weight",          "attn.to_v.weight",
                                       "attn.to_out.0.weight",    "attn.norm_q.weight",        "attn.norm_k.weight",
                                       "img_mlp.proj.weight",     "img_mlp.gate_layer.weight", "img_mlp.out.weight",
                                       "img_mlp.gate_up.weight"};
    for (const char *k : subs)
        if (s == k) return true;
    return false;
}

}  // namespace

extern "C" {

int qimm_gguf_open(const char *path, qimm_gguf **out, char *err, size_t err_len) {
    if (!path || !out) {
        put_err(err, err_len, "null argument");
        return QIMM_ERR_ARG;
    }
    *out = nullptr;
    auto *g = new (std::nothrow) qimm_gguf;
    if (!g) return QIMM_ERR_OOM;
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        put_err(err, err_len, std::string("cannot open ") + path);
        delete g;
        return QIMM_ERR_ARG;
    }
    g->size = (uint64_t)st.st_size;
    if (g->size < 24) {
        put_err(err, err_len, "file too short for a GGUF header");
        delete g;
        return QIMM_ERR_FORMAT;
    }
    void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        put_err(err, err_len, std::string("cannot map ") + path);
        delete g;
        return QIMM_ERR_ARG;
    }
    g->map = (const uint8_t *)m;
    std::string why;
    if (!parse(g, why)) {
        put_err(err, err_len, why);
        delete g;
        return QIMM_ERR_FORMAT;
    }
    *out = g;
    return QIMM_OK;
}

int qimm_gguf_close(qimm_gguf *g) {
    delete g;
    return QIMM_OK;
}

int qimm_gguf_header(const qimm_gguf *g, uint32_t *version, int64_t *n_tensors, int64_t *n_kv,
                     uint32_t *alignment, uint64_t *data_offset) {
    if (!g) return QIMM_ERR_ARG;
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = (int64_t)g->tensors.size();
    if (n_kv) *n_kv = (int64_t)g->meta.size();
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_off;
    return QIMM_OK;
}

int qimm_gguf_tensor_at(const qimm_gguf *g, int64_t i, qimm_gguf_tensor_info *info) {
    if (!g || !info || i < 0 || i >= (int64_t)g->tensors.size()) return QIMM_ERR_ARG;
    fill(g, g->tensors[(size_t)i], info);
    return QIMM_OK;
}

int qimm_gguf_find(const qimm_gguf *g, const char *name, qimm_gguf_tensor_info *info) {
    if (!g || !name || !info) return QIMM_ERR_ARG;
    const Tensor *t = g->find_tensor(name);
    if (!t) return QIMM_ERR_NOT_FOUND;
    fill(g, *t, info);
    return QIMM_OK;
}

int qimm_gguf_meta_at(const qimm_gguf *g, int64_t i, const char **key, int *type, int *elem_type,
                      uint64_t *count) {
    if (!g || i < 0 || i >= (int64_t)g->meta.size()) return QIMM_ERR_ARG;
    const Meta &m = g->meta[(size_t)i];
    if (key) *key = m.key.c_str();
    if (type) *type = m.type;
    if (elem_type) *elem_type = m.elem_type;
    if (count) *count = m.count;
    return QIMM_OK;
}

int qimm_gguf_meta_int(const qimm_gguf *g, const char *key, int64_t *out) {
    if (!g || !key || !out) return QIMM_ERR_ARG;
    const Meta *m = g->find_meta(key);
    if (!m) return QIMM_ERR_NOT_FOUND;
    const uint8_t *p = g->map + m->value_off;
    switch (m->type) {
    case QIMM_GGUF_U8: *out = *p; return QIMM_OK;
    case QIMM_GGUF_BOOL: *out = *p ? 1 : 0; return QIMM_OK;
    case QIMM_GGUF_I8: *out = (int8_t)*p; return QIMM_OK;
    case QIMM_GGUF_U16: { uint16_t v; memcpy(&v, p, 2); *out = v; return QIMM_OK; }
    case QIMM_GGUF_I16: { int16_t v; memcpy(&v, p, 2); *out = v; return QIMM_OK; }
    case QIMM_GGUF_U32: { uint32_t v; memcpy(&v, p, 4); *out = v; return QIMM_OK; }
    case QIMM_GGUF_I32: { int32_t v; memcpy(&v, p, 4); *out = v; return QIMM_OK; }
    case QIMM_GGUF_I64: { int64_t v; memcpy(&v, p, 8); *out = v; return QIMM_OK; }
    case QIMM_GGUF_U64: {
        uint64_t v;
        memcpy(&v, p, 8);
        if (v > (uint64_t)INT64_MAX) return QIMM_ERR_TYPE;
        *out = (int64_t)v;
        return QIMM_OK;
    }
    default: return QIMM_ERR_TYPE;
    }
}

int qimm_gguf_meta_float(const qimm_gguf *g, const char *key, double *out) {
    if (!g || !key || !out) return QIMM_ERR_ARG;
    const Meta *m = g->find_meta(key);
    if (!m) return QIMM_ERR_NOT_FOUND;
    const uint8_t *p = g->map + m->value_off;
    if (m->type == QIMM_GGUF_F32) {
        float v;
        memcpy(&v, p, 4);
        *out = v;
        return QIMM_OK;
    }
    if (m->type == QIMM_GGUF_F64) {
        memcpy(out, p, 8);
        return QIMM_OK;
    }
    return QIMM_ERR_TYPE;
}

int qimm_gguf_meta_string(const qimm_gguf *g, const char *key, const char **str, uint64_t *len) {
    if (!g || !key || !str || !len) return QIMM_ERR_ARG;
    const Meta *m = g->find_meta(key);
    if (!m) return QIMM_ERR_NOT_FOUND;
    if (m->type != QIMM_GGUF_STRING) return QIMM_ERR_TYPE;
    memcpy(len, g->map + m->value_off, 8);
    *str = (const char *)g->map + m->value_off + 8;
    return QIMM_OK;
}

int qimm_gguf_is_known_name(const char *name) {
    if (!name) return 0;
    std::string s(name);
    if (s.compare(0, strlen(kPrefix), kPrefix) == 0) s = s.substr(strlen(kPrefix));
    static const char *const globals[] = {"time_text_embed.timestep_embedder.linear_1.weight",
                                          "time_text_embed.timestep_embedder.linear_2.weight",
                                          "norm_out.linear.weight", "proj_out.weight", "img_in.weight",
                                          "txt_in.in_layer.weight", "txt_in.out_layer.weight",
                                          "txt_in.text_norm.weight", "modulation.1.weight"};
    for (const char *k : globals)
        if (s == k) return 1;
    const std::string pre = "transformer_blocks.";
    if (s.compare(0, pre.size(), pre) != 0) return 0;
    const size_t dot = s.find('.', pre.size());
    if (dot == std::string::npos) return 0;
    size_t k0 = pre.size();
    if (k0 < dot && s[k0] == '+') k0++;  // the index parses as a Rust usize: one leading '+'
    if (k0 == dot) return 0;
    for (size_t k = k0; k < dot; k++)
        if (s[k] < '0' || s[k] > '9') return 0;
    return known_block_sub(s.substr(dot + 1)) ? 1 : 0;
}

int qimm_gguf_block_tensors(const qimm_gguf *g, int64_t layer, qimm_block_tensors *out, char *err,
                            size_t err_len) {
    if (!g || !out || layer < 0) {
        put_err(err, err_len, "null argument or negative layer");
        return QIMM_ERR_ARG;
    }
    memset(out, 0, sizeof(*out));
    const std::string pre = "transformer_blocks." + std::to_string(layer) + ".";
    auto get = [&](const char *sub, qimm_tensor &dst, bool required) -> int {
        const Tensor *t = g->find_tensor(pre + sub);
        if (!t) {
            if (!required) return QIMM_OK;
            put_err(err, err_len, "missing tensor " + pre + sub);
            return QIMM_ERR_NOT_FOUND;
        }
        if (!t->nbytes) {
            put_err(err, err_len, pre + sub + ": GGML type " + std::to_string(t->type) + " has no known layout");
            return QIMM_ERR_TYPE;
        }
        if (t->ne[2] != 1 || t->ne[3] != 1) {
            put_err(err, err_len, pre + sub + " is not a matrix");
            return QIMM_ERR_SHAPE;
        }
        dst.ggml_type = t->type;
        dst.rows = t->ne[1];
        dst.cols = t->ne[0];
        dst.data = g->map + t->abs_off;
        dst.nbytes = (size_t)t->nbytes;
        return QIMM_OK;
    };
    int st;
    if ((st = get("attn.to_q.weight", out->to_q, true))) return st;
    if ((st = get("attn.to_k.weight", out->to_k, true))) return st;
    if ((st = get("attn.to_v.weight", out->to_v, true))) return st;
    if ((st = get("attn.to_out.0.weight", out->to_out, true))) return st;
    if ((st = get("attn.norm_q.weight", out->norm_q, true))) return st;
    if ((st = get("attn.norm_k.weight", out->norm_k, true))) return st;
    if ((st = get("img_mlp.gate_up.weight", out->gate_up, false))) return st;
    if (!out->gate_up.data) {
        if ((st = get("img_mlp.proj.weight", out->proj, true))) return st;
        if ((st = get("img_mlp.gate_layer.weight", out->gate_layer, true))) return st;
    }
    return get("img_mlp.out.weight", out->mlp_out, true);
}

int qimm_gguf_model_tensors(const qimm_gguf *g, qimm_model_tensors *out, char *err, size_t err_len) {
    if (!g || !out) {
        put_err(err, err_len, "null argument");
        return QIMM_ERR_ARG;
    }
    memset(out, 0, sizeof(*out));
    auto get = [&](const char *name, qimm_tensor &dst, bool required) -> int {
        const Tensor *t = g->find_tensor(name);
        if (!t) {
            if (!required) return QIMM_OK;
            put_err(err, err_len, std::string("missing tensor ") + name);
            return QIMM_ERR_NOT_FOUND;
        }
        if (!t->nbytes) {
            put_err(err, err_len, std::string(name) + ": GGML type " + std::to_string(t->type) + " has no known layout");
            return QIMM_ERR_TYPE;
        }
        if (t->ne[2] != 1 || t->ne[3] != 1) {
            put_err(err, err_len, std::string(name) + " is not a matrix");
            return QIMM_ERR_SHAPE;
        }
        dst.ggml_type = t->type;
        dst.rows = t->ne[1];
        dst.cols = t->ne[0];
        dst.data = g->map + t->abs_off;
        dst.nbytes = (size_t)t->nbytes;
        return QIMM_OK;
    };
    int st;
    if ((st = get("img_in.weight", out->img_in, true))) return st;
    if ((st = get("time_text_embed.timestep_embedder.linear_1.weight", out->t_linear_1, true))) return st;
    if ((st = get("time_text_embed.timestep_embedder.linear_2.weight", out->t_linear_2, true))) return st;
    if ((st = get("modulation.1.weight", out->modulation, true))) return st;
    if ((st = get("norm_out.linear.weight", out->norm_out, true))) return st;
    if ((st = get("proj_out.weight", out->proj_out, true))) return st;
    if (g->find_tensor("txt_in.in_layer.weight")) {  // src/quantized_transformer.rs:406-411
        if ((st = get("txt_in.text_norm.weight", out->txt_norm, true))) return st;
        if ((st = get("txt_in.in_layer.weight", out->txt_in, true))) return st;
        if ((st = get("txt_in.out_layer.weight", out->txt_out, true))) return st;
    }
    return QIMM_OK;
}

}  // extern "C"
