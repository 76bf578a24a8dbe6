// GGUF container parsing and model-config extraction (host code).
//
// Restates src/model/gguf.zig (parse, parseWithOptions :335-419, Reader
// :421-546, MetadataValue conversions :136-193, TensorInfo.sizeBytes
// :222-229) and the dense / MoE part of extractConfigWithLogging
// (src/model/loader.zig:81-346) over a read-only private mmap, as
// loader.load does (loader.zig:420-445). Differences from the reference:
// every read is bounds-checked (a truncated file is an error, not a fault),
// and metadata arrays are recorded by element type, count and file offset
// instead of being materialised (the path reads no array values).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/zinc_hip.h"

namespace {

constexpr uint32_t GGUF_MAGIC = 0x46554747u;  // "GGUF" read as a little-endian u32

// GGMLType block geometry (gguf.zig:75-124): elements per block, bytes per
// block; types without a geometry there have block 1 and 0 bytes.
void ggml_geometry(uint32_t t, uint32_t &bs, uint32_t &bpb) {
    switch (t) {
    case 0: bs = 1; bpb = 4; return;    // f32
    case 1: bs = 1; bpb = 2; return;    // f16
    case 30: bs = 1; bpb = 2; return;   // bf16
    case 28: bs = 1; bpb = 8; return;   // f64
    case 24: bs = 1; bpb = 1; return;   // i8
    case 25: bs = 1; bpb = 2; return;   // i16
    case 26: bs = 1; bpb = 4; return;   // i32
    case 27: bs = 1; bpb = 8; return;   // i64
    case 2: bs = 32; bpb = 18; return;  // q4_0
    case 3: bs = 32; bpb = 20; return;  // q4_1
    case 6: bs = 32; bpb = 22; return;  // q5_0
    case 7: bs = 32; bpb = 24; return;  // q5_1
    case 8: bs = 32; bpb = 34; return;  // q8_0
    case 9: bs = 32; bpb = 36; return;  // q8_1
    case 39: bs = 32; bpb = 17; return; // mxfp4
    case 10: bs = 256; bpb = 84; return;  // q2_k
    case 11: bs = 256; bpb = 110; return; // q3_k
    case 12: bs = 256; bpb = 144; return; // q4_k
    case 13: bs = 256; bpb = 176; return; // q5_k
    case 14: bs = 256; bpb = 210; return; // q6_k
    case 15: bs = 256; bpb = 292; return; // q8_k
    default: bs = 1; bpb = 0; return;
    }
}

struct Value {
    uint32_t type = 0;
    uint64_t bits = 0;      // scalar payload (zero-extended integers, f32/f64 bit patterns)
    std::string str;        // ZH_GGUF_STRING
    uint32_t elem = 0;      // ZH_GGUF_ARRAY: element tag, count, offset of the first element
    uint64_t count = 0, at = 0;
};

struct TensorRec {
    std::string name;
    uint32_t n_dims = 0, type = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint64_t offset = 0;
};

// Sequential little-endian reader; a read past the end sets `bad` and
// returns zeros (the caller checks once per item).
struct Reader {
    const uint8_t *p;
    uint64_t n, pos = 0;
    bool bad = false;
    bool need(uint64_t k) {
        if (bad || k > n - pos) { bad = true; return false; }
        return true;
    }
    uint64_t le(int k) {
        if (!need((uint64_t)k)) return 0;
        uint64_t v = 0;
        for (int i = 0; i < k; i++) v |= (uint64_t)p[pos + i] << (8 * i);
        pos += (uint64_t)k;
        return v;
    }
    std::string str() {
        const uint64_t len = le(8);
        if (!need(len)) return std::string();
        std::string s((const char *)p + pos, (size_t)len);
        pos += len;
        return s;
    }
    void skip_str() {
        const uint64_t len = le(8);
        if (need(len)) pos += len;
    }
};

int scalar_size(uint32_t t) {
    switch (t) {
    case ZH_GGUF_U8: case ZH_GGUF_I8: case ZH_GGUF_BOOL: return 1;
    case ZH_GGUF_U16: case ZH_GGUF_I16: return 2;
    case ZH_GGUF_U32: case ZH_GGUF_I32: case ZH_GGUF_F32: return 4;
    case ZH_GGUF_U64: case ZH_GGUF_I64: case ZH_GGUF_F64: return 8;
    default: return 0;
    }
}

int64_t sext(uint64_t v, int bytes) {
    const int sh = 64 - 8 * bytes;
    return (int64_t)(v << sh) >> sh;
}

// MetadataValue conversions (gguf.zig:143-193)
bool as_u32(const Value &v, uint32_t &o) {
    if (v.type == ZH_GGUF_U32) { o = (uint32_t)v.bits; return true; }
    if (v.type == ZH_GGUF_I32) { const int64_t s = sext(v.bits, 4); if (s < 0) return false; o = (uint32_t)s; return true; }
    if (v.type == ZH_GGUF_U64) { if (v.bits > 0xFFFFFFFFull) return false; o = (uint32_t)v.bits; return true; }
    return false;
}
bool as_u64(const Value &v, uint64_t &o) {
    if (v.type == ZH_GGUF_U64 || v.type == ZH_GGUF_U32) { o = v.bits; return true; }
    if (v.type == ZH_GGUF_I64) { const int64_t s = (int64_t)v.bits; if (s < 0) return false; o = (uint64_t)s; return true; }
    return false;
}
bool as_f32(const Value &v, float &o) {
    if (v.type == ZH_GGUF_F32) { uint32_t b = (uint32_t)v.bits; memcpy(&o, &b, 4); return true; }
    if (v.type == ZH_GGUF_F64) { double d; memcpy(&d, &v.bits, 8); o = (float)d; return true; }
    return false;
}
bool as_bool(const Value &v, int &o) {
    if (v.type == ZH_GGUF_BOOL || v.type == ZH_GGUF_U8 || v.type == ZH_GGUF_U32) { o = v.bits != 0; return true; }
    if (v.type == ZH_GGUF_I32) { o = (uint32_t)v.bits != 0; return true; }
    return false;
}

}  // namespace

struct zh_gguf {
    int fd = -1;
    const uint8_t *data = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t data_offset = 0;
    std::vector<std::pair<std::string, Value>> meta;   // in file order
    std::unordered_map<std::string, size_t> meta_idx;  // key -> last entry with it (the map's put)
    std::vector<TensorRec> tensors;
    std::unordered_map<std::string, size_t> tensor_idx;  // name -> first tensor with it (findTensor)
    std::string err;

    const Value *get(const char *key) const {
        if (!key) return nullptr;
        auto it = meta_idx.find(key);
        return it == meta_idx.end() ? nullptr : &meta[it->second].second;
    }
};

namespace {

std::string g_open_err;  // detail of the last failed zh_gguf_open

int fail(zh_gguf *f, int status, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    f->err = buf;
    return status;
}

// readMetadataValue / readTypedValue (gguf.zig:475-545): an array's elements
// are scalars or strings; elements of any other tag (an array of arrays
// included) are UnknownMetadataType, which the reference only meets when the
// array has at least one element.
int read_value(zh_gguf *f, Reader &r, uint32_t type, Value &v) {
    v.type = type;
    if (type == ZH_GGUF_STRING) {
        v.str = r.str();
    } else if (type == ZH_GGUF_ARRAY) {
        v.elem = (uint32_t)r.le(4);
        v.count = r.le(8);
        v.at = r.pos;
        if (v.elem == ZH_GGUF_STRING) {
            for (uint64_t i = 0; i < v.count && !r.bad; i++) r.skip_str();
        } else {
            const int k = scalar_size(v.elem);
            if (k == 0) {
                if (r.bad || v.count == 0) return ZH_OK;
                return fail(f, ZH_ERR_UNKNOWN_METADATA_TYPE, "array element type %u", v.elem);
            }
            if (v.count > (r.n - r.pos) / (uint64_t)k) r.bad = true;
            else r.pos += v.count * (uint64_t)k;
        }
    } else {
        const int k = scalar_size(type);
        if (k == 0) return fail(f, ZH_ERR_UNKNOWN_METADATA_TYPE, "Unknown GGUF metadata type: %u", type);
        v.bits = r.le(k);
        if (type == ZH_GGUF_BOOL) v.bits = v.bits != 0;
    }
    return ZH_OK;
}

int parse(zh_gguf *f) {
    Reader r{f->data, f->size};
    const uint32_t magic = (uint32_t)r.le(4);
    if (r.bad) return fail(f, ZH_ERR_TRUNCATED_FILE, "file shorter than the GGUF header");
    if (magic != GGUF_MAGIC) return fail(f, ZH_ERR_INVALID_MAGIC, "Invalid GGUF magic: 0x%08x (expected 0x%08x)", magic, GGUF_MAGIC);
    f->version = (uint32_t)r.le(4);
    const uint64_t n_tensors = r.le(8), n_meta = r.le(8);
    if (r.bad) return fail(f, ZH_ERR_TRUNCATED_FILE, "file shorter than the GGUF header");
    // every entry takes at least 12 bytes: a count beyond that is a corrupt header
    if (n_meta > f->size / 12 || n_tensors > f->size / 12)
        return fail(f, ZH_ERR_TRUNCATED_FILE, "counts (%llu tensors, %llu metadata) exceed the file",
                    (unsigned long long)n_tensors, (unsigned long long)n_meta);
    f->meta.reserve((size_t)n_meta);
    for (uint64_t i = 0; i < n_meta; i++) {
        std::string key = r.str();
        const uint32_t type = (uint32_t)r.le(4);
        if (r.bad) return fail(f, ZH_ERR_TRUNCATED_FILE, "metadata entry %llu runs past the end", (unsigned long long)i);
        Value v;
        const int rc = read_value(f, r, type, v);
        if (rc) return rc;
        if (r.bad) return fail(f, ZH_ERR_TRUNCATED_FILE, "metadata '%s' runs past the end", key.c_str());
        f->meta_idx[key] = f->meta.size();
        f->meta.emplace_back(std::move(key), std::move(v));
    }
    f->tensors.reserve((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        TensorRec t;
        t.name = r.str();
        t.n_dims = (uint32_t)r.le(4);
        if (!r.bad && (t.n_dims == 0 || t.n_dims > 4))
            return fail(f, ZH_ERR_INVALID_ARGUMENT, "tensor '%s': %u dimensions", t.name.c_str(), t.n_dims);
        for (uint32_t d = 0; d < t.n_dims; d++) t.dims[d] = r.le(8);
        t.type = (uint32_t)r.le(4);
        t.offset = r.le(8);
        if (r.bad) return fail(f, ZH_ERR_TRUNCATED_FILE, "tensor descriptor %llu runs past the end", (unsigned long long)i);
        f->tensor_idx.emplace(t.name, f->tensors.size());
        f->tensors.push_back(std::move(t));
    }
    // tensor data starts at the next general.alignment boundary (default 32)
    uint64_t align = 32;
    if (const Value *a = f->get("general.alignment")) {
        uint64_t v;
        if (as_u64(*a, v)) align = v;
    }
    if (align == 0 || (align & (align - 1))) return fail(f, ZH_ERR_INVALID_ARGUMENT, "general.alignment %llu", (unsigned long long)align);
    f->data_offset = (r.pos + align - 1) & ~(align - 1);
    return ZH_OK;
}

uint64_t size_bytes(const TensorRec &t) {
    uint64_t n = 1;
    for (uint32_t d = 0; d < t.n_dims; d++) n *= t.dims[d];
    uint32_t bs, bpb;
    ggml_geometry(t.type, bs, bpb);
    return (n + bs - 1) / bs * bpb;
}

}  // namespace

extern "C" int zh_gguf_open(const char *path, zh_gguf **out) {
    if (!path || !out) return ZH_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    zh_gguf *f = new zh_gguf();
    f->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st;
    if (f->fd < 0 || fstat(f->fd, &st) != 0) {
        g_open_err = std::string("open ") + path + ": " + strerror(errno);
        if (f->fd >= 0) close(f->fd);
        delete f;
        return ZH_ERR_IO;
    }
    f->size = (uint64_t)st.st_size;
    if (f->size) {
        void *m = mmap(nullptr, (size_t)f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
        if (m == MAP_FAILED) {
            g_open_err = std::string("mmap ") + path + ": " + strerror(errno);
            close(f->fd);
            delete f;
            return ZH_ERR_IO;
        }
        f->data = (const uint8_t *)m;
    }
    const int rc = parse(f);
    if (rc) {
        g_open_err = f->err;
        zh_gguf_close(f);
        return rc;
    }
    g_open_err.clear();
    *out = f;
    return ZH_OK;
}

extern "C" void zh_gguf_close(zh_gguf *f) {
    if (!f) return;
    if (f->data) munmap((void *)f->data, (size_t)f->size);
    if (f->fd >= 0) close(f->fd);
    delete f;
}

extern "C" const char *zh_gguf_last_error(const zh_gguf *f) { return f ? f->err.c_str() : g_open_err.c_str(); }
extern "C" uint32_t zh_gguf_version(const zh_gguf *f) { return f ? f->version : 0; }
extern "C" uint64_t zh_gguf_tensor_count(const zh_gguf *f) { return f ? f->tensors.size() : 0; }
extern "C" uint64_t zh_gguf_metadata_count(const zh_gguf *f) { return f ? f->meta.size() : 0; }
extern "C" uint64_t zh_gguf_data_offset(const zh_gguf *f) { return f ? f->data_offset : 0; }
extern "C" const void *zh_gguf_data(const zh_gguf *f) { return f ? f->data : nullptr; }
extern "C" uint64_t zh_gguf_file_size(const zh_gguf *f) { return f ? f->size : 0; }

extern "C" int zh_gguf_tensor_info(const zh_gguf *f, uint64_t i, const char **name, uint32_t *n_dims, uint64_t *dims,
                                   uint32_t *type, uint64_t *offset, uint64_t *bytes) {
    if (!f || i >= f->tensors.size()) return ZH_ERR_INVALID_ARGUMENT;
    const TensorRec &t = f->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (n_dims) *n_dims = t.n_dims;
    if (dims) for (int d = 0; d < 4; d++) dims[d] = t.dims[d];
    if (type) *type = t.type;
    if (offset) *offset = t.offset;
    if (bytes) *bytes = size_bytes(t);
    return ZH_OK;
}

extern "C" int64_t zh_gguf_find_tensor(const zh_gguf *f, const char *name) {
    if (!f || !name) return -1;
    auto it = f->tensor_idx.find(name);
    return it == f->tensor_idx.end() ? -1 : (int64_t)it->second;
}

extern "C" int zh_gguf_get_u32(const zh_gguf *f, const char *key, uint32_t *v) {
    const Value *x = f ? f->get(key) : nullptr;
    uint32_t o;
    if (!x || !as_u32(*x, o)) return ZH_ERR_NOT_FOUND;
    if (v) *v = o;
    return ZH_OK;
}
extern "C" int zh_gguf_get_u64(const zh_gguf *f, const char *key, uint64_t *v) {
    const Value *x = f ? f->get(key) : nullptr;
    uint64_t o;
    if (!x || !as_u64(*x, o)) return ZH_ERR_NOT_FOUND;
    if (v) *v = o;
    return ZH_OK;
}
extern "C" int zh_gguf_get_f32(const zh_gguf *f, const char *key, float *v) {
    const Value *x = f ? f->get(key) : nullptr;
    float o;
    if (!x || !as_f32(*x, o)) return ZH_ERR_NOT_FOUND;
    if (v) *v = o;
    return ZH_OK;
}
extern "C" int zh_gguf_get_bool(const zh_gguf *f, const char *key, int *v) {
    const Value *x = f ? f->get(key) : nullptr;
    int o;
    if (!x || !as_bool(*x, o)) return ZH_ERR_NOT_FOUND;
    if (v) *v = o;
    return ZH_OK;
}
extern "C" int zh_gguf_get_string(const zh_gguf *f, const char *key, const char **s, uint64_t *len) {
    const Value *x = f ? f->get(key) : nullptr;
    if (!x || x->type != ZH_GGUF_STRING) return ZH_ERR_NOT_FOUND;
    if (s) *s = x->str.c_str();
    if (len) *len = x->str.size();
    return ZH_OK;
}
extern "C" int zh_gguf_metadata_entry(const zh_gguf *f, uint64_t i, const char **key, uint32_t *type,
                                      uint32_t *elem_type, uint64_t *count) {
    if (!f || i >= f->meta.size()) return ZH_ERR_INVALID_ARGUMENT;
    const auto &e = f->meta[(size_t)i];
    if (key) *key = e.first.c_str();
    if (type) *type = e.second.type;
    if (elem_type) *elem_type = e.second.elem;
    if (count) *count = e.second.type == ZH_GGUF_ARRAY ? e.second.count : 1;
    return ZH_OK;
}

// extractConfigWithLogging (loader.zig:81-346), the fields a dense qwen3 or
// a qwen3moe decoder needs; arch-prefixed keys with the reference's defaults.
extern "C" int zh_gguf_model_config(const zh_gguf *f, uint32_t max_ctx, zh_model_config *cfg) {
    if (!f || !cfg) return ZH_ERR_INVALID_ARGUMENT;
    zh_gguf *fm = const_cast<zh_gguf *>(f);
    const char *arch_c = nullptr;
    std::string arch = zh_gguf_get_string(f, "general.architecture", &arch_c, nullptr) == ZH_OK ? arch_c : "unknown";
    // parseArchitecture (config.zig:53-77): qwen3 -> the dense qwen2 path,
    // qwen3moe -> the qwen2_moe path. qwen2 / qwen2moe map there too but carry
    // Q/K/V biases and no q/k norms, which this decoder does not implement.
    const bool moe = arch == "qwen3moe";
    if (arch != "qwen3" && !moe)
        return fail(fm, ZH_ERR_UNSUPPORTED_ARCHITECTURE, "architecture '%s' (supported here: qwen3, qwen3moe)",
                    arch.c_str());
    auto key = [&](const char *suffix) { return arch + "." + suffix; };
    auto u32_or = [&](const char *suffix, uint32_t dflt) {
        uint32_t v;
        return zh_gguf_get_u32(f, key(suffix).c_str(), &v) == ZH_OK ? v : dflt;
    };
    zh_model_config c;
    memset(&c, 0, sizeof c);
    c.n_layers = u32_or("block_count", 0);
    c.n_heads = u32_or("attention.head_count", 0);
    c.n_kv_heads = u32_or("attention.head_count_kv", c.n_heads);
    c.hidden = u32_or("embedding_length", 0);
    c.head_dim = u32_or("attention.key_length", c.n_heads ? c.hidden / c.n_heads : 0);
    const uint32_t exp_ffn = u32_or("expert_feed_forward_length", 0);
    const uint32_t inter = exp_ffn > 0 ? exp_ffn : u32_or("feed_forward_length", 0);
    c.n_experts = u32_or("expert_count", 0);
    c.n_experts_used = u32_or("expert_used_count", 0);
    if (c.n_experts) c.expert_ffn = inter;
    else c.ffn = inter;
    // vocab: metadata, else the rows of output.weight / token_embd.weight
    c.vocab = u32_or("vocab_size", 0);
    if (c.vocab == 0) {
        int64_t ti = zh_gguf_find_tensor(f, "output.weight");
        if (ti < 0) ti = zh_gguf_find_tensor(f, "token_embd.weight");
        if (ti >= 0) c.vocab = (uint32_t)f->tensors[(size_t)ti].dims[1];
    }
    float eps;
    c.eps = zh_gguf_get_f32(f, key("attention.layer_norm_rms_epsilon").c_str(), &eps) == ZH_OK ? eps : 1e-6f;
    // rope.freq_base: an f32, or a u32 taken as a float, else 10000
    c.rope_base = 10000.0f;
    if (const Value *rb = f->get(key("rope.freq_base").c_str())) {
        if (rb->type == ZH_GGUF_F32) as_f32(*rb, c.rope_base);
        else if (rb->type == ZH_GGUF_U32) c.rope_base = (float)(uint32_t)rb->bits;
    }
    uint32_t ctx_len = u32_or("context_length", 4096);
    uint32_t mc = max_ctx ? max_ctx : ctx_len;
    c.max_ctx = (mc + 15) / 16 * 16;
    // per-class storage types from the tensors of blk.0 (each tensor keeps its
    // own type when the engine loads the file)
    auto type_of = [&](const std::string &name, uint32_t dflt) {
        const int64_t ti = zh_gguf_find_tensor(f, name.c_str());
        return ti >= 0 ? f->tensors[(size_t)ti].type : dflt;
    };
    c.type_embd = type_of("token_embd.weight", ZH_Q4_K);
    c.type_lm_head = type_of("output.weight", c.type_embd);
    c.type_attn = type_of("blk.0.attn_q.weight", ZH_Q4_K);
    c.type_ffn_gate_up = type_of(moe ? "blk.0.ffn_gate_exps.weight" : "blk.0.ffn_gate.weight", ZH_Q4_K);
    c.type_ffn_down = type_of(moe ? "blk.0.ffn_down_exps.weight" : "blk.0.ffn_down.weight", ZH_Q6_K);
    c.type_router = moe ? type_of("blk.0.ffn_gate_inp.weight", ZH_F32) : (uint32_t)ZH_Q8_0;
    c.type_more_bits = 0;
    c.seed = 0;
    if (c.n_layers == 0 || c.n_heads == 0 || c.hidden == 0 || c.vocab == 0 || inter == 0)
        return fail(fm, ZH_ERR_INVALID_ARGUMENT, "incomplete %s metadata (layers %u heads %u hidden %u vocab %u ffn %u)",
                    arch.c_str(), c.n_layers, c.n_heads, c.hidden, c.vocab, inter);
    *cfg = c;
    return ZH_OK;
}
