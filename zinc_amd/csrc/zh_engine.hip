// zh_engine.hip — the decode-loop engine: InferenceEngine's init /
// decodeStep / sampleGreedy / generate (src/compute/forward.zig:1226,
// :4299-7865, :10338, :10983-11192) on one MI355X.
//
// A token step is a fixed sequence of kernel launches whose every varying
// input (token id, position, generated-token slot) lives in a small device
// state block, so one step is captured once into a hipGraph and replayed:
// greedy decode feeds each argmax back on the device with no host round trip
// (the reference does one submitAndWait + 4-byte readback per token).
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <stdlib.h>

#include <functional>
#include <map>
#include <string>
#include <vector>

#include "zh_device.h"
#include "zh_internal.h"
#include "zh_xcd.h"

// Tensor stream ids (shared with oracle/zinc_oracle.c).
enum : uint64_t { S_TOKEN_EMBD = 1, S_OUTPUT_NORM = 2, S_OUTPUT = 3 };
enum { K_ATTN_NORM = 1, K_WQ, K_WK, K_WV, K_WO, K_Q_NORM, K_K_NORM, K_FFN_NORM, K_GATE, K_UP, K_DOWN, K_ROUTER,
       K_EXP_GATE, K_EXP_UP, K_EXP_DOWN };
static inline uint64_t S_LAYER(uint32_t l, int kind) { return ((uint64_t)(l + 1) << 8) | (uint64_t)kind; }
static inline uint64_t S_KV(uint32_t l, uint32_t which) { return 0x100000ull + 2ull * l + which; }

// Device state words.
enum { ST_STEP = 0, ST_NPROMPT = 2, ST_TOKEN_OUT = 3, ST_POS = 5, ST_TOKEN_IN = 6, ST_GEN = 7, ST_WORDS = 16 };
// words per layer of the routing buffer: [ids u32 x n_experts_used][weights f32 x n_experts_used]
constexpr uint32_t ZH_ROUTE_WORDS = 32;
constexpr uint32_t MAX_PROMPT = 8192;
constexpr uint32_t MAX_GEN = 65536;

struct Tensor {
    uint64_t off = 0, bytes = 0;
    uint32_t type = 0;
    uint64_t rows = 0, cols = 0;
};

struct Layer {
    Tensor attn_norm, wq, wk, wv, wo, q_norm, k_norm, ffn_norm, gate, up, down, router, egate, eup, edown;
    uint16_t *kc = nullptr, *vc = nullptr;
};

struct zh_engine {
    zh_ctx *ctx = nullptr;
    zh_model_config c{};
    uint8_t *arena = nullptr;  // all weights
    bool owns_arena = true;    // false: the weights of another engine (zh_engine_create_shared)
    uint64_t arena_bytes = 0;
    std::map<uint64_t, Tensor> tensors;
    Tensor embd, out_norm, lm;
    std::vector<Layer> L;
    uint16_t *kv = nullptr;  // all caches
    uint32_t *pages = nullptr, n_pages = 0;
    bool pages_ident = true;  // pages[i] == i: the decode step may use the identity-table attention
    float *inv_freq = nullptr;
    float *rope_cs = nullptr;  // [max_ctx][64] (cos, sin)
    // activations
    float *hidden = nullptr, *norm = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr;
    float *s = nullptr, *logits = nullptr, *rl = nullptr, *edown_out = nullptr, *fd_part = nullptr;
    float *u = nullptr;  // up projection when gate and up differ in format (dense)
    uint8_t *xq_h = nullptr, *xq_q = nullptr, *xq_f = nullptr;
    uint32_t *force_ids = nullptr;  // zh_engine_force_routing: [n_layers][n_experts_used] (nullptr: off)
    uint32_t *routing = nullptr, *am_part = nullptr, *st = nullptr, *prompt = nullptr, *ring = nullptr;
    uint32_t *grp_cnt = nullptr;  // SwiGLU-output XQ: one counter per 32-row group (kept zero between launches)
    uint32_t *router_cnt = nullptr;
    uint32_t *am_cnt = nullptr;      // k_argmax_advance: workgroups finished (kept zero between launches)
    // persistent decode-layers kernel: barrier / merge words (zero between
    // launches) and the device table of layer pointers
    uint32_t *step_ctl = nullptr;
    zh_step_layer *step_layers = nullptr;
    bool persistent = false;  // zh_engine_set_persistent
    bool fused_qa = true;     // zh_engine_set_fused_attn: Q/K/V + attention in one launch where it applies
    uint32_t *qa_flags = nullptr;  // its XCD-local flag and epoch words (zero at creation)
    uint64_t *qa_xrows = nullptr;  // its epoch-tagged Q/K/V rows (zero at creation)
    float *xin = nullptr;          // with the O projection in that launch: copy of the residual stream at layer entry
    bool fused_ffn = true;         // zh_engine_set_fused_ffn: the dense FFN as one per-XCD launch where it applies
    uint32_t *ffn_flags = nullptr; // its XCD-local flag and epoch words (zero at creation)
    // split residual of the per-XCD launches: the residual stream is
    // rres[r] + dres[d] (plain rows + atomic sums), alternating per launch
    float *rres = nullptr;         // [2][H]
    zh_fix *dres = nullptr;        // [3][H] (64-bit fixed point: zh_xcd.h)
    // the per-XCD FFN's copy of every layer's ffn_down (zhk_ffn_pack_down),
    // made before a step runs when the arena may have changed since, and its
    // partial sums
    uint8_t *down_pk = nullptr;
    bool pk_stale = true;
    float *ffn_part = nullptr;
    // the per-XCD MoE FFN (k_moe_xcd): flags, scratch (partials, logits) and
    // its packed copy of every layer's expert down matrices
    uint32_t *moe_flags = nullptr;
    float *moe_scratch = nullptr;
    void *act_arena = nullptr;
    hipGraphExec_t g_out = nullptr, g_noout = nullptr;
    uint32_t place_gen = 0;  // the context's place_gen the graphs were recorded under
    bool have_logits = false;
    // batched prefill activations (allocated on first use, PF_CHUNK tokens)
    struct {
        float *hid = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *g = nullptr, *u = nullptr;
        _Float16 *xh = nullptr, *att = nullptr, *s = nullptr;
        float *s_unscale = nullptr;
        uint32_t *ids = nullptr;
        void *arena = nullptr;
    } pf;
};
constexpr uint32_t PF_CHUNK = 512;  // tokens per prefill batch

#define EHIP(e, call) ZH_HIP((e)->ctx, call)
#define ERC(x)                 \
    do {                       \
        int rc_ = (x);         \
        if (rc_) return rc_;   \
    } while (0)

static uint64_t align256(uint64_t x) { return (x + 255) & ~255ull; }

// ---------------------------------------------------------------------------
// Small kernels owned by the engine.
// ---------------------------------------------------------------------------
__global__ void k_advance(uint32_t *st, const uint32_t *prompt) {
    // End of a step: count the generated token, move to the next position and
    // pick the next input token (prompt while it lasts, else the argmax).
    uint32_t s = st[ST_STEP], np = st[ST_NPROMPT];
    if (s + 1 >= np) st[ST_GEN] += 1;
    s += 1;
    st[ST_STEP] = s;
    st[ST_POS] += 1;
    st[ST_TOKEN_IN] = (s < np) ? prompt[s] : st[ST_TOKEN_OUT];
}

// The step's greedy token and the step advance in one launch: every
// workgroup reduces a strided share of the logits (first maximum wins) and
// publishes it with device-scope stores; the last workgroup to count itself
// in (a relaxed device-scope counter after s_waitcnt 0, the engine's
// publication pattern) reduces the shares, records the token
// (argmaxGreedy, forward.zig:10348-10356) and advances the state as
// k_advance. The counter is left zero for the next launch.
constexpr uint32_t TAIL_WGS = 256;  // (am_part holds 256 (value, index) pairs)
__global__ __launch_bounds__(256) void k_argmax_advance(const float *__restrict__ x, uint32_t n, uint32_t *partials,
                                                        uint32_t *cnt, uint32_t *ring, uint32_t *st,
                                                        const uint32_t *prompt) {
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    // 4 logits per load (x is 16-byte aligned); workgroup 0 also takes the n % 4 last ones
    const uint32_t n4 = n / 4;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n4; i += gridDim.x * 256) {
        const float4 v = ((const float4 *)x)[i];
        am_better(bv, bi, v.x, 4 * i);
        am_better(bv, bi, v.y, 4 * i + 1);
        am_better(bv, bi, v.z, 4 * i + 2);
        am_better(bv, bi, v.w, 4 * i + 3);
    }
    if (blockIdx.x == 0 && 4 * n4 + threadIdx.x < n) am_better(bv, bi, x[4 * n4 + threadIdx.x], 4 * n4 + threadIdx.x);
    am_wave(bv, bi);
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    __shared__ uint32_t s_last;
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) am_better(bv, bi, sv[w], si[w]);
        __hip_atomic_store(partials + 2 * blockIdx.x, __float_as_uint(bv), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(partials + 2 * blockIdx.x + 1, bi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        s_last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last) return;
    bv = -INFINITY;
    bi = 0xFFFFFFFFu;
    for (uint32_t i = threadIdx.x; i < gridDim.x; i += 256)
        am_better(bv, bi, __uint_as_float(__hip_atomic_load(partials + 2 * i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)),
                  __hip_atomic_load(partials + 2 * i + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    am_wave(bv, bi);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) am_better(bv, bi, sv[w], si[w]);
        if (bi == 0xFFFFFFFFu) bi = 0;  // all NaN: the scan keeps index 0
        st[ST_TOKEN_OUT] = bi;
        ring[st[ST_GEN]] = bi;
        __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // k_advance
        uint32_t s = st[ST_STEP], np = st[ST_NPROMPT];
        if (s + 1 >= np) st[ST_GEN] += 1;
        s += 1;
        st[ST_STEP] = s;
        st[ST_POS] += 1;
        st[ST_TOKEN_IN] = (s < np) ? prompt[s] : bi;
    }
}

// Seeded N(0,1) fp16 values for logical tokens [0, n) of one layer, written
// into the head-major cache; counter = t*kv_dim + h*head_dim + d, as the
// oracle's token-major fill.
__global__ void k_prefill_kv(uint16_t *cache, uint32_t nkv, uint32_t cache_tokens, uint32_t hd, uint32_t n,
                             uint64_t key, const uint32_t *pages) {
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t total = (uint64_t)n * nkv * hd;
    if (i >= total) return;
    uint32_t d = i % hd;
    uint64_t r = i / hd;
    uint32_t h = r % nkv;
    uint32_t t = (uint32_t)(r / nkv);
    uint64_t z = key + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z = z ^ (z >> 31);
    int sm = (int)(z & 0xFFFF) + (int)((z >> 16) & 0xFFFF) + (int)((z >> 32) & 0xFFFF) + (int)((z >> 48) & 0xFFFF) -
             131070;
    const uint32_t phys = pages[t / 16] * 16 + t % 16;  // logicalTokenToPhysicalToken
    cache[((size_t)h * cache_tokens + phys) * hd + d] = f2h_rn(__fmul_rn((float)sm, 2.6429573e-05f));
}

__global__ void k_gather_kv(const uint16_t *cache, uint32_t nkv, uint32_t cache_tokens, uint32_t hd,
                            const uint32_t *pages, uint32_t t0, uint32_t n, uint16_t *dst) {
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n * nkv * hd) return;
    uint32_t d = i % hd;
    uint64_t r = i / hd;
    uint32_t h = r % nkv, t = t0 + (uint32_t)(r / nkv);
    uint32_t phys = pages[t / 16] * 16 + t % 16;
    dst[i] = cache[((size_t)h * cache_tokens + phys) * hd + d];
}

__global__ void k_fill_pages(uint32_t *pages, uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) pages[i] = i;
}

static uint64_t host_key(uint64_t seed, uint64_t stream) {
    uint64_t z = seed ^ (stream * 0xD1B54A32D192ED03ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// ---------------------------------------------------------------------------
// init
// ---------------------------------------------------------------------------
static bool dmmv_type_ok(uint32_t t) { return t == ZH_Q4_K || t == ZH_Q5_K || t == ZH_Q6_K || t == ZH_Q8_0 || t == ZH_MXFP4; }

// use_more_bits(i_layer, n_layers) of llama.cpp's quantizer: the layers the
// Q4_K_M / Q5_K_M mix stores attn_v and ffn_down in more bits.
static bool more_bits_layer(uint32_t i, uint32_t n) { return i < n / 8 || i >= 7 * n / 8 || (i - n / 8) % 3 == 2; }

// The storage type a tensor gets from the model config: the per-class types,
// with attn_v and ffn_down of the use_more_bits layers in type_more_bits
// when that is set.
static uint32_t config_type(const zh_model_config &c, uint64_t stream, uint32_t cls_type) {
    if (!c.type_more_bits || stream <= 0xFF) return cls_type;
    const uint32_t l = (uint32_t)(stream >> 8) - 1, kind = (uint32_t)(stream & 0xFF);
    if ((kind == K_WV || kind == K_DOWN || kind == K_EXP_DOWN) && more_bits_layer(l, c.n_layers)) return c.type_more_bits;
    return cls_type;
}

// How engine_build fills the weights: per-tensor types (default: from the
// config), seeded synthetic values or left for the caller to upload, and
// whether the LM head shares token_embd (a GGUF file without output.weight).
struct BuildOpts {
    std::function<uint32_t(uint64_t stream, uint32_t dflt)> type_of;
    bool synth = true;
    bool tied_lm = false;
    uint8_t *shared_arena = nullptr;  // use these weights (same layout) instead of allocating
};

static int engine_build(zh_ctx *ctx, const zh_model_config *cfg, const BuildOpts &opt, zh_engine **out) {
    if (!ctx || !cfg || !out) return ZH_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    const zh_model_config &c = *cfg;
    if (c.n_layers == 0 || c.hidden % 256 || c.head_dim != 128 || c.n_kv_heads == 0 || c.n_heads % c.n_kv_heads ||
        c.n_heads / c.n_kv_heads > 8 || ((c.n_heads / c.n_kv_heads) & (c.n_heads / c.n_kv_heads - 1)) || c.vocab == 0 || c.max_ctx == 0 || c.max_ctx % 16)
        return zh_set_err(ctx, ZH_ERR_INVALID_ARGUMENT, "unsupported model shape");
    if (c.n_experts == 0 && (c.ffn == 0 || c.ffn % 256))
        return zh_set_err(ctx, ZH_ERR_INVALID_ARGUMENT, "ffn must be a positive multiple of 256");
    if (c.n_experts && (c.n_experts > 256 || c.n_experts_used == 0 || c.n_experts_used > 16 ||
                        c.n_experts_used > c.n_experts || c.expert_ffn % 256))
        return zh_set_err(ctx, ZH_ERR_INVALID_ARGUMENT, "unsupported MoE shape");
    uint32_t types[] = {c.type_attn, c.type_ffn_gate_up, c.type_ffn_down, c.type_lm_head, c.type_embd};
    for (uint32_t t : types)
        if (!dmmv_type_ok(t)) return zh_set_err(ctx, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "type %u", t);
    if (c.n_experts && !dmmv_type_ok(c.type_router) && c.type_router != ZH_F32)
        return zh_set_err(ctx, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "router");
    if (c.type_more_bits && !dmmv_type_ok(c.type_more_bits))
        return zh_set_err(ctx, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "type_more_bits %u", c.type_more_bits);

    zh_engine *e = new zh_engine();
    e->ctx = ctx;
    e->c = c;
    const uint32_t H = c.hidden, hd = c.head_dim, qd = c.n_heads * hd, kvd = c.n_kv_heads * hd;
    // --- weight layout
    uint64_t off = 0;
    auto add = [&](uint64_t stream, uint32_t type, uint64_t rows, uint64_t cols) -> Tensor {
        Tensor t;
        if (type != ZH_F32) {
            type = config_type(c, stream, type);
            if (opt.type_of) type = opt.type_of(stream, type);
        }
        t.type = type;
        t.rows = rows;
        t.cols = cols;
        t.bytes = (type == ZH_F32) ? rows * cols * 4 : zh_tensor_bytes(type, rows, cols);
        t.off = off;
        off = align256(off + t.bytes);
        e->tensors[stream] = t;
        return t;
    };
    // The f32 norm vectors of every layer first, contiguous (1.2 MB for the 8B
    // shape): read by every workgroup of the projections each step, they stay
    // in the memory-side cache and on few pages, while the matrices stream.
    e->out_norm = add(S_OUTPUT_NORM, ZH_F32, 1, H);
    e->L.resize(c.n_layers);
    for (uint32_t l = 0; l < c.n_layers; l++) {
        Layer &y = e->L[l];
        y.attn_norm = add(S_LAYER(l, K_ATTN_NORM), ZH_F32, 1, H);
        y.q_norm = add(S_LAYER(l, K_Q_NORM), ZH_F32, 1, hd);
        y.k_norm = add(S_LAYER(l, K_K_NORM), ZH_F32, 1, hd);
        y.ffn_norm = add(S_LAYER(l, K_FFN_NORM), ZH_F32, 1, H);
    }
    e->embd = add(S_TOKEN_EMBD, c.type_embd, c.vocab, H);
    if (opt.tied_lm) e->tensors[S_OUTPUT] = e->lm = e->embd;
    else e->lm = add(S_OUTPUT, c.type_lm_head, c.vocab, H);
    for (uint32_t l = 0; l < c.n_layers; l++) {
        Layer &y = e->L[l];
        y.wq = add(S_LAYER(l, K_WQ), c.type_attn, qd, H);
        y.wk = add(S_LAYER(l, K_WK), c.type_attn, kvd, H);
        y.wv = add(S_LAYER(l, K_WV), c.type_attn, kvd, H);
        y.wo = add(S_LAYER(l, K_WO), c.type_attn, H, qd);
        if (c.n_experts == 0) {
            y.gate = add(S_LAYER(l, K_GATE), c.type_ffn_gate_up, c.ffn, H);
            y.up = add(S_LAYER(l, K_UP), c.type_ffn_gate_up, c.ffn, H);
            y.down = add(S_LAYER(l, K_DOWN), c.type_ffn_down, H, c.ffn);
        } else {
            y.router = add(S_LAYER(l, K_ROUTER), c.type_router, c.n_experts, H);
            y.egate = add(S_LAYER(l, K_EXP_GATE), c.type_ffn_gate_up, (uint64_t)c.n_experts * c.expert_ffn, H);
            y.eup = add(S_LAYER(l, K_EXP_UP), c.type_ffn_gate_up, (uint64_t)c.n_experts * c.expert_ffn, H);
            y.edown = add(S_LAYER(l, K_EXP_DOWN), c.type_ffn_down, (uint64_t)c.n_experts * H, c.expert_ffn);
        }
    }
    // every matrix in a format the mat-vec kernels take; the embedding in one
    // the row gather takes; expert gate and up in one format
    // norm weights are f32; a MoE router is f32 or a mat-vec format; every
    // other matrix is in a mat-vec format
    for (auto &kv : e->tensors) {
        const Tensor &t = kv.second;
        const uint64_t kind = kv.first & 0xFF;
        const bool norm = kv.first == S_OUTPUT_NORM || (kv.first > 0xFF && (kind == K_ATTN_NORM || kind == K_Q_NORM ||
                                                                             kind == K_K_NORM || kind == K_FFN_NORM));
        const bool router = kv.first > 0xFF && kind == K_ROUTER;
        const bool ok = norm ? t.type == ZH_F32 : (dmmv_type_ok(t.type) || (router && t.type == ZH_F32));
        if (!ok) {
            const uint64_t st = kv.first;
            delete e;
            return zh_set_err(ctx, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "tensor %llu: type %u", (unsigned long long)st, t.type);
        }
    }
    for (const Layer &y : e->L)
        if (c.n_experts && y.egate.type != y.eup.type) {
            delete e;
            return zh_set_err(ctx, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "expert gate/up types differ");
        }
    e->arena_bytes = off + 256;
    hipError_t he = hipSuccess;
    if (opt.shared_arena) {
        e->arena = opt.shared_arena;
        e->owns_arena = false;
    } else {
        he = hipMalloc((void **)&e->arena, e->arena_bytes);
        if (he != hipSuccess) {
            delete e;
            return zh_set_err(ctx, ZH_ERR_OUT_OF_MEMORY, "weights (%llu B): %s", (unsigned long long)off,
                              hipGetErrorString(he));
        }
    }
    // --- synthetic weights (same streams as the oracle)
    for (auto &kv : e->tensors) {
        if (!opt.synth || opt.shared_arena) break;
        if (kv.first == S_OUTPUT && opt.tied_lm) continue;
        const Tensor &t = kv.second;
        int rc;
        uint64_t kind = kv.first & 0xFF;
        bool is_norm = kv.first == S_OUTPUT_NORM || (kv.first > 0xFF && (kind == K_ATTN_NORM || kind == K_Q_NORM ||
                                                                         kind == K_K_NORM || kind == K_FFN_NORM));
        if (is_norm) rc = zhk_synth_vector(ctx, e->arena + t.off, 2, t.rows * t.cols, 1.f, c.seed, kv.first);
        else rc = zhk_synth_tensor(ctx, e->arena + t.off,
                                   t.type | 0x100u /* centered model init */ |
                                       (kv.first > 0xFF && kind == K_ROUTER ? 0x200u | zh_router_shift(t.cols) << 12 : 0u),
                                   t.rows, t.cols, c.seed, kv.first);
        if (rc) { zh_engine_destroy(e); return rc; }
    }
    // --- KV cache [layer][K|V][nkv][max_ctx][hd] fp16 and identity page table
    uint64_t per = (uint64_t)c.n_kv_heads * c.max_ctx * hd;
    he = hipMalloc((void **)&e->kv, per * 2 * 2 * c.n_layers + 256);
    if (he != hipSuccess) { zh_engine_destroy(e); return zh_set_err(ctx, ZH_ERR_OUT_OF_MEMORY, "kv cache"); }
    for (uint32_t l = 0; l < c.n_layers; l++) {
        e->L[l].kc = e->kv + per * (2 * l);
        e->L[l].vc = e->kv + per * (2 * l + 1);
    }
    e->n_pages = c.max_ctx / 16;
    // --- activations in one arena
    uint32_t F = c.n_experts ? c.expert_ffn * c.n_experts_used : c.ffn;
    uint32_t XK = H > qd ? H : qd;
    struct { void **p; uint64_t bytes; } acts[] = {
        {(void **)&e->hidden, 4ull * H}, {(void **)&e->norm, 4ull * XK}, {(void **)&e->q, 4ull * qd},
        {(void **)&e->k, 4ull * kvd}, {(void **)&e->v, 4ull * kvd}, {(void **)&e->attn, 4ull * qd},
        {(void **)&e->s, 4ull * F}, {(void **)&e->u, 4ull * F}, {(void **)&e->logits, 4ull * c.vocab},
        {(void **)&e->rl, 4ull * 256},
        {(void **)&e->edown_out, 4ull * H * (c.n_experts_used ? c.n_experts_used : 1)},
        {(void **)&e->fd_part, zhk_flash_decode_partials_bytes(c.n_heads, c.n_kv_heads, hd, c.max_ctx)},
        {(void **)&e->xq_h, zh_xq_bytes_int(H)}, {(void **)&e->xq_q, zh_xq_bytes_int(qd)},
        {(void **)&e->xq_f, zh_xq_bytes_int(c.n_experts ? c.expert_ffn : c.ffn) * (c.n_experts_used ? c.n_experts_used : 1)},
        {(void **)&e->routing, 4ull * ZH_ROUTE_WORDS * (c.n_layers ? c.n_layers : 1)}, {(void **)&e->am_part, 8ull * 256}, {(void **)&e->st, 4ull * ST_WORDS},
        {(void **)&e->prompt, 4ull * MAX_PROMPT}, {(void **)&e->ring, 4ull * MAX_GEN}, {(void **)&e->pages, 4ull * e->n_pages},
        {(void **)&e->inv_freq, 4ull * hd / 2}, {(void **)&e->rope_cs, 8ull * c.max_ctx * (hd / 2)},
        {(void **)&e->grp_cnt, 4ull * (F / 32 + 1)}, {(void **)&e->router_cnt, 4}, {(void **)&e->am_cnt, 4},
        {(void **)&e->step_ctl, zh_step_ctl_bytes()}, {(void **)&e->step_layers, sizeof(zh_step_layer) * c.n_layers},
        {(void **)&e->qa_flags, 4ull * zhk_qkv_attn_flag_words()}, {(void **)&e->xin, 4ull * H},
        {(void **)&e->ffn_flags, 4ull * zhk_ffn_xcd_flag_words()}, {(void **)&e->qa_xrows, zhk_qkv_attn_xrows_bytes()}, {(void **)&e->rres, 8ull * H},
        {(void **)&e->dres, 24ull * H},
        {(void **)&e->ffn_part, c.ffn == 12288 && H == 4096 ? zhk_ffn_part_bytes() : 0ull},
        {(void **)&e->moe_flags, 4ull * zhk_moe_xcd_flag_words()},
        {(void **)&e->moe_scratch, c.n_experts ? zhk_moe_part_bytes() : 0ull},
    };
    uint64_t aoff = 0;
    for (auto &a : acts) aoff = align256(aoff + a.bytes);
    he = hipMalloc(&e->act_arena, aoff + 256);
    if (he != hipSuccess) { zh_engine_destroy(e); return zh_set_err(ctx, ZH_ERR_OUT_OF_MEMORY, "activations"); }
    aoff = 0;
    for (auto &a : acts) {
        *a.p = (char *)e->act_arena + aoff;
        aoff = align256(aoff + a.bytes);
    }
    // the exchange words zh_sync resets after a wait gave up
    ctx->xwords.push_back({e, e->qa_flags, 4ull * zhk_qkv_attn_flag_words()});
    ctx->xwords.push_back({e, e->qa_xrows, zhk_qkv_attn_xrows_bytes()});
    ctx->xwords.push_back({e, e->ffn_flags, 4ull * zhk_ffn_xcd_flag_words()});
    if (c.ffn == 12288 && H == 4096) ctx->xwords.push_back({e, e->ffn_part, zhk_ffn_part_bytes()});
    ctx->xwords.push_back({e, e->moe_flags, 4ull * zhk_moe_xcd_flag_words()});
    if (c.n_experts) ctx->xwords.push_back({e, e->moe_scratch, zhk_moe_part_bytes()});
    hipError_t me = hipMemsetAsync(e->act_arena, 0, aoff, ctx->stream);
    if (me != hipSuccess) { zh_engine_destroy(e); return ZH_ERR_HIP; }
    me = hipMemsetAsync(e->kv, 0, per * 4 * c.n_layers, ctx->stream);
    if (me != hipSuccess) { zh_engine_destroy(e); return ZH_ERR_HIP; }
    hipLaunchKernelGGL(k_fill_pages, dim3((e->n_pages + 255) / 256), dim3(256), 0, ctx->stream, e->pages, e->n_pages);
    zhk_xcd_round_robin(ctx);  // (once per context, outside any graph capture: it synchronises)
    // RoPE inverse frequencies: 1/base^(2k/rope_dim) on the host in f32
    // (forward.zig:1495-1500).
    std::vector<float> inv(hd / 2);
    for (uint32_t k = 0; k < hd / 2; k++) inv[k] = 1.0f / powf(c.rope_base, (float)(2 * k) / (float)hd);
    me = hipMemcpyAsync(e->inv_freq, inv.data(), 4ull * hd / 2, hipMemcpyHostToDevice, ctx->stream);
    // the layer table of the persistent decode-layers kernel (addresses only:
    // valid before the weights are written)
    std::vector<zh_step_layer> tab(c.n_layers);
    for (uint32_t l = 0; l < c.n_layers; l++) {
        const Layer &y = e->L[l];
        const uint8_t *A = e->arena;
        tab[l] = zh_step_layer{A + y.wq.off, A + y.wk.off, A + y.wv.off, A + y.wo.off, A + y.gate.off, A + y.up.off,
                               A + y.down.off, (const float *)(A + y.attn_norm.off), (const float *)(A + y.ffn_norm.off),
                               (const float *)(A + y.q_norm.off), (const float *)(A + y.k_norm.off), y.kc, y.vc};
    }
    if (me == hipSuccess)
        me = hipMemcpyAsync(e->step_layers, tab.data(), sizeof(zh_step_layer) * c.n_layers, hipMemcpyHostToDevice,
                            ctx->stream);
    if (me == hipSuccess && zhk_rope_table(ctx, e->inv_freq, c.max_ctx, e->rope_cs) != ZH_OK) me = hipErrorUnknown;
    if (me != hipSuccess || hipStreamSynchronize(ctx->stream) != hipSuccess) {
        zh_engine_destroy(e);
        return zh_set_err(ctx, ZH_ERR_HIP, "engine init");
    }
    *out = e;
    return ZH_OK;
}

extern "C" int zh_engine_create(zh_ctx *ctx, const zh_model_config *cfg, zh_engine **out) {
    return engine_build(ctx, cfg, BuildOpts{}, out);
}

// GGUF tensor name of an engine tensor (llama.cpp's naming, as the
// reference's forward pass looks tensors up: "blk.{l}.attn_q.weight", ...).
static std::string gguf_name(uint64_t stream) {
    if (stream == S_TOKEN_EMBD) return "token_embd.weight";
    if (stream == S_OUTPUT_NORM) return "output_norm.weight";
    if (stream == S_OUTPUT) return "output.weight";
    static const char *kinds[] = {nullptr, "attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "attn_q_norm",
                                  "attn_k_norm", "ffn_norm", "ffn_gate", "ffn_up", "ffn_down", "ffn_gate_inp",
                                  "ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"};
    const uint64_t kind = stream & 0xFF, l = (stream >> 8) - 1;
    if (stream <= 0xFF || kind == 0 || kind > K_EXP_DOWN) return std::string();
    return "blk." + std::to_string(l) + "." + kinds[kind] + ".weight";
}

// loader.load + InferenceEngine.init (loader.zig:414-486, forward.zig:1226):
// the engine's layout with each tensor in the file's storage type, then every
// tensor copied from the mapped file into its slot.
extern "C" int zh_engine_create_gguf(zh_ctx *ctx, const zh_gguf *f, uint32_t max_ctx, zh_engine **out) {
    if (!ctx || !f || !out) return ZH_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    zh_model_config cfg;
    int rc = zh_gguf_model_config(f, max_ctx, &cfg);
    if (rc) return zh_set_err(ctx, rc, "%s", zh_gguf_last_error(f));
    BuildOpts o;
    o.synth = false;
    o.tied_lm = zh_gguf_find_tensor(f, "output.weight") < 0;
    o.type_of = [f](uint64_t stream, uint32_t dflt) {
        const int64_t ti = zh_gguf_find_tensor(f, gguf_name(stream).c_str());
        uint32_t t = dflt;
        if (ti >= 0) zh_gguf_tensor_info(f, (uint64_t)ti, nullptr, nullptr, nullptr, &t, nullptr, nullptr);
        return t;
    };
    zh_engine *e = nullptr;
    ERC(engine_build(ctx, &cfg, o, &e));
    const uint8_t *data = (const uint8_t *)zh_gguf_data(f);
    const uint64_t fsize = zh_gguf_file_size(f), doff = zh_gguf_data_offset(f);
    for (auto &kv : e->tensors) {
        if (kv.first == S_OUTPUT && o.tied_lm) continue;
        const Tensor &t = kv.second;
        const std::string name = gguf_name(kv.first);
        const int64_t ti = zh_gguf_find_tensor(f, name.c_str());
        uint32_t nd = 0, type = 0;
        uint64_t dims[4], off = 0, bytes = 0;
        if (ti < 0) rc = zh_set_err(ctx, ZH_ERR_TENSOR_NOT_FOUND, "%s", name.c_str());
        else zh_gguf_tensor_info(f, (uint64_t)ti, nullptr, &nd, dims, &type, &off, &bytes);
        // ggml order: dims[0] is the contiguous (column) extent; rows are the
        // product of the rest (expert tensors stack n_experts matrices)
        const uint64_t rows = dims[1] * dims[2] * dims[3];
        if (!rc && (type != t.type || dims[0] != t.cols || rows != t.rows || bytes != t.bytes))
            rc = zh_set_err(ctx, ZH_ERR_INVALID_ARGUMENT,
                            "%s: type %u dims [%llu, %llu, %llu] (%llu B), engine expects type %u %llu x %llu", name.c_str(),
                            type, (unsigned long long)dims[0], (unsigned long long)dims[1], (unsigned long long)dims[2],
                            (unsigned long long)bytes, t.type, (unsigned long long)t.rows, (unsigned long long)t.cols);
        if (!rc && (doff + off < doff || doff + off > fsize || bytes > fsize - doff - off))
            rc = zh_set_err(ctx, ZH_ERR_TRUNCATED_FILE, "%s: data [%llu, +%llu) past the end of the file", name.c_str(),
                            (unsigned long long)(doff + off), (unsigned long long)bytes);
        if (!rc && hipMemcpy(e->arena + t.off, data + doff + off, bytes, hipMemcpyHostToDevice) != hipSuccess)
            rc = zh_set_err(ctx, ZH_ERR_HIP, "upload of %s", name.c_str());
        if (rc) {
            zh_engine_destroy(e);
            return rc;
        }
    }
    *out = e;
    return ZH_OK;
}

// InferenceEngine.sample (forward.zig:10360-10367): the greedy token of the
// last step when the params need no logits, else sampleFromLogits on the
// device over the last step's logits.
extern "C" int zh_engine_sample(zh_engine *e, const zh_sampling_params *p, const uint32_t *history, uint32_t nh,
                                double u, uint32_t *token) {
    if (!e || !p || !token) return ZH_ERR_INVALID_ARGUMENT;
    if (!zhk_sampling_requires_readback(p)) return zh_engine_sample_greedy(e, token);
    if (!e->have_logits) return zh_set_err(e->ctx, ZH_ERR_INVALID_ARGUMENT, "sample: no logits (run a step with collect_output)");
    return zhk_sample_host(e->ctx, e->logits, e->c.vocab, p, history, nh, u, token);
}

// A second engine over the weights of `base`, on its own context (stream),
// with its own KV cache, activations and step graph: independent sequences
// decode concurrently on one device, reading one copy of the weights. Both
// contexts are marked concurrent (the attention merge then never waits on
// other workgroups of its grid; base's captured step graphs are dropped and
// re-captured that way). Destroy sharing engines before base.
extern "C" int zh_engine_create_shared(zh_ctx *ctx, zh_engine *base, uint32_t max_ctx, zh_engine **out) {
    if (!ctx || !base || !out) return ZH_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    if (base->ctx->device != ctx->device) return zh_set_err(ctx, ZH_ERR_INVALID_ARGUMENT, "shared engine on another device");
    zh_model_config cfg = base->c;
    if (max_ctx) cfg.max_ctx = (max_ctx + 15) / 16 * 16;
    BuildOpts o;
    o.synth = false;
    o.shared_arena = base->arena;
    o.tied_lm = base->lm.off == base->embd.off;
    o.type_of = [base](uint64_t stream, uint32_t dflt) {
        auto it = base->tensors.find(stream);
        return it == base->tensors.end() ? dflt : it->second.type;
    };
    zh_engine *e = nullptr;
    ERC(engine_build(ctx, &cfg, o, &e));
    for (auto &kv : e->tensors) {  // same layout over the same arena
        auto it = base->tensors.find(kv.first);
        if (it == base->tensors.end() || it->second.off != kv.second.off || it->second.bytes != kv.second.bytes) {
            zh_engine_destroy(e);
            return zh_set_err(ctx, ZH_ERR_INVALID_ARGUMENT, "shared engine layout differs (tensor %llu)",
                              (unsigned long long)kv.first);
        }
    }
    ctx->concurrent = true;
    if (!base->ctx->concurrent) {
        base->ctx->concurrent = true;
        hipStreamSynchronize(base->ctx->stream);
        if (base->g_out) hipGraphExecDestroy(base->g_out);
        if (base->g_noout) hipGraphExecDestroy(base->g_noout);
        base->g_out = base->g_noout = nullptr;
    }
    *out = e;
    return ZH_OK;
}

extern "C" int zh_engine_tensor_type(zh_engine *e, uint64_t stream, uint32_t *type) {
    if (!e || !type) return ZH_ERR_INVALID_ARGUMENT;
    auto it = e->tensors.find(stream);
    if (it == e->tensors.end()) return zh_set_err(e->ctx, ZH_ERR_TENSOR_NOT_FOUND, "stream %llu", (unsigned long long)stream);
    *type = it->second.type;
    return ZH_OK;
}

extern "C" void zh_engine_destroy(zh_engine *e) {
    if (!e) return;
    hipStreamSynchronize(e->ctx->stream);
    auto &xw = e->ctx->xwords;
    for (size_t i = xw.size(); i-- > 0;)
        if (xw[i].owner == e) xw.erase(xw.begin() + i);
    if (e->g_out) hipGraphExecDestroy(e->g_out);
    if (e->g_noout) hipGraphExecDestroy(e->g_noout);
    if (e->arena && e->owns_arena) hipFree(e->arena);
    if (e->kv) hipFree(e->kv);
    if (e->act_arena) hipFree(e->act_arena);
    if (e->pf.arena) hipFree(e->pf.arena);
    if (e->down_pk) hipFree(e->down_pk);
    if (e->force_ids) hipFree(e->force_ids);
    delete e;
}

extern "C" int zh_engine_prefill_kv_random(zh_engine *e, uint32_t n, uint64_t seed) {
    if (!e) return ZH_ERR_INVALID_ARGUMENT;
    if (n > e->c.max_ctx) return zh_set_err(e->ctx, ZH_ERR_CONTEXT_LENGTH_EXCEEDED, "prefill %u > max_ctx", n);
    uint32_t nkv = e->c.n_kv_heads, hd = e->c.head_dim;
    uint64_t total = (uint64_t)n * nkv * hd;
    if (total == 0) return ZH_OK;
    for (uint32_t l = 0; l < e->c.n_layers; l++)
        for (uint32_t w = 0; w < 2; w++) {
            hipLaunchKernelGGL(k_prefill_kv, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, e->ctx->stream,
                               w ? e->L[l].vc : e->L[l].kc, nkv, e->c.max_ctx, hd, n, host_key(seed, S_KV(l, w)),
                               (const uint32_t *)e->pages);
            ZH_LAUNCH_CHECK(e->ctx);
        }
    return ZH_OK;
}

// The sequence's page table: logical 16-token page i of every layer's cache
// lives in physical page pages[i] (logicalTokenToPhysicalToken,
// forward.zig:677-698; the pages come from a KvPagePool, kv_cache.zig:43-125,
// or zh_kv_pool_alloc). n must be max_ctx / 16 and every entry a physical
// page below that; entries need not be distinct for the kernels, but two
// logical pages sharing a physical one overwrite each other's tokens. The
// step graphs are rebuilt: an identity table keeps the attention kernel that
// skips lookups, any other table selects the paged kernel.
extern "C" int zh_engine_set_pages(zh_engine *e, const uint32_t *pages, uint32_t n) {
    if (!e || !pages) return ZH_ERR_INVALID_ARGUMENT;
    if (n != e->n_pages)
        return zh_set_err(e->ctx, ZH_ERR_INVALID_ARGUMENT, "page table of %u entries, the engine has %u pages", n,
                          e->n_pages);
    bool ident = true;
    for (uint32_t i = 0; i < n; i++) {
        if (pages[i] >= e->n_pages)
            return zh_set_err(e->ctx, ZH_ERR_INVALID_ARGUMENT, "page %u of entry %u outside the cache (%u pages)",
                              pages[i], i, e->n_pages);
        ident = ident && pages[i] == i;
    }
    EHIP(e, hipStreamSynchronize(e->ctx->stream));  // no step in flight reads the old table
    EHIP(e, hipMemcpy(e->pages, pages, 4ull * n, hipMemcpyHostToDevice));
    e->pages_ident = ident;
    if (e->g_out) hipGraphExecDestroy(e->g_out);
    if (e->g_noout) hipGraphExecDestroy(e->g_noout);
    e->g_out = e->g_noout = nullptr;
    return ZH_OK;
}

static void drop_graphs(zh_engine *e) {
    if (e->g_out) hipGraphExecDestroy(e->g_out);
    if (e->g_noout) hipGraphExecDestroy(e->g_noout);
    e->g_out = e->g_noout = nullptr;
}

extern "C" int zh_engine_set_fused_attn(zh_engine *e, int on) {
    if (!e) return ZH_ERR_INVALID_ARGUMENT;
    if (e->fused_qa != (on != 0)) {
        ZH_HIP(e->ctx, hipStreamSynchronize(e->ctx->stream));
        drop_graphs(e);
        e->fused_qa = on != 0;
    }
    return ZH_OK;
}

extern "C" int zh_engine_set_fused_ffn(zh_engine *e, int on) {
    if (!e) return ZH_ERR_INVALID_ARGUMENT;
    if (e->fused_ffn != (on != 0)) {
        ZH_HIP(e->ctx, hipStreamSynchronize(e->ctx->stream));
        drop_graphs(e);
        e->fused_ffn = on != 0;
    }
    return ZH_OK;
}

static bool step_moe(zh_engine *e);

// Test hook (no counterpart in the reference): the per-XCD MoE launch runs
// the given experts of each layer (ids [n_layers][n_experts_used], weighted
// by the softmax over their router logits) instead of its own selection,
// which it still records (zh_engine_routing); ids == nullptr switches it off.
// Lets a parity test follow another implementation's routing through near
// ties without the selections drifting apart.
extern "C" int zh_engine_force_routing(zh_engine *e, const uint32_t *ids, uint32_t n) {
    if (!e) return ZH_ERR_INVALID_ARGUMENT;
    const zh_model_config &m = e->c;
    ZH_HIP(e->ctx, hipStreamSynchronize(e->ctx->stream));
    if (!ids) {
        if (e->force_ids) {
            drop_graphs(e);
            hipFree(e->force_ids);
            e->force_ids = nullptr;
        }
        return ZH_OK;
    }
    if (!step_moe(e) || m.n_experts_used != 8 || n != m.n_layers * m.n_experts_used)
        return zh_set_err(e->ctx, ZH_ERR_INVALID_ARGUMENT, "forced routing: the per-XCD MoE launch, %u ids",
                          m.n_layers * m.n_experts_used);
    for (uint32_t i = 0; i < n; i++)
        if (ids[i] >= m.n_experts) return zh_set_err(e->ctx, ZH_ERR_INVALID_ARGUMENT, "expert id %u", ids[i]);
    if (!e->force_ids) {
        if (hipMalloc((void **)&e->force_ids, 4ull * n) != hipSuccess) {
            e->force_ids = nullptr;
            return zh_set_err(e->ctx, ZH_ERR_OUT_OF_MEMORY, "forced routing ids");
        }
        drop_graphs(e);
    }
    ZH_HIP(e->ctx, hipMemcpy(e->force_ids, ids, 4ull * n, hipMemcpyHostToDevice));
    return ZH_OK;
}

extern "C" int zh_engine_set_persistent(zh_engine *e, int on) {
    if (!e) return ZH_ERR_INVALID_ARGUMENT;
    if (e->persistent != (on != 0)) {
        ZH_HIP(e->ctx, hipStreamSynchronize(e->ctx->stream));
        if (e->g_out) hipGraphExecDestroy(e->g_out);
        if (e->g_noout) hipGraphExecDestroy(e->g_noout);
        e->g_out = e->g_noout = nullptr;
        e->persistent = on != 0;
    }
    return ZH_OK;
}

// ---------------------------------------------------------------------------
// Host page pool: KvPagePool (src/scheduler/kv_cache.zig:43-125) -- a stack
// of free page ids (allocation pops from the end, so a fresh pool hands out
// pages in descending order), an owner per page, KvCacheExhausted when too
// few pages are free.
// ---------------------------------------------------------------------------
struct zh_kv_pool {
    std::vector<uint64_t> owner;  // request id + 1 (0: free)
    std::vector<uint32_t> free_list;
    uint32_t page_size = 16;
};
extern "C" int zh_kv_pool_create(uint32_t total_pages, uint32_t page_size, zh_kv_pool **out) {
    if (!out || total_pages == 0 || page_size == 0) return ZH_ERR_INVALID_ARGUMENT;
    zh_kv_pool *p = new zh_kv_pool;
    p->owner.assign(total_pages, 0);
    p->free_list.resize(total_pages);
    for (uint32_t i = 0; i < total_pages; i++) p->free_list[i] = i;
    p->page_size = page_size;
    *out = p;
    return ZH_OK;
}
extern "C" void zh_kv_pool_destroy(zh_kv_pool *p) { delete p; }
extern "C" int zh_kv_pool_alloc(zh_kv_pool *p, uint64_t request_id, uint32_t count, uint32_t *page_ids) {
    if (!p || (count && !page_ids)) return ZH_ERR_INVALID_ARGUMENT;
    if (p->free_list.size() < count) return ZH_ERR_KV_CACHE_EXHAUSTED;
    for (uint32_t i = 0; i < count; i++) {
        const uint32_t id = p->free_list.back();
        p->free_list.pop_back();
        p->owner[id] = request_id + 1;
        page_ids[i] = id;
    }
    return ZH_OK;
}
extern "C" void zh_kv_pool_free(zh_kv_pool *p, uint64_t request_id) {
    if (!p) return;
    for (uint32_t id = 0; id < (uint32_t)p->owner.size(); id++)
        if (p->owner[id] == request_id + 1) {
            p->owner[id] = 0;
            p->free_list.push_back(id);
        }
}
extern "C" uint32_t zh_kv_pool_free_count(const zh_kv_pool *p) { return p ? (uint32_t)p->free_list.size() : 0u; }
extern "C" uint32_t zh_kv_pool_max_context(const zh_kv_pool *p, uint32_t page_count) {
    return p ? page_count * p->page_size : 0u;
}

// ---------------------------------------------------------------------------
// One token step (the body of decodeStep, forward.zig:4376-7754).
// ---------------------------------------------------------------------------
// output_norm -> LM head -> greedy argmax on e->hidden (forward.zig:7757-7772,
// sampleGreedy :10338-10357); the token goes to ST_TOKEN_OUT and the ring.
// advance: the whole step's tail (the argmax and the step advance in one
// launch, k_argmax_advance); else the argmax alone.
static int record_collect(zh_engine *e, bool advance = false) {
    zh_ctx *c = e->ctx;
    const zh_model_config &m = e->c;
    const uint32_t H = m.hidden;
    const uint8_t *A = e->arena;
    if (!zh_knob("ZH_NO_LPB") && zhk_lpb_supported(e->lm.type, H) && m.vocab % 2 == 0) {
        const uint8_t *wl = A + e->lm.off;
        float *yl = e->logits;
        const uint32_t mv = m.vocab;
        ERC(zhk_dmmv_lpb(c, e->lm.type, 0, 1, &wl, nullptr, &yl, &mv, e->hidden,
                         (const float *)(A + e->out_norm.off), m.eps, nullptr, H, 0));
    } else {
        ERC(zhk_rms_norm(c, e->hidden, (const float *)(A + e->out_norm.off), H, e->norm, e->xq_h, H, 1, m.eps));
        ERC(zhk_dmmv(c, e->lm.type, A + e->lm.off, e->xq_h, e->logits, m.vocab, H, 0));
    }
    if (advance) {
        hipLaunchKernelGGL(k_argmax_advance, dim3(TAIL_WGS), dim3(256), 0, c->stream, e->logits, m.vocab, e->am_part,
                           e->am_cnt, e->ring, e->st, (const uint32_t *)e->prompt);
        ZH_LAUNCH_CHECK(c);
        return ZH_OK;
    }
    return zhk_argmax(c, e->logits, m.vocab, e->st + ST_TOKEN_OUT, e->am_part, e->ring, e->st + ST_GEN);
}

// Launch groups of one layer (the unit zh_engine_time_kernel replays).
enum : uint32_t { SK_QKV = 1, SK_ATTN = 2, SK_O = 4, SK_FFN_IN = 8, SK_FFN_OUT = 16, SK_ALL = 31, SK_HEAD = 32 };

// The persistent decode-layers kernel's arguments for the whole step, and
// whether it takes this engine's model (dense, every layer in the formats it
// is built for, no engine sharing the device).
static bool step_args(zh_engine *e, zh_step_args &a) {
    const zh_model_config &m = e->c;
    a = zh_step_args{};
    a.layers = e->step_layers;
    a.l0 = 0;
    a.l1 = m.n_layers;
    a.hidden = m.hidden; a.n_heads = m.n_heads; a.n_kv_heads = m.n_kv_heads; a.ffn = m.ffn; a.max_ctx = m.max_ctx;
    a.eps = m.eps; a.scale = 1.0f / sqrtf((float)m.head_dim);
    a.x = e->hidden; a.q = e->q; a.k = e->k; a.v = e->v; a.attn = e->attn; a.s = e->s;
    a.xq_attn = e->xq_q; a.xq_s = e->xq_f; a.grp_cnt = e->grp_cnt;
    a.rope_cs = e->rope_cs; a.pages = e->pages; a.n_pages = e->n_pages; a.ident = e->pages_ident ? 1u : 0u;
    a.pos = zh_pos_src{0, e->st + ST_POS};
    a.part = e->fd_part;
    a.ctl = e->step_ctl;
    if (!e->persistent || m.n_experts || !zhk_step_supported(e->ctx, a)) return false;
    for (const Layer &y : e->L) {
        const Tensor *q4[] = {&y.wq, &y.wk, &y.wv, &y.wo, &y.gate, &y.up};
        for (const Tensor *t : q4)
            if (t->type != ZH_Q4_K || t->off % 16) return false;
        if (y.down.type != ZH_Q6_K || y.down.off % 16) return false;
    }
    return true;
}

// Whether a layer's Q/K/V and attention run as one launch (k_qkv_attn).
static bool layer_qa(zh_engine *e, const Layer &y) {
    const zh_model_config &m = e->c;
    const uint32_t H = m.hidden, qd = m.n_heads * m.head_dim;
    // hidden 4096: Q4_K Q/K/V (and an O projection the tile kernels take);
    // hidden 2048: Q8_0 Q/K/V
    const uint32_t qt = H == 2048 ? ZH_Q8_0 : ZH_Q4_K;
    return e->fused_qa && e->pages_ident && !zh_knob("ZH_NO_LPB") && y.wq.type == qt && y.wk.type == qt &&
           y.wv.type == qt && (H == 2048 || zhk_lpb_supported(y.wo.type, qd)) &&
           zhk_qkv_attn_supported(e->ctx, H, m.n_heads, m.n_kv_heads, m.head_dim, m.max_ctx);
}

static bool step_moe(zh_engine *e);

// Whether every layer's O projection also runs in that launch: then the
// residual stream is kept twice at layer entry (the embedding and every down
// projection write e->xin beside e->hidden), the launch reads its input from
// e->xin and adds the O projection into e->hidden with device atomics.
static bool step_qa_o(zh_engine *e) {
    const zh_model_config &m = e->c;
    if (m.n_experts) {  // hidden 2048, Q8_0 O: only with the MoE FFN launch (the split residual)
        if (!step_moe(e)) return false;
        for (const Layer &y : e->L)
            if (!layer_qa(e, y) || y.wo.type != ZH_Q8_0 || y.wo.off % 16) return false;
        return true;
    }
    if (m.n_heads != 4 * m.n_kv_heads) return false;
    for (const Layer &y : e->L)
        if (!layer_qa(e, y) || y.wo.type != ZH_Q4_K || y.gate.type != ZH_Q4_K || y.up.type != ZH_Q4_K ||
            y.down.type != ZH_Q6_K || !zhk_lpb_supported(ZH_Q6_K, m.ffn))
            return false;
    return true;
}

// Whether the dense FFN also runs as one per-XCD launch (k_ffn_xcd): then
// both launches of a layer take the split residual. Launch k of the step
// (attention 2l, FFN 2l + 1) reads rres[k % 2] + dres[k % 3], writes their
// sum into rres[(k + 1) % 2], adds its projection into dres[(k + 1) % 3] with
// device atomics and zeroes dres[(k + 2) % 3] (last read by launch k - 1,
// next added into by launch k + 1). The step starts from the embedding in
// rres[0] and dres all zero; k_fold_residual leaves the sum in e->hidden and
// dres zero again. dres is 64-bit fixed point (zh_xcd.h fix_add): its sums do
// not depend on the order of the atomics, so the step is deterministic.
static bool step_xcd(zh_engine *e) {
    return e->fused_ffn && !zh_knob("ZH_NO_FFN_XCD") && zhk_ffn_xcd_supported(e->ctx, e->c.hidden, e->c.ffn) &&
           step_qa_o(e);
}

// Whether every layer's MoE FFN runs as one per-XCD launch (k_moe_xcd): the
// O projection then also writes the residual into e->xin, which the launch
// reads while it adds into e->hidden.
static bool step_moe(zh_engine *e) {
    const zh_model_config &m = e->c;
    if (!e->fused_ffn || zh_knob("ZH_NO_MOE_XCD") || zh_knob("ZH_NO_LDS_DMMV") || m.n_experts == 0 ||
        !zhk_moe_xcd_supported(e->ctx, m.hidden, m.n_experts, m.n_experts_used, m.expert_ffn))
        return false;
    const uint32_t qd = m.n_heads * m.head_dim;
    for (const Layer &y : e->L)
        if (y.router.type != ZH_Q8_0 || y.egate.type != ZH_Q4_K || y.eup.type != ZH_Q4_K || y.edown.type != ZH_Q4_K ||
            y.ffn_norm.off % 16 || y.router.off % 16 || y.egate.off % 16 || y.eup.off % 16 ||
            (!zh_knob("ZH_NO_LPB") && zhk_lpb_supported(y.wo.type, qd)))
            return false;
    return true;
}

// The per-XCD FFN launch's packed copy of every layer's ffn_down: allocated
// on first use, rewritten from the arena when it may have changed (outside
// any capture).
static int ensure_packed(zh_engine *e) {
    if (!step_xcd(e)) return ZH_OK;
    const uint64_t per = zhk_ffn_pack_bytes();
    if (!e->down_pk && hipMalloc((void **)&e->down_pk, per * e->c.n_layers) != hipSuccess) {
        e->down_pk = nullptr;
        return zh_set_err(e->ctx, ZH_ERR_OUT_OF_MEMORY, "packed ffn_down (%llu B)",
                          (unsigned long long)(per * e->c.n_layers));
    }
    if (e->pk_stale) {
        for (uint32_t l = 0; l < e->c.n_layers; l++)
            ERC(zhk_ffn_pack_down(e->ctx, e->arena + e->L[l].down.off, e->down_pk + per * l));
        e->pk_stale = false;
    }
    return ZH_OK;
}

__global__ void k_fold_residual(float *hidden, const float *r, zh_fix *d, uint32_t kd, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    hidden[i] = r[i] + fix_to_f(d[kd * n + i]);
    d[i] = 0;
    d[n + i] = 0;
    d[2 * n + i] = 0;
}

// Records the decode step: embedding, layers [l0, l1) (only the launch
// groups in `mask`), then (whole steps only) the output head and the step
// advance.
static int record_step(zh_engine *e, bool collect, uint32_t l0 = 0, uint32_t l1 = ~0u, uint32_t mask = SK_ALL) {
    zh_ctx *c = e->ctx;
    const zh_model_config &m = e->c;
    const uint32_t H = m.hidden, hd = m.head_dim, qd = m.n_heads * hd, kvd = m.n_kv_heads * hd;
    const uint8_t *A = e->arena;
    auto W = [&](const Tensor &t) { return A + t.off; };
    auto Wf = [&](const Tensor &t) { return (const float *)(A + t.off); };
    zh_pos_src pos{0, e->st + ST_POS}, seq{1, e->st + ST_POS};
    const float scale = 1.0f / sqrtf((float)hd);
    const bool whole = mask == SK_ALL && l0 == 0 && l1 >= m.n_layers;
    const bool lpb = !zh_knob("ZH_NO_LPB");
    // LDS-staged kernels with the norms, router top-k and expert combine fused
    const bool lds = !zh_knob("ZH_NO_LDS_DMMV");
    // the whole step's layers in one persistent launch when it takes the model
    zh_step_args sa;
    const bool persistent = whole && step_args(e, sa);
    const bool qa_o = !persistent && step_qa_o(e);
    const bool xl = qa_o && (m.n_experts ? true : step_xcd(e));  // qa_o with MoE implies its FFN launch
    const bool moe_x = !persistent && step_moe(e);
    zh_fix *const D = e->dres;
    auto dr = [&](uint32_t k) { return D + (size_t)(k % 3) * H; };
    // embedToken (forward.zig:4255-4290), on the device.
    if (whole) {
        ERC(zhk_dequant_rows(c, e->embd.type, W(e->embd), 0, 1, H, xl ? e->rres : e->hidden, e->st + ST_TOKEN_IN,
                             m.vocab));
        if (qa_o && !xl)
            ERC(zhk_dequant_rows(c, e->embd.type, W(e->embd), 0, 1, H, e->xin, e->st + ST_TOKEN_IN, m.vocab));
    }
    if (persistent) ERC(zhk_step_layers(c, sa));
    for (uint32_t l = persistent ? m.n_layers : l0; l < m.n_layers && l < l1; l++) {
        const Layer &y = e->L[l];
        uint32_t *const rt = e->routing + (size_t)ZH_ROUTE_WORDS * l;  // this layer's selection
        // kernel choice per layer, from the layer's own tensor types (a GGUF
        // Q4_K_M file mixes Q4_K and Q6_K attn_v / ffn_down across layers)
        const bool lpb_attn = lpb && zhk_lpb_supported(y.wq.type, H) && zhk_lpb_supported(y.wk.type, H) &&
                              zhk_lpb_supported(y.wv.type, H) && zhk_lpb_supported(y.wo.type, qd) && qd % 2 == 0 &&
                              kvd % 2 == 0;
        const bool lpb_ffn = lpb && m.n_experts == 0 && y.gate.type == ZH_Q4_K && y.up.type == ZH_Q4_K &&
                             zhk_lpb_supported(ZH_Q4_K, H) && zhk_lpb_supported(y.down.type, m.ffn);
        const bool lds_moe = lds && m.n_experts && m.n_experts <= 256 && m.n_experts_used <= 8 &&
                             (y.router.type == ZH_F32 || zhk_dmmv_lds_supported(y.router.type, H)) &&
                             zhk_dmmv_lds_supported(y.edown.type, m.expert_ffn) && m.expert_ffn % 32 == 0;
        // Q, K and V: one launch per run of equal types (one launch when all agree)
        const Tensor *qkv_t[3] = {&y.wq, &y.wk, &y.wv};
        float *qkv_y[3] = {e->q, e->k, e->v};
        const uint32_t qkv_m[3] = {qd, kvd, kvd};
        // Q/K/V and attention in one launch: 8 kv heads, one per XCD
        // (and the O projection, qa_o, when the launch group includes it)
        const bool qa = (mask & SK_QKV) && (mask & SK_ATTN) && layer_qa(e, y);
        const bool with_o = qa && qa_o && (mask & SK_O);
        const uint32_t ka = 2 * l;  // the split residual's launch index (xl)
        if (qa && with_o && xl) {
            ERC(zhk_qkv_attn(c, W(y.wq), W(y.wk), W(y.wv), e->rres, Wf(y.attn_norm), e->q, e->k, e->v,
                             Wf(y.q_norm), Wf(y.k_norm), e->rope_cs, y.kc, y.vc, m.max_ctx, e->attn, e->xq_q,
                             m.n_heads, pos, scale, m.eps, e->fd_part, e->qa_flags, W(y.wo), dr(ka + 1), dr(ka),
                             e->rres + H, dr(ka + 2), H, e->qa_xrows));
        } else if (qa) {
            ERC(zhk_qkv_attn(c, W(y.wq), W(y.wk), W(y.wv), qa_o ? e->xin : e->hidden, Wf(y.attn_norm), e->q, e->k,
                             e->v, Wf(y.q_norm), Wf(y.k_norm), e->rope_cs, y.kc, y.vc, m.max_ctx, e->attn, e->xq_q,
                             m.n_heads, pos, scale, m.eps, e->fd_part, e->qa_flags, with_o ? W(y.wo) : nullptr,
                             with_o ? e->hidden : nullptr, nullptr, nullptr, nullptr, H, e->qa_xrows));
        } else if (!(mask & SK_QKV)) {
        } else if (lpb_attn) {
            // attn_norm fused into the Q/K/V mat-vec (every workgroup normalises x)
            for (uint32_t i0 = 0; i0 < 3;) {
                uint32_t i1 = i0 + 1;
                while (i1 < 3 && qkv_t[i1]->type == qkv_t[i0]->type) i1++;
                const uint8_t *ws[3];
                for (uint32_t i = i0; i < i1; i++) ws[i - i0] = W(*qkv_t[i]);
                ERC(zhk_dmmv_lpb(c, qkv_t[i0]->type, 0, i1 - i0, ws, nullptr, qkv_y + i0, qkv_m + i0, e->hidden,
                                 Wf(y.attn_norm), m.eps, nullptr, H, 0));
                i0 = i1;
            }
        } else if (lds && qkv_t[0]->type == qkv_t[1]->type && qkv_t[1]->type == qkv_t[2]->type &&
                   zhk_dmmv_lds_supported(y.wq.type, H) && qkv_m[0] % 2 == 0 && qkv_m[1] % 2 == 0) {
            // formats without a tile kernel (Q8_0, MXFP4): attn_norm fused into
            // the LDS-staged mat-vec of the three stacked matrices
            const uint8_t *ws[3] = {W(y.wq), W(y.wk), W(y.wv)};
            ERC(zhk_dmmv_lds_plain(c, y.wq.type, 3, ws, qkv_y, qkv_m, e->hidden, Wf(y.attn_norm), m.eps, H, 0,
                                   nullptr, 0, nullptr, nullptr));
        } else {
            ERC(zhk_rms_norm(c, e->hidden, Wf(y.attn_norm), H, e->norm, e->xq_h, H, 1, m.eps));
            for (uint32_t i0 = 0; i0 < 3;) {
                uint32_t i1 = i0 + 1;
                while (i1 < 3 && qkv_t[i1]->type == qkv_t[i0]->type) i1++;
                const uint8_t *ws[3];
                for (uint32_t i = i0; i < i1; i++) ws[i - i0] = W(*qkv_t[i]);
                ERC(zhk_dmmv_multi(c, qkv_t[i0]->type, i1 - i0, ws, qkv_y + i0, qkv_m + i0, e->xq_h, H));
                i0 = i1;
            }
        }
        if ((mask & SK_ATTN) && !qa)
            ERC(zhk_attn_decode_fused(c, e->q, e->k, e->v, Wf(y.q_norm), Wf(y.k_norm), e->rope_cs, y.kc, y.vc,
                                  e->pages, e->n_pages, m.max_ctx, e->attn, e->xq_q, m.n_heads, m.n_kv_heads, pos,
                                  m.max_ctx, scale, m.eps, e->fd_part, e->pages_ident));
        if (!(mask & SK_O) || with_o) {
        } else if (lpb_attn) {
            // the merge kernel already emitted the attention output as XQ
            const uint8_t *wo = W(y.wo);
            float *yo = e->hidden;
            const uint32_t mo = H;
            ERC(zhk_dmmv_lpb(c, y.wo.type, 0, 1, &wo, nullptr, &yo, &mo, nullptr, nullptr, 0.f, nullptr, qd, 1,
                             e->xq_q));
        } else {
            ERC(zhk_dmmv(c, y.wo.type, W(y.wo), e->xq_q, e->hidden, H, qd, 1, moe_x ? e->xin : nullptr));
        }
        if (lpb_ffn && xl && (mask & SK_FFN_IN) && (mask & SK_FFN_OUT)) {
            // ffn_norm, gate/up + SwiGLU and down in one launch, split by XCD
            ERC(zhk_ffn_xcd(c, e->rres + H, dr(ka + 1), Wf(y.ffn_norm), m.eps, W(y.gate), W(y.up),
                            e->down_pk + zhk_ffn_pack_bytes() * l, e->ffn_part, e->rres, dr(ka + 2), dr(ka + 3),
                            e->ffn_flags));
            continue;
        }
        if (lpb_ffn) {
            // ffn_norm fused into gate/up; SwiGLU fused into its epilogue
            const uint8_t *wg = W(y.gate);
            float *ys = e->s;
            const uint32_t mf = m.ffn;
            // gate/up also emits its output as XQ (quantised per 32-row group by
            // the group's last batch), so the down projection copies XQ instead of
            // every workgroup re-quantising the f32 vector
            const bool swiglu_xq = m.ffn % 32 == 0 && H / 256 <= 32 && !zh_knob("ZH_NO_TILE");
            if (mask & SK_FFN_IN)
                ERC(zhk_dmmv_lpb(c, ZH_Q4_K, 1, 1, &wg, W(y.up), &ys, &mf, e->hidden, Wf(y.ffn_norm), m.eps, nullptr,
                                 H, 0, nullptr, swiglu_xq ? e->xq_f : nullptr, swiglu_xq ? e->grp_cnt : nullptr));
            const uint8_t *wd = W(y.down);
            float *yd = e->hidden;
            const uint32_t mh = H;
            if (mask & SK_FFN_OUT)
                ERC(zhk_dmmv_lpb(c, y.down.type, 0, 1, &wd, nullptr, &yd, &mh, swiglu_xq ? nullptr : e->s,
                                 nullptr, 0.f, nullptr, m.ffn, 1, swiglu_xq ? e->xq_f : nullptr, nullptr, nullptr,
                                 qa_o ? e->xin : nullptr));
            continue;
        }
        if (moe_x && (mask & SK_FFN_IN) && (mask & SK_FFN_OUT)) {
            // ffn_norm, router, top-k, the selected experts and the weighted
            // sum in one launch, one expert per XCD
            // (split residual when the attention launch takes the O projection)
            if (xl)
                ERC(zhk_moe_xcd(c, e->rres + H, Wf(y.ffn_norm), m.eps, W(y.router), W(y.egate), W(y.eup),
                                W(y.edown), dr(ka + 2), e->moe_scratch, rt,
                                e->moe_flags, dr(ka + 1), e->rres, dr(ka + 3),
                                e->force_ids ? e->force_ids + (size_t)m.n_experts_used * l : nullptr));
            else
                ERC(zhk_moe_xcd(c, e->xin, Wf(y.ffn_norm), m.eps, W(y.router), W(y.egate), W(y.eup),
                                W(y.edown), e->hidden, e->moe_scratch, rt,
                                e->moe_flags, nullptr, nullptr, nullptr,
                                e->force_ids ? e->force_ids + (size_t)m.n_experts_used * l : nullptr));
            continue;
        }
        if (lds_moe) {
            // ffn_norm + router + top-k in one launch (it also leaves the
            // normed activation as XQ for the experts); experts gate/up +
            // SwiGLU; their outputs as XQ; then the selected down projections
            // with the weighted sum added to the residual
            const uint32_t F = m.expert_ffn, k = m.n_experts_used, E = m.n_experts;
            const uint8_t *wr = W(y.router);
            float *rl = e->rl;
            if (mask & SK_FFN_IN) {
                if (y.router.type == ZH_F32) {
                    // an f32 router: ffn_norm (also leaving the XQ activation
                    // for the experts), the f32 mat-vec, then top-k
                    ERC(zhk_rms_norm(c, e->hidden, Wf(y.ffn_norm), H, e->norm, e->xq_h, H, 1, m.eps));
                    ERC(zhk_matvec_f32(c, Wf(y.router), e->norm, e->rl, E, H));
                    ERC(zhk_softmax_topk(c, e->rl, E, k, rt));
                } else {
                    ERC(zhk_dmmv_lds_plain(c, y.router.type, 1, &wr, &rl, &E, e->hidden, Wf(y.ffn_norm), m.eps, H, 0,
                                           e->xq_h, k, rt, e->router_cnt));
                }
                ERC(zhk_dmmv_moe(c, y.egate.type, W(y.egate), zh_tensor_bytes(y.egate.type, F, H),
                                 rt, e->xq_h, 0, e->s, F, H, k, 1, W(y.eup), m.n_experts));
            }
            if (mask & SK_FFN_OUT) {
                ERC(zhk_quantize_xq(c, e->s, e->xq_f, F, k, F));
                ERC(zhk_dmmv_lds_down_acc(c, y.edown.type, W(y.edown), zh_tensor_bytes(y.edown.type, H, F),
                                          rt, k, m.n_experts, e->xq_f, e->hidden, H, F));
            }
            continue;
        }
        if (!(mask & SK_FFN_IN) || !(mask & SK_FFN_OUT)) continue;  // not split: timed as whole steps only
        ERC(zhk_rms_norm(c, e->hidden, Wf(y.ffn_norm), H, e->norm, e->xq_h, H, 1, m.eps));
        if (m.n_experts == 0) {
            if (y.gate.type == y.up.type) {
                ERC(zhk_dmmv_gate_up(c, y.gate.type, W(y.gate), W(y.up), e->xq_h, e->s, m.ffn, H));
            } else {  // gate and up in different formats: two mat-vecs, then SwiGLU
                const uint32_t F = m.ffn;
                ERC(zhk_dmmv(c, y.gate.type, W(y.gate), e->xq_h, e->s, F, H, 0));
                ERC(zhk_dmmv(c, y.up.type, W(y.up), e->xq_h, e->u, F, H, 0));
                ERC(zhk_swiglu(c, e->s, e->u, e->s, F));
            }
            ERC(zhk_quantize_xq(c, e->s, e->xq_f, m.ffn, 1, 0));
            ERC(zhk_dmmv(c, y.down.type, W(y.down), e->xq_f, e->hidden, H, m.ffn, 1));
        } else {
            const uint32_t F = m.expert_ffn, k = m.n_experts_used;
            if (y.router.type == ZH_F32) ERC(zhk_matvec_f32(c, Wf(y.router), e->norm, e->rl, m.n_experts, H));
            else ERC(zhk_dmmv(c, y.router.type, W(y.router), e->xq_h, e->rl, m.n_experts, H, 0));
            ERC(zhk_softmax_topk(c, e->rl, m.n_experts, k, rt));
            ERC(zhk_dmmv_moe(c, y.egate.type, W(y.egate), zh_tensor_bytes(y.egate.type, F, H), rt,
                             e->xq_h, 0, e->s, F, H, k, 1, W(y.eup), m.n_experts));
            ERC(zhk_quantize_xq(c, e->s, e->xq_f, F, k, F));
            ERC(zhk_dmmv_moe(c, y.edown.type, W(y.edown), zh_tensor_bytes(y.edown.type, H, F), rt,
                             e->xq_f, zh_xq_bytes_int(F), e->edown_out, H, F, k, 0, nullptr, m.n_experts));
            ERC(zhk_moe_weighted_acc(c, e->hidden, e->edown_out, rt, H, k, H));
        }
    }
    if (!whole) return ZH_OK;
    if (xl) {
        hipLaunchKernelGGL(k_fold_residual, dim3((H + 255) / 256), dim3(256), 0, c->stream, e->hidden, e->rres,
                           e->dres, (2 * m.n_layers) % 3, H);
        ZH_LAUNCH_CHECK(c);
    }
    if (collect) return record_collect(e, true);  // (with the step advance)
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(1), 0, c->stream, e->st, (const uint32_t *)e->prompt);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

// Measurement entry (no counterpart in the reference): the kernels one
// launch group of layer 0 launches, read from the graph the group's launches
// capture into (each kernel node's function, named by the runtime), joined
// with "; " into names (at most len bytes, NUL-terminated).
extern "C" int zh_engine_group_kernels(zh_engine *e, uint32_t group, char *names, size_t len) {
    if (!e || !names || len == 0 || group == 0 || (group != SK_HEAD && (group & ~(uint32_t)SK_ALL)))
        return ZH_ERR_INVALID_ARGUMENT;
    zh_ctx *c = e->ctx;
    ERC(ensure_packed(e));
    hipGraph_t g = nullptr;
    EHIP(e, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    int rc = group == SK_HEAD ? record_collect(e) : record_step(e, false, 0, 1, group);
    const hipError_t ce = hipStreamEndCapture(c->stream, &g);
    if (rc) return rc;
    if (ce != hipSuccess) return zh_set_err(c, ZH_ERR_HIP, "capture: %s", hipGetErrorString(ce));
    size_t n = 0;
    std::string out;
    if (hipGraphGetNodes(g, nullptr, &n) == hipSuccess && n) {
        std::vector<hipGraphNode_t> nodes(n);
        if (hipGraphGetNodes(g, nodes.data(), &n) == hipSuccess) {
            // capture order: a node's position in the chain of dependencies
            for (size_t i = 0; i < n; i++) {
                hipGraphNodeType t;
                hipKernelNodeParams kp;
                if (hipGraphNodeGetType(nodes[i], &t) != hipSuccess || t != hipGraphNodeTypeKernel) continue;
                if (hipGraphKernelNodeGetParams(nodes[i], &kp) != hipSuccess) continue;
                hipFunction_t f = nullptr;
                const char *nm = hipGetFuncBySymbol(&f, kp.func) == hipSuccess && f ? hipKernelNameRef(f) : nullptr;
                if (!nm) nm = hipKernelNameRefByPtr(kp.func, c->stream);
                if (!out.empty()) out += "; ";
                out += nm ? nm : "?";
            }
        }
    }
    hipGraphDestroy(g);
    (void)hipGetLastError();  // a name lookup that failed is reported as "?", not by the next launch check
    snprintf(names, len, "%s", out.c_str());
    return ZH_OK;
}


// Measurement entry (no counterpart in the reference; the benchmark uses it
// for per-kernel bandwidth): the average duration of one launch group --
// exactly the launches, arguments and state of the decode step -- over
// `iters` launches rotating through the layers (so weights stream from HBM),
// timed with HIP events on the engine's stream. Activations are left changed.
extern "C" int zh_engine_time_kernel(zh_engine *e, uint32_t group, uint32_t iters, float *us_per_launch) {
    const bool head = group == SK_HEAD;  // output norm + LM head + argmax (one launch group, not per layer)
    if (!e || !us_per_launch || group == 0 || (!head && (group & ~(uint32_t)SK_ALL)) || iters == 0)
        return e ? zh_set_err(e->ctx, ZH_ERR_INVALID_ARGUMENT, "time_kernel group %u", group) : ZH_ERR_INVALID_ARGUMENT;
    zh_ctx *c = e->ctx;
    const uint32_t L = e->c.n_layers;
    auto launch = [&](uint32_t i) { return head ? record_collect(e) : record_step(e, false, i % L, i % L + 1, group); };
    ERC(ensure_packed(e));
    for (uint32_t l = 0; l < (head ? 1u : L); l++) ERC(launch(l));
    hipEvent_t ev[2];
    EHIP(e, hipEventCreate(&ev[0]));
    if (hipEventCreate(&ev[1]) != hipSuccess) {
        hipEventDestroy(ev[0]);
        return zh_set_err(c, ZH_ERR_HIP, "event");
    }
    int rc = hipEventRecord(ev[0], c->stream) == hipSuccess ? ZH_OK : ZH_ERR_HIP;
    for (uint32_t i = 0; rc == ZH_OK && i < iters; i++) rc = launch(i);
    float ms = 0.f;
    if (rc == ZH_OK && (hipEventRecord(ev[1], c->stream) != hipSuccess || hipEventSynchronize(ev[1]) != hipSuccess ||
                        hipEventElapsedTime(&ms, ev[0], ev[1]) != hipSuccess))
        rc = zh_set_err(c, ZH_ERR_HIP, "time_kernel events");
    hipEventDestroy(ev[0]);
    hipEventDestroy(ev[1]);
    if (rc == ZH_OK) *us_per_launch = ms * 1e3f / (float)iters;
    // the replays leave atomic sums in the split residual's dres, which a
    // decode step expects zero
    if (rc == ZH_OK && hipMemsetAsync(e->dres, 0, 24ull * e->c.hidden, c->stream) != hipSuccess)
        rc = zh_set_err(c, ZH_ERR_HIP, "time_kernel reset");
    return rc;
}

static int ensure_graphs(zh_engine *e) {
    if (e->g_out && e->g_noout) return ZH_OK;
    zh_ctx *c = e->ctx;
    for (int collect = 0; collect < 2; collect++) {
        hipGraph_t g;
        EHIP(e, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        int rc = record_step(e, collect != 0);
        hipError_t ce = hipStreamEndCapture(c->stream, &g);
        if (rc) return rc;
        if (ce != hipSuccess) return zh_set_err(c, ZH_ERR_HIP, "capture: %s", hipGetErrorString(ce));
        hipGraphExec_t x;
        ce = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
        hipGraphDestroy(g);
        if (ce != hipSuccess) return zh_set_err(c, ZH_ERR_HIP, "instantiate: %s", hipGetErrorString(ce));
        (collect ? e->g_out : e->g_noout) = x;
    }
    return ZH_OK;
}

static int set_state(zh_engine *e, uint32_t n_prompt, uint32_t pos, uint32_t first_token) {
    uint32_t st[ST_WORDS] = {0};
    st[ST_STEP] = 0;
    st[ST_NPROMPT] = n_prompt;
    st[ST_POS] = pos;
    st[ST_TOKEN_IN] = first_token;
    st[ST_GEN] = 0;
    EHIP(e, hipMemcpyAsync(e->st, st, sizeof st, hipMemcpyHostToDevice, e->ctx->stream));
    return ZH_OK;
}

static int run_step(zh_engine *e, bool collect) {
    if (e->place_gen != e->ctx->place_gen) {
        // a bounded wait gave up since the graphs were recorded and zh_sync
        // checked the placement again: record the step anew (with the
        // per-group launches if the check failed)
        if (e->g_out) hipGraphExecDestroy(e->g_out);
        if (e->g_noout) hipGraphExecDestroy(e->g_noout);
        e->g_out = e->g_noout = nullptr;
        e->place_gen = e->ctx->place_gen;
    }
    ERC(ensure_packed(e));
    if (zh_knob("ZH_NO_GRAPH")) return record_step(e, collect);
    ERC(ensure_graphs(e));
    EHIP(e, hipGraphLaunch(collect ? e->g_out : e->g_noout, e->ctx->stream));
    return ZH_OK;
}

extern "C" int zh_engine_decode_step(zh_engine *e, uint32_t token, uint32_t position, int collect) {
    if (!e) return ZH_ERR_INVALID_ARGUMENT;
    if (position >= e->c.max_ctx)
        return zh_set_err(e->ctx, ZH_ERR_CONTEXT_LENGTH_EXCEEDED, "position %u >= %u", position, e->c.max_ctx);
    ERC(set_state(e, 1, position, token));
    ERC(run_step(e, collect != 0));
    if (collect) e->have_logits = true;
    return ZH_OK;
}

extern "C" int zh_engine_sample_greedy(zh_engine *e, uint32_t *token) {
    if (!e || !token) return ZH_ERR_INVALID_ARGUMENT;
    EHIP(e, hipMemcpyAsync(token, e->st + ST_TOKEN_OUT, 4, hipMemcpyDeviceToHost, e->ctx->stream));
    EHIP(e, hipStreamSynchronize(e->ctx->stream));
    return ZH_OK;
}

// ---------------------------------------------------------------------------
// Batched decode: n engines sharing one copy of the weights (zh_engine_create_
// shared on one context) step in lockstep, one token each per step. The
// projections and the LM head run as batched DMMV launches (the weights
// stream once for all sequences, recordBatchDispatchPush dmmv.zig:880-925);
// embedding, attention over each sequence's own KV cache, argmax and the step
// advance stay per sequence. The scheduler's decode batch
// (src/scheduler/scheduler.zig activeDecoding) on one weight stream.
// ---------------------------------------------------------------------------
static bool batch_layer_ok(const zh_engine *e, const Layer &y) {
    const zh_model_config &m = e->c;
    const uint32_t H = m.hidden, qd = m.n_heads * m.head_dim;
    auto kq = [](const Tensor &t) { return t.type == ZH_Q4_K || t.type == ZH_Q6_K; };
    return kq(y.wq) && kq(y.wk) && kq(y.wv) && kq(y.wo) && y.gate.type == ZH_Q4_K && y.up.type == ZH_Q4_K &&
           kq(y.down) && zhk_lpb_supported(y.wq.type, H) && zhk_lpb_supported(y.wk.type, H) &&
           zhk_lpb_supported(y.wv.type, H) && zhk_lpb_supported(y.wo.type, qd) && zhk_lpb_supported(ZH_Q4_K, H) &&
           zhk_lpb_supported(y.down.type, m.ffn);
}

static int record_step_batch(zh_engine *const *es, uint32_t n, bool collect) {
    zh_engine *e0 = es[0];
    zh_ctx *c = e0->ctx;
    const zh_model_config &m = e0->c;
    const uint32_t H = m.hidden, hd = m.head_dim, qd = m.n_heads * hd, kvd = m.n_kv_heads * hd;
    const uint8_t *A = e0->arena;
    auto W = [&](const Tensor &t) { return A + t.off; };
    auto Wf = [&](const Tensor &t) { return (const float *)(A + t.off); };
    const float scale = 1.0f / sqrtf((float)hd);
    std::vector<const float *> xs(n);
    std::vector<const void *> xqs(n);
    std::vector<float *> ys(3 * n);
    for (uint32_t v = 0; v < n; v++)
        ERC(zhk_dequant_rows(c, e0->embd.type, W(e0->embd), 0, 1, H, es[v]->hidden, es[v]->st + ST_TOKEN_IN, m.vocab));
    for (uint32_t l = 0; l < m.n_layers; l++) {
        const Layer &y = e0->L[l];
        // Q, K, V (attn_norm fused): one batched launch per run of equal types
        const Tensor *qkv_t[3] = {&y.wq, &y.wk, &y.wv};
        const uint32_t qkv_m[3] = {qd, kvd, kvd};
        for (uint32_t i0 = 0; i0 < 3;) {
            uint32_t i1 = i0 + 1;
            while (i1 < 3 && qkv_t[i1]->type == qkv_t[i0]->type) i1++;
            const uint8_t *ws[3];
            for (uint32_t i = i0; i < i1; i++) ws[i - i0] = W(*qkv_t[i]);
            for (uint32_t v = 0; v < n; v++) {
                xs[v] = es[v]->hidden;
                float *qkv_y[3] = {es[v]->q, es[v]->k, es[v]->v};
                for (uint32_t i = i0; i < i1; i++) ys[(i - i0) * n + v] = qkv_y[i];
            }
            ERC(zhk_dmmv_batched(c, qkv_t[i0]->type, 0, i1 - i0, ws, nullptr, qkv_m + i0, H, n, xs.data(), nullptr,
                                 ys.data(), Wf(y.attn_norm), m.eps, 0));
            i0 = i1;
        }
        // attention over each sequence's own KV cache: up to 4 sequences per
        // launch (grid z = sequence) when they share a 1-4 q-head group,
        // else one launch each (forking the sequences onto auxiliary streams,
        // joined before O, measured slower than in-order launches)
        bool all_ident = true;  // the several-sequence kernel reads identity page tables only
        for (uint32_t v = 0; v < n; v++) all_ident = all_ident && es[v]->pages_ident;
        if (m.n_heads / m.n_kv_heads <= 4 && all_ident) {
            for (uint32_t v0 = 0; v0 < n; v0 += 4) {
                const uint32_t nz = n - v0 < 4 ? n - v0 : 4;
                const float *aq[4], *ak[4], *av[4];
                uint16_t *akc[4], *avc[4];
                float *aout[4], *apart[4];
                void *axq[4];
                const uint32_t *apos[4];
                for (uint32_t z = 0; z < nz; z++) {
                    zh_engine *ev = es[v0 + z];
                    aq[z] = ev->q; ak[z] = ev->k; av[z] = ev->v;
                    akc[z] = ev->L[l].kc; avc[z] = ev->L[l].vc;
                    aout[z] = ev->attn; axq[z] = ev->xq_q; apart[z] = ev->fd_part; apos[z] = ev->st + ST_POS;
                }
                ERC(zhk_attn_decode_fused_z(c, nz, aq, ak, av, Wf(y.q_norm), Wf(y.k_norm), e0->rope_cs, akc, avc,
                                            e0->pages, e0->n_pages, m.max_ctx, aout, axq, m.n_heads, m.n_kv_heads,
                                            apos, m.max_ctx, scale, m.eps, apart));
            }
        } else {
            for (uint32_t v = 0; v < n; v++) {
                zh_engine *ev = es[v];
                const Layer &yv = ev->L[l];
                zh_pos_src pos{0, ev->st + ST_POS};
                ERC(zhk_attn_decode_fused(c, ev->q, ev->k, ev->v, Wf(y.q_norm), Wf(y.k_norm), ev->rope_cs, yv.kc,
                                          yv.vc, ev->pages, ev->n_pages, m.max_ctx, ev->attn, ev->xq_q, m.n_heads,
                                          m.n_kv_heads, pos, m.max_ctx, scale, m.eps, ev->fd_part, ev->pages_ident));
            }
        }
        // O (+ residual) on each sequence's XQ attention output
        const uint8_t *wo = W(y.wo), *wg = W(y.gate), *wd = W(y.down);
        for (uint32_t v = 0; v < n; v++) {
            xqs[v] = es[v]->xq_q;
            ys[v] = es[v]->hidden;
        }
        ERC(zhk_dmmv_batched(c, y.wo.type, 0, 1, &wo, nullptr, &H, qd, n, nullptr, xqs.data(), ys.data(), nullptr,
                             0.f, 1));
        // ffn_norm + gate/up + SwiGLU, then down (+ residual)
        const uint32_t F = m.ffn;
        for (uint32_t v = 0; v < n; v++) {
            xs[v] = es[v]->hidden;
            ys[v] = es[v]->s;
        }
        ERC(zhk_dmmv_batched(c, ZH_Q4_K, 1, 1, &wg, W(y.up), &F, H, n, xs.data(), nullptr, ys.data(),
                             Wf(y.ffn_norm), m.eps, 0));
        for (uint32_t v = 0; v < n; v++) {
            xs[v] = es[v]->s;
            ys[v] = es[v]->hidden;
        }
        ERC(zhk_dmmv_batched(c, y.down.type, 0, 1, &wd, nullptr, &H, F, n, xs.data(), nullptr, ys.data(), nullptr,
                             0.f, 1));
    }
    if (collect) {
        const uint8_t *wl = A + e0->lm.off;
        const uint32_t V = m.vocab;
        for (uint32_t v = 0; v < n; v++) {
            xs[v] = es[v]->hidden;
            ys[v] = es[v]->logits;
        }
        ERC(zhk_dmmv_batched(c, e0->lm.type, 0, 1, &wl, nullptr, &V, H, n, xs.data(), nullptr, ys.data(),
                             (const float *)(A + e0->out_norm.off), m.eps, 0));
        for (uint32_t v = 0; v < n; v++)
            ERC(zhk_argmax(c, es[v]->logits, V, es[v]->st + ST_TOKEN_OUT, es[v]->am_part, es[v]->ring,
                           es[v]->st + ST_GEN));
    }
    for (uint32_t v = 0; v < n; v++)
        hipLaunchKernelGGL(k_advance, dim3(1), dim3(1), 0, c->stream, es[v]->st, (const uint32_t *)es[v]->prompt);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

extern "C" int zh_engine_generate_batch(zh_engine *const *engines, uint32_t n_seq, const uint32_t *prompts,
                                        uint32_t n_prompt, uint32_t start_pos, uint32_t max_tokens,
                                        uint32_t *out_tokens) {
    if (!engines || n_seq == 0 || !engines[0] || !prompts || n_prompt == 0 || !out_tokens)
        return ZH_ERR_INVALID_ARGUMENT;
    zh_engine *e0 = engines[0];
    zh_ctx *c = e0->ctx;
    const zh_model_config &m = e0->c;
    if (n_prompt > MAX_PROMPT || max_tokens > MAX_GEN) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "too long");
    for (uint32_t v = 0; v < n_seq; v++) {
        const zh_engine *ev = engines[v];
        if (!ev || ev->ctx != c || ev->arena != e0->arena || ev->c.n_layers != m.n_layers ||
            ev->c.max_ctx != m.max_ctx)
            return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT,
                              "batch: engine %u does not share the weights and context of engine 0", v);
        for (uint32_t w = 0; w < v; w++)
            if (engines[w] == ev) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "batch: engine %u repeated", v);
    }
    if (m.n_experts || !zhk_lpb_supported(e0->lm.type, m.hidden) ||
        (e0->lm.type != ZH_Q4_K && e0->lm.type != ZH_Q6_K))
        return zh_set_err(c, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "batch: dense models on Q4_K / Q6_K projections only");
    for (uint32_t l = 0; l < m.n_layers; l++)
        if (!batch_layer_ok(e0, e0->L[l]))
            return zh_set_err(c, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "batch: layer %u has a format without a tile kernel", l);
    if ((uint64_t)start_pos + n_prompt + max_tokens > m.max_ctx + 1ull)
        return zh_set_err(c, ZH_ERR_CONTEXT_LENGTH_EXCEEDED, "context %u + %u + %u > %u", start_pos, n_prompt,
                          max_tokens, m.max_ctx);
    if (max_tokens == 0) return ZH_OK;
    for (uint32_t v = 0; v < n_seq; v++) {
        zh_engine *ev = engines[v];
        EHIP(ev, hipMemcpyAsync(ev->prompt, prompts + (size_t)v * n_prompt, 4ull * n_prompt, hipMemcpyHostToDevice,
                                c->stream));
        ERC(set_state(ev, n_prompt, start_pos, prompts[(size_t)v * n_prompt]));
    }
    for (uint32_t i = 0; i + 1 < n_prompt; i++) ERC(record_step_batch(engines, n_seq, false));
    for (uint32_t i = 0; i < max_tokens; i++) ERC(record_step_batch(engines, n_seq, true));
    for (uint32_t v = 0; v < n_seq; v++) {
        EHIP(engines[v], hipMemcpyAsync(out_tokens + (size_t)v * max_tokens, engines[v]->ring, 4ull * max_tokens,
                                        hipMemcpyDeviceToHost, c->stream));
        engines[v]->have_logits = true;
    }
    EHIP(e0, hipStreamSynchronize(c->stream));
    return ZH_OK;
}

extern "C" int zh_engine_generate(zh_engine *e, const uint32_t *prompt, uint32_t n_prompt, uint32_t start_pos,
                                  uint32_t max_tokens, uint32_t eos, uint32_t *out_tokens, uint32_t *n_out) {
    if (!e || !prompt || n_prompt == 0 || !out_tokens || !n_out) return ZH_ERR_INVALID_ARGUMENT;
    *n_out = 0;
    if (n_prompt > MAX_PROMPT || max_tokens > MAX_GEN) return zh_set_err(e->ctx, ZH_ERR_INVALID_ARGUMENT, "too long");
    if ((uint64_t)start_pos + n_prompt + max_tokens > e->c.max_ctx + 1ull)
        return zh_set_err(e->ctx, ZH_ERR_CONTEXT_LENGTH_EXCEEDED, "context %u + %u + %u > %u", start_pos, n_prompt,
                          max_tokens, e->c.max_ctx);
    if (max_tokens == 0) return ZH_OK;
    EHIP(e, hipMemcpyAsync(e->prompt, prompt, 4ull * n_prompt, hipMemcpyHostToDevice, e->ctx->stream));
    ERC(set_state(e, n_prompt, start_pos, prompt[0]));
    for (uint32_t i = 0; i + 1 < n_prompt; i++) ERC(run_step(e, false));
    for (uint32_t i = 0; i < max_tokens; i++) ERC(run_step(e, true));
    EHIP(e, hipMemcpyAsync(out_tokens, e->ring, 4ull * max_tokens, hipMemcpyDeviceToHost, e->ctx->stream));
    EHIP(e, hipStreamSynchronize(e->ctx->stream));
    e->have_logits = true;
    uint32_t n = max_tokens;
    if (eos != 0xFFFFFFFFu)
        for (uint32_t i = 0; i < max_tokens; i++)
            if (out_tokens[i] == eos) { n = i + 1; break; }
    *n_out = n;
    return ZH_OK;
}

// ---------------------------------------------------------------------------
// Batched prefill (prefillBatched, forward.zig:9330-9735): tokens at
// positions start_pos .. start_pos+n-1 in chunks of PF_CHUNK, every
// projection as an MFMA dequant-GEMM over the chunk, per layer:
// RMSNorm -> Q/K/V -> q/k norm + RoPE + KV write -> causal attention ->
// O (+residual) -> RMSNorm -> gate, up -> SwiGLU -> down (+residual).
// The last token's hidden state becomes the decode state; with `collect`
// its logits and greedy token are produced as decodeStep(collect) does.
// MoE models (no batched expert GEMM here) run the decode step per token.
// ---------------------------------------------------------------------------
static bool prefill_batched_ok(const zh_engine *e) {
    const zh_model_config &m = e->c;
    auto gemm_t = [](const Tensor &t) { return t.type == ZH_Q4_K || t.type == ZH_Q6_K; };
    if (m.n_experts || m.head_dim != 128 || m.hidden % 256 || m.ffn % 256 || (m.n_heads * m.head_dim) % 256 ||
        m.hidden > 16384 || m.ffn > 16384)  // the row kernels hold a row in registers
        return false;
    for (const Layer &y : e->L)
        if (!gemm_t(y.wq) || !gemm_t(y.wk) || !gemm_t(y.wv) || !gemm_t(y.wo) || !gemm_t(y.gate) || !gemm_t(y.up) ||
            !gemm_t(y.down))
            return false;
    return true;
}

static int ensure_prefill(zh_engine *e) {
    if (e->pf.arena) return ZH_OK;
    const zh_model_config &m = e->c;
    const uint64_t C = PF_CHUNK, H = m.hidden, qd = (uint64_t)m.n_heads * m.head_dim,
                   kvd = (uint64_t)m.n_kv_heads * m.head_dim, F = m.ffn, XK = H > qd ? H : qd;
    struct { void **p; uint64_t bytes; } a[] = {
        {(void **)&e->pf.hid, 4 * C * H}, {(void **)&e->pf.q, 4 * C * qd}, {(void **)&e->pf.k, 4 * C * kvd},
        {(void **)&e->pf.v, 4 * C * kvd}, {(void **)&e->pf.g, 4 * C * F}, {(void **)&e->pf.u, 4 * C * F},
        {(void **)&e->pf.xh, 2 * C * XK}, {(void **)&e->pf.att, 2 * C * qd}, {(void **)&e->pf.s, 2 * C * F},
        {(void **)&e->pf.ids, 4ull * MAX_PROMPT}, {(void **)&e->pf.s_unscale, 4 * C},
    };
    uint64_t off = 0;
    for (auto &x : a) off = align256(off + x.bytes);
    EHIP(e, hipMalloc(&e->pf.arena, off + 256));
    off = 0;
    for (auto &x : a) {
        *x.p = (char *)e->pf.arena + off;
        off = align256(off + x.bytes);
    }
    return ZH_OK;
}

extern "C" int zh_engine_prefill(zh_engine *e, const uint32_t *tokens, uint32_t n, uint32_t start_pos, int collect) {
    if (!e || !tokens || n == 0) return ZH_ERR_INVALID_ARGUMENT;
    if (n > MAX_PROMPT) return zh_set_err(e->ctx, ZH_ERR_INVALID_ARGUMENT, "prefill of %u tokens > %u", n, MAX_PROMPT);
    if ((uint64_t)start_pos + n > e->c.max_ctx)
        return zh_set_err(e->ctx, ZH_ERR_CONTEXT_LENGTH_EXCEEDED, "context %u + %u > %u", start_pos, n, e->c.max_ctx);
    zh_ctx *c = e->ctx;
    const zh_model_config &m = e->c;
    if (!prefill_batched_ok(e)) {
        EHIP(e, hipMemcpyAsync(e->prompt, tokens, 4ull * n, hipMemcpyHostToDevice, c->stream));
        ERC(set_state(e, n, start_pos, tokens[0]));
        for (uint32_t i = 0; i < n; i++) ERC(run_step(e, collect && i + 1 == n));
        if (collect) e->have_logits = true;
        return ZH_OK;
    }
    ERC(ensure_prefill(e));
    const uint32_t H = m.hidden, hd = m.head_dim, qd = m.n_heads * hd, kvd = m.n_kv_heads * hd, F = m.ffn;
    const uint8_t *A = e->arena;
    auto W = [&](const Tensor &t) { return A + t.off; };
    auto Wf = [&](const Tensor &t) { return (const float *)(A + t.off); };
    const float scale = 1.0f / sqrtf((float)hd);
    EHIP(e, hipMemcpyAsync(e->pf.ids, tokens, 4ull * n, hipMemcpyHostToDevice, c->stream));
    uint32_t last = 0;
    for (uint32_t off = 0; off < n; off += PF_CHUNK) {
        const uint32_t nt = n - off < PF_CHUNK ? n - off : PF_CHUNK, pos0 = start_pos + off;
        last = nt;
        ERC(zhk_dequant_rows(c, e->embd.type, W(e->embd), 0, nt, H, e->pf.hid, e->pf.ids + off, m.vocab, 1));
        for (uint32_t l = 0; l < m.n_layers; l++) {
            const Layer &y = e->L[l];
            // attn_norm: layer 0 here, later layers in the previous layer's down projection
            if (l == 0) ERC(zhk_rms_norm_rows_f16(c, e->pf.hid, Wf(y.attn_norm), e->pf.xh, H, nt, m.eps));
            {  // Q, K and V: one launch per run of equal types (one when all agree)
                const Tensor *ts[3] = {&y.wq, &y.wk, &y.wv};
                float *ys[3] = {e->pf.q, e->pf.k, e->pf.v};
                const uint32_t ld[3] = {qd, kvd, kvd}, ms[3] = {qd, kvd, kvd};
                // one launch for all three (head_dim 128): q/k norm, RoPE and the
                // KV-cache write in its epilogue
                const zh_gemm_rope rope = {Wf(y.q_norm), Wf(y.k_norm), e->inv_freq, y.kc, y.vc, e->pages,
                                           e->n_pages, m.max_ctx, m.n_heads, m.n_kv_heads, pos0, m.eps};
                const bool fused = hd == 128 && ts[0]->type == ts[1]->type && ts[1]->type == ts[2]->type;
                for (uint32_t i0 = 0; i0 < 3;) {
                    uint32_t i1 = i0 + 1;
                    while (i1 < 3 && ts[i1]->type == ts[i0]->type) i1++;
                    const uint8_t *ws[3];
                    for (uint32_t i = i0; i < i1; i++) ws[i - i0] = W(*ts[i]);
                    ERC(zhk_gemm_multi(c, ts[i0]->type, i1 - i0, ws, e->pf.xh, H, ys + i0, ld + i0, ms + i0, H, nt, 0,
                                       nullptr, nullptr, nullptr, 0.f, fused ? &rope : nullptr));
                    i0 = i1;
                }
                if (!fused)
                    ERC(zhk_qk_norm_rope_kv(c, e->pf.q, Wf(y.q_norm), e->pf.k, Wf(y.k_norm), e->pf.v, e->inv_freq, y.kc,
                                            y.vc, e->pages, e->n_pages, m.max_ctx, m.n_heads, m.n_kv_heads, hd,
                                            zh_pos_src{pos0, nullptr}, m.eps, nt));
            }
            ERC(zhk_attn_prefill(c, e->pf.q, y.kc, y.vc, e->pages, e->n_pages, m.max_ctx, m.n_heads, m.n_kv_heads, hd,
                                 pos0, nt, scale, e->pf.att));
            // O added into the residual, then ffn_norm (one pass with the split-K sums)
            ERC(zhk_gemm_norm(c, y.wo.type, W(y.wo), e->pf.att, qd, e->pf.hid, H, qd, nt, 1, nullptr,
                              Wf(y.ffn_norm), e->pf.xh, m.eps));
            if (y.gate.type == y.up.type) {  // gate and up in one launch
                const uint8_t *ws[2] = {W(y.gate), W(y.up)};
                float *ys[2] = {e->pf.g, e->pf.u};
                const uint32_t ld[2] = {F, F}, ms[2] = {F, F};
                ERC(zhk_gemm_multi(c, y.gate.type, 2, ws, e->pf.xh, H, ys, ld, ms, H, nt, 0));
            } else {
                ERC(zhk_gemm(c, y.gate.type, W(y.gate), e->pf.xh, H, e->pf.g, F, F, H, nt, 0));
                ERC(zhk_gemm(c, y.up.type, W(y.up), e->pf.xh, H, e->pf.u, F, F, H, nt, 0));
            }
            ERC(zhk_swiglu_rows_f16(c, e->pf.g, e->pf.u, e->pf.s, e->pf.s_unscale, F, nt));
            if (l + 1 < m.n_layers)  // down added into the residual, then the next layer's attn_norm
                ERC(zhk_gemm_norm(c, y.down.type, W(y.down), e->pf.s, F, e->pf.hid, H, F, nt, 1, e->pf.s_unscale,
                                  Wf(e->L[l + 1].attn_norm), e->pf.xh, m.eps));
            else
                ERC(zhk_gemm(c, y.down.type, W(y.down), e->pf.s, F, e->pf.hid, H, H, F, nt, 1, e->pf.s_unscale));
        }
    }
    EHIP(e, hipMemcpyAsync(e->hidden, e->pf.hid + (size_t)(last - 1) * H, 4ull * H, hipMemcpyDeviceToDevice,
                           c->stream));
    if (collect) {
        ERC(set_state(e, 1, start_pos + n - 1, tokens[n - 1]));
        ERC(record_collect(e));
        e->have_logits = true;
    }
    return ZH_OK;
}

extern "C" int zh_engine_logits(zh_engine *e, float *dst) {
    if (!e || !dst) return ZH_ERR_INVALID_ARGUMENT;
    EHIP(e, hipMemcpyAsync(dst, e->logits, 4ull * e->c.vocab, hipMemcpyDeviceToHost, e->ctx->stream));
    EHIP(e, hipStreamSynchronize(e->ctx->stream));
    return ZH_OK;
}
extern "C" int zh_engine_hidden(zh_engine *e, float *dst) {
    if (!e || !dst) return ZH_ERR_INVALID_ARGUMENT;
    EHIP(e, hipMemcpyAsync(dst, e->hidden, 4ull * e->c.hidden, hipMemcpyDeviceToHost, e->ctx->stream));
    EHIP(e, hipStreamSynchronize(e->ctx->stream));
    return ZH_OK;
}

// Inspection entry (no counterpart in the reference): the experts the last
// decode step selected in `layer` and their routing weights (n_experts_used
// of each), as the step's router top-k left them on the device.
extern "C" int zh_engine_routing(zh_engine *e, uint32_t layer, uint32_t *ids, float *weights) {
    if (!e || !ids || !weights || e->c.n_experts == 0 || layer >= e->c.n_layers) return ZH_ERR_INVALID_ARGUMENT;
    const uint32_t k = e->c.n_experts_used;
    uint32_t w[ZH_ROUTE_WORDS];
    EHIP(e, hipMemcpyAsync(w, e->routing + (size_t)ZH_ROUTE_WORDS * layer, 8ull * k, hipMemcpyDeviceToHost,
                           e->ctx->stream));
    EHIP(e, hipStreamSynchronize(e->ctx->stream));
    for (uint32_t i = 0; i < k; i++) {
        ids[i] = w[i];
        memcpy(&weights[i], &w[k + i], 4);
    }
    return ZH_OK;
}

extern "C" int zh_engine_tensor(zh_engine *e, uint64_t stream, zh_buf **buf, uint64_t *offset, uint64_t *bytes) {
    if (!e || !buf || !offset || !bytes) return ZH_ERR_INVALID_ARGUMENT;
    auto it = e->tensors.find(stream);
    if (it == e->tensors.end()) return zh_set_err(e->ctx, ZH_ERR_TENSOR_NOT_FOUND, "stream %llu", (unsigned long long)stream);
    e->pk_stale = true;  // the caller may write the weights through the view
    static thread_local zh_buf view;
    view.ptr = e->arena;
    view.size = e->arena_bytes;
    *buf = &view;
    *offset = it->second.off;
    *bytes = it->second.bytes;
    return ZH_OK;
}

extern "C" int zh_engine_read_kv(zh_engine *e, uint32_t layer, uint32_t which, uint32_t t0, uint32_t n, uint16_t *dst) {
    if (!e || !dst || layer >= e->c.n_layers || which > 1) return ZH_ERR_INVALID_ARGUMENT;
    if ((uint64_t)t0 + n > e->c.max_ctx) return zh_set_err(e->ctx, ZH_ERR_INVALID_ARGUMENT, "kv range");
    if (n == 0) return ZH_OK;
    uint32_t nkv = e->c.n_kv_heads, hd = e->c.head_dim;
    uint64_t cnt = (uint64_t)n * nkv * hd;
    void *scr;
    ERC(zh_scratch(e->ctx, cnt * 2, &scr));
    hipLaunchKernelGGL(k_gather_kv, dim3((unsigned)((cnt + 255) / 256)), dim3(256), 0, e->ctx->stream,
                       (const uint16_t *)(which ? e->L[layer].vc : e->L[layer].kc), nkv, e->c.max_ctx, hd,
                       (const uint32_t *)e->pages, t0, n, (uint16_t *)scr);
    ZH_LAUNCH_CHECK(e->ctx);
    EHIP(e, hipMemcpyAsync(dst, scr, cnt * 2, hipMemcpyDeviceToHost, e->ctx->stream));
    EHIP(e, hipStreamSynchronize(e->ctx->stream));
    return ZH_OK;
}

extern "C" uint64_t zh_engine_bytes_per_token(zh_engine *e, uint32_t Lctx) {
    if (!e) return 0;
    const zh_model_config &c = e->c;
    uint64_t b = e->lm.bytes + e->out_norm.bytes + zh_tensor_bytes(e->embd.type, 1, c.hidden);
    for (const Layer &y : e->L) {
        b += y.attn_norm.bytes + y.wq.bytes + y.wk.bytes + y.wv.bytes + y.wo.bytes + y.q_norm.bytes + y.k_norm.bytes +
             y.ffn_norm.bytes;
        if (c.n_experts == 0) b += y.gate.bytes + y.up.bytes + y.down.bytes;
        else
            b += y.router.bytes + (uint64_t)c.n_experts_used *
                                      (zh_tensor_bytes(y.egate.type, c.expert_ffn, c.hidden) * 2 +
                                       zh_tensor_bytes(y.edown.type, c.hidden, c.expert_ffn));
        b += 2ull * c.n_kv_heads * c.head_dim * 2ull * Lctx;  // fp16 K and V
    }
    return b;
}

// Algorithmic bytes of one launch group of layer 0 at context length Lctx:
// the weights it reads, its activation inputs and outputs, the KV rows the
// attention reads and writes (internal scratch traffic such as attention
// partials is not counted).
extern "C" uint64_t zh_engine_group_bytes(zh_engine *e, uint32_t group, uint32_t Lctx) {
    if (!e || e->L.empty()) return 0;
    const zh_model_config &c = e->c;
    const Layer &y = e->L[0];
    const uint64_t H = c.hidden, hd = c.head_dim, qd = (uint64_t)c.n_heads * hd, kvd = (uint64_t)c.n_kv_heads * hd;
    const uint64_t F = c.n_experts ? c.expert_ffn : c.ffn, k = c.n_experts ? c.n_experts_used : 1;
    auto xqb = [](uint64_t n) { return n / 32 * 108; };
    switch (group) {
    case SK_QKV | SK_ATTN:
        return zh_engine_group_bytes(e, SK_QKV, Lctx) + zh_engine_group_bytes(e, SK_ATTN, Lctx) - (qd + 2 * kvd) * 8;
    case SK_QKV | SK_ATTN | SK_O:  // the attention output stays on chip; O adds into x
        return zh_engine_group_bytes(e, SK_QKV | SK_ATTN, Lctx) + y.wo.bytes + H * 4 - xqb(qd);
    case SK_QKV: return y.wq.bytes + y.wk.bytes + y.wv.bytes + 2 * H * 4 + (qd + 2 * kvd) * 4;
    case SK_ATTN:
        return 2 * kvd * 2 * Lctx + (qd + 2 * kvd) * 4 + 2 * hd * 4 + hd * 4 + 2 * kvd * 2 + qd * 4 + xqb(qd);
    case SK_O: return y.wo.bytes + xqb(qd) + 2 * H * 4;
    case SK_FFN_IN | SK_FFN_OUT:
        // MoE (k_moe_xcd): the router, the selected experts, x and norm in, the sums added into y
        if (c.n_experts)
            return y.router.bytes + k * 3 * zh_tensor_bytes(y.egate.type, (uint32_t)F, (uint32_t)H) + 4 * H * 4;
        // dense (k_ffn_xcd): x = two vectors in, one out, the sums added into a third
        return y.gate.bytes + y.up.bytes + y.down.bytes + 5 * H * 4;
    case SK_FFN_IN:
        if (c.n_experts == 0) return y.gate.bytes + y.up.bytes + 2 * H * 4 + F * 4 + xqb(F);
        return y.router.bytes + 2 * k * zh_tensor_bytes(y.egate.type, (uint32_t)F, (uint32_t)H) + 2 * H * 4 +
               xqb(H) + (uint64_t)c.n_experts * 4 + 8 * k + k * F * 4;
    case SK_FFN_OUT:
        if (c.n_experts == 0) return y.down.bytes + xqb(F) + 2 * H * 4;
        return k * zh_tensor_bytes(y.edown.type, (uint32_t)H, (uint32_t)F) + k * F * 4 + 2 * k * xqb(F) + 8 * k +
               2 * H * 4;
    default: return 0;
    }
}
