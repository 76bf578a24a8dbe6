// zh_ops.hip — RMSNorm, fused QK-norm/RoPE/KV write, split-context
// flash-decode with LSE merge, SwiGLU, MoE routing and argmax for gfx950.
#include <mutex>

#include "zh_device.h"
#include "zh_internal.h"
#include "zh_attn_common.h"

static bool in_range(const zh_buf *b, uint64_t off, uint64_t n) { return b && off <= b->size && n <= b->size - off; }
#define DPTR(b, off, T) ((T *)((char *)(b)->ptr + (off)))

// Quantise one 32-element block held one value per lane across a 32-lane
// group (l = lane index within the group) into XQ block `blk`.

// ---------------------------------------------------------------------------
// RMSNorm (rms_norm_mul.comp / cpuRmsNormMul forward.zig:618-626).
// One 256-thread workgroup per group; optional XQ output for a DMMV consumer.
// ---------------------------------------------------------------------------
// 1024 threads; every element a thread owns is loaded before any reduction so
// the kernel pays one memory latency, not one per loop trip.
constexpr int RMS_T = 1024, RMS_E = 8;  // up to 8192 elements per group in registers
__global__ __launch_bounds__(RMS_T) void k_rms_norm(const float *__restrict__ x, const float *__restrict__ w,
                                                    uint32_t w_len, float *__restrict__ out, uint8_t *xq,
                                                    uint32_t n, float eps) {
    const uint32_t g = blockIdx.x, t = threadIdx.x;
    const float *xg = x + (size_t)g * n;
    __shared__ float red[RMS_T / 64];
    float v[RMS_E], wv[RMS_E];
#pragma unroll
    for (int j = 0; j < RMS_E; j++) {
        uint32_t i = t + RMS_T * j;
        v[j] = i < n ? xg[i] : 0.f;
        wv[j] = i < n ? w[i % w_len] : 0.f;
    }
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < RMS_E; j++) sq = fmaf(v[j], v[j], sq);
    sq = wave_sum(sq);
    if ((t & 63) == 0) red[t >> 6] = sq;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int k = 0; k < RMS_T / 64; k++) tot += red[k];
    const float rms_inv = 1.0f / sqrtf(tot / (float)n + eps);
    XQView q = xq_view(xq, n / 32);
#pragma unroll
    for (int j = 0; j < RMS_E; j++) {
        uint32_t i = t + RMS_T * j;
        if (RMS_T * j >= n) break;  // uniform across the workgroup
        float o = wv[j] * (v[j] * rms_inv);
        if (i < n) out[(size_t)g * n + i] = o;
        if (xq && i < n) xq_store_block32(o, t & 31, q, (g * n + i) / 32);
    }
}

int zhk_rms_norm(zh_ctx *c, const float *x, const float *w, uint32_t w_len, float *out, void *xq, uint32_t n,
                 uint32_t n_groups, float eps) {
    if (n > RMS_T * RMS_E) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "rms_norm n=%u > %d", n, RMS_T * RMS_E);
    if (xq && n % 32) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "rms_norm xq needs n %% 32 == 0");
    hipLaunchKernelGGL(k_rms_norm, dim3(n_groups), dim3(RMS_T), 0, c->stream, x, w, w_len, out, (uint8_t *)xq, n, eps);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

extern "C" int zh_rms_norm(zh_ctx *c, const zh_buf *x, uint64_t x_off, const zh_buf *w, uint32_t w_len, zh_buf *out,
                           uint64_t out_off, uint32_t n, uint32_t n_groups, float eps) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    uint64_t tot = (uint64_t)n * n_groups * 4;
    if (n == 0 || n_groups == 0 || w_len == 0 || !in_range(x, x_off, tot) || !in_range(out, out_off, tot) ||
        !in_range(w, 0, (uint64_t)w_len * 4) || (x_off & 3) || (out_off & 3))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "rms_norm shape/range");
    return zhk_rms_norm(c, DPTR(x, x_off, const float), (const float *)w->ptr, w_len, DPTR(out, out_off, float),
                        nullptr, n, n_groups, eps);
}

// ---------------------------------------------------------------------------
// SwiGLU (swiglu.comp, cpuSwiGLU forward_metal.zig:6567-6572)
// ---------------------------------------------------------------------------
__global__ void k_swiglu(const float *g, const float *u, float *out, uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}
int zhk_swiglu(zh_ctx *c, const float *g, const float *u, float *out, uint32_t n) {
    hipLaunchKernelGGL(k_swiglu, dim3((n + 255) / 256), dim3(256), 0, c->stream, g, u, out, n);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
extern "C" int zh_swiglu(zh_ctx *c, const zh_buf *g, uint64_t g_off, const zh_buf *u, uint64_t u_off, zh_buf *out,
                         uint64_t out_off, uint32_t n) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (n == 0 || !in_range(g, g_off, n * 4ull) || !in_range(u, u_off, n * 4ull) || !in_range(out, out_off, n * 4ull))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "swiglu range");
    return zhk_swiglu(c, DPTR(g, g_off, const float), DPTR(u, u_off, const float), DPTR(out, out_off, float), n);
}

// ---------------------------------------------------------------------------
// Fused per-head Q/K RMSNorm + NeoX RoPE + fp16 KV write
// (qk_norm_rope_kv_write.comp:67-171). Workgroups [0, nq) are Q heads
// (in place), [nq, nq+nkv) are K heads, which also store V.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_qk_norm_rope_kv(float *q, const float *qw, const float *k, const float *kw,
                                                        const float *v, const float *inv_freq, uint16_t *kc,
                                                        uint16_t *vc, const uint32_t *pages, uint32_t n_pages,
                                                        uint32_t cache_tokens, uint32_t nq, uint32_t hd,
                                                        zh_pos_src pos_src, float eps, uint32_t q_stride,
                                                        uint32_t kv_stride) {
    // blockIdx.y = token of a batch (prefill): rows q_stride / kv_stride apart, position + token
    const uint32_t wg = blockIdx.x, lane = threadIdx.x, tok = blockIdx.y;
    q += (size_t)tok * q_stride;
    k += (size_t)tok * kv_stride;
    v += (size_t)tok * kv_stride;
    const bool is_q = wg < nq;
    const uint32_t head = is_q ? wg : wg - nq;
    const float *src = is_q ? q + (size_t)head * hd : k + (size_t)head * hd;
    const float *wt = is_q ? qw : kw;
    const uint32_t pos = read_pos(pos_src) + tok;
    float sq = 0.f;
    for (uint32_t i = lane; i < hd; i += 64) sq = fmaf(src[i], src[i], sq);
    sq = wave_sum(sq);
    const float rms_inv = 1.0f / sqrtf(sq / (float)hd + eps);
    const uint32_t half = hd / 2;
    uint32_t slot = pos / 16;
    bool ok = slot < n_pages;
    uint32_t phys = ok ? pages[slot] * 16 + pos % 16 : 0;
    ok = ok && phys < cache_tokens;
    uint16_t *kdst = kc + ((size_t)head * cache_tokens + phys) * hd;
    uint16_t *vdst = vc + ((size_t)head * cache_tokens + phys) * hd;
    for (uint32_t i = lane; i < half; i += 64) {
        float lo = wt[i] * (src[i] * rms_inv);
        float hi = wt[i + half] * (src[i + half] * rms_inv);
        float th = (float)pos * inv_freq[i];
        float s, co;
        sincosf(th, &s, &co);
        float rlo = lo * co - hi * s;
        float rhi = lo * s + hi * co;
        if (is_q) {
            q[(size_t)head * hd + i] = rlo;
            q[(size_t)head * hd + i + half] = rhi;
        } else if (ok) {
            kdst[i] = f2h_rn(rlo);
            kdst[i + half] = f2h_rn(rhi);
        }
    }
    if (!is_q && ok)
        for (uint32_t i = lane; i < hd; i += 64) vdst[i] = f2h_rn(v[(size_t)head * hd + i]);
}

int zhk_qk_norm_rope_kv(zh_ctx *c, float *q, const float *qw, const float *k, const float *kw, const float *v,
                        const float *inv_freq, uint16_t *kc, uint16_t *vc, const uint32_t *pages, uint32_t n_pages,
                        uint32_t cache_tokens, uint32_t nq, uint32_t nkv, uint32_t hd, zh_pos_src pos, float eps,
                        uint32_t n_tok) {
    hipLaunchKernelGGL(k_qk_norm_rope_kv, dim3(nq + nkv, n_tok), dim3(64), 0, c->stream, q, qw, k, kw, v, inv_freq,
                       kc, vc, pages, n_pages, cache_tokens, nq, hd, pos, eps, nq * hd, nkv * hd);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

extern "C" int zh_qk_norm_rope_kv_write(zh_ctx *c, zh_buf *q, const zh_buf *qw, const zh_buf *k, const zh_buf *kw,
                                        const zh_buf *v, const zh_buf *inv_freq, zh_buf *kc, zh_buf *vc,
                                        const zh_buf *pages, uint32_t n_pages, uint32_t cache_tokens, uint32_t nq,
                                        uint32_t nkv, uint32_t hd, uint32_t position, float eps) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (hd == 0 || hd % 2 || nq == 0 || nkv == 0 || nq % nkv)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "head shape");
    if (!in_range(q, 0, 4ull * nq * hd) || !in_range(k, 0, 4ull * nkv * hd) || !in_range(v, 0, 4ull * nkv * hd) ||
        !in_range(qw, 0, 4ull * hd) || !in_range(kw, 0, 4ull * hd) || !in_range(inv_freq, 0, 2ull * hd) ||
        !in_range(kc, 0, 2ull * nkv * cache_tokens * hd) || !in_range(vc, 0, 2ull * nkv * cache_tokens * hd) ||
        !in_range(pages, 0, 4ull * n_pages))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "qk_norm_rope_kv range");
    // logicalTokenToPhysicalToken (forward.zig:694-698)
    if (position / 16 >= n_pages) return zh_set_err(c, ZH_ERR_CONTEXT_LENGTH_EXCEEDED, "position %u", position);
    uint32_t page = 0;
    int rc = zh_buf_download(c, pages, 4ull * (position / 16), &page, 4);
    if (rc) return rc;
    if ((uint64_t)page * 16 + position % 16 >= cache_tokens)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "page %u beyond cache", page);
    return zhk_qk_norm_rope_kv(c, (float *)q->ptr, (const float *)qw->ptr, (const float *)k->ptr,
                               (const float *)kw->ptr, (const float *)v->ptr, (const float *)inv_freq->ptr,
                               (uint16_t *)kc->ptr, (uint16_t *)vc->ptr, (const uint32_t *)pages->ptr, n_pages,
                               cache_tokens, nq, nkv, hd, zh_pos_src{position, nullptr}, eps);
}

// ---------------------------------------------------------------------------
// Decode attention (flash_decode.comp + the qk_norm_rope_kv_write.comp work
// of the new token, forward.zig decodeStep attention block), one kernel:
//
//   grid (n_kv_heads, n_chunks), 256 threads = 4 waves x TW tokens, so a
//   workgroup covers a chunk (of 4 TW-token sub-chunks) of one kv head's GQA
//   group.
//   - FUSED: q (raw Q projection), the new token's raw k/v, per-head RMSNorm
//     weights and RoPE frequencies come in; every wave normalises and ropes q
//     in registers, and the wave that owns the new position also normalises
//     and ropes k, writes k/v to the fp16 cache and substitutes them for the
//     cache rows it loaded before the write.
//   - scores / chunk softmax / P*V per wave, the waves combined in LDS
//     with log-sum-exp weights, one partial (O, m, l) per q head and chunk.
//   - the last workgroup to finish for a kv head (agent-scope counter) merges
//     the chunks and writes the attention output (f32, optional XQ) and
//     resets the counter for the next launch.
// Dims are held as (d, d+64) pairs, sub*8..sub*8+7 and 64+sub*8.., so NeoX
// RoPE pairs stay inside a lane. Cache layout [kv_head][token][128] fp16,
// addressed through 16-token pages.
// ---------------------------------------------------------------------------
ZH_TRACE_DUMP_FN(zh_debug_trace_ops)

uint64_t zhk_flash_decode_partials_bytes(uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_seq) {
    // partials + two counter words per kv head (at most nh words)
    return (uint64_t)nh * attn_n_chunks(max_seq, attn_nd(nkv, 256)) * (hd + 2) * 4 + 4ull * nh + 256;
}

template <int G, bool FUSED, int MODE, int TW>
__global__ __launch_bounds__(AD_T, 1) void k_attn_decode(AttnP p) {
#include "zh_attn_body.inc"

}


// Several sequences in one launch (batched decode): blockIdx.z selects the
// sequence, whose buffers replace those of p0 (the weights, RoPE table and
// geometry are shared; the sequences are at the same position).
constexpr int AD_MAXZ = 4;
struct AttnZ {
    const float *q[AD_MAXZ], *k_new[AD_MAXZ], *v_new[AD_MAXZ];
    uint16_t *kc[AD_MAXZ], *vc[AD_MAXZ];
    const uint32_t *pos[AD_MAXZ];
    float *part[AD_MAXZ], *out[AD_MAXZ];
    uint32_t *counters[AD_MAXZ];
    uint8_t *xq[AD_MAXZ];
};
template <int G, int TW>
__global__ __launch_bounds__(AD_T, 1) void k_attn_decode_z(AttnP p0, AttnZ z) {
    constexpr bool FUSED = true;
    constexpr int MODE = AD_IDENT;
    AttnP p = p0;
    {
        const uint32_t s = blockIdx.z;
        p.q = z.q[s]; p.k_new = z.k_new[s]; p.v_new = z.v_new[s];
        p.kc = z.kc[s]; p.vc = z.vc[s]; p.pos.dev = z.pos[s];
        p.part = z.part[s]; p.out = z.out[s]; p.counters = z.counters[s]; p.xq = z.xq[s];
    }
#include "zh_attn_body.inc"
}

#include "zh_attn_ring.inc"

// partials: zhk_flash_decode_partials_bytes(nh, nkv, hd, max_seq) bytes; the
// counter words at its end must be zero before the first launch (each
// launch leaves them zero).
static int attn_launch(zh_ctx *c, const AttnP &p0, uint32_t nkv, uint32_t G, uint32_t max_seq, bool fused,
                       bool ident) {
    AttnP p = p0;
    p.nd = attn_nd(nkv, c->cu_count);
    p.no_wait = c->concurrent ? 1u : 0u;
    p.ctl = c->err_dev;
    // tokens per wave (see AD_W): sub-chunks only with identity pages and at
    // most 4 q heads per kv head
    const bool sub = ident && G <= 4;
    const uint32_t tw = !sub ? 40u : max_seq <= 8192 ? 24u : 32u;
    p.n_chunks = attn_n_chunks(max_seq, p.nd, AD_W * tw);
    // identity pages: at most nd chunks per kv head at any context (longer
    // chunks hold several sub-chunks)
    if (sub && p.n_chunks > p.nd) p.n_chunks = p.nd;
    dim3 grid(nkv, p.n_chunks);
    // one workgroup per CU: a grid within the CU count is resident at once
    const bool rev = (uint64_t)nkv * p.n_chunks > (uint64_t)c->cu_count;
#define AD_K(GG, FF, MM, TT) hipLaunchKernelGGL((k_attn_decode<GG, FF, MM, TT>), grid, dim3(AD_T), 0, c->stream, p)
#define AD_LAUNCH1(GG, FF)                                                   \
    if (ident && GG <= 4 && tw == 24) AD_K(GG, FF, AD_IDENT, GG <= 4 ? 24 : 40); \
    else if (ident && GG <= 4) AD_K(GG, FF, AD_IDENT, GG <= 4 ? 32 : 40);        \
    else if (ident) AD_K(GG, FF, AD_IDENT, 40);                                 \
    else if (rev) AD_K(GG, FF, AD_PAGED_REV, 40);                               \
    else AD_K(GG, FF, AD_PAGED, 40)
#define AD_LAUNCH(GG)          \
    if (fused) {               \
        AD_LAUNCH1(GG, true);  \
    } else {                   \
        AD_LAUNCH1(GG, false); \
    }
    switch (G) {
    case 1: AD_LAUNCH(1); break;
    case 2: AD_LAUNCH(2); break;
    case 4: AD_LAUNCH(4); break;
    case 8: AD_LAUNCH(8); break;
    default: return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "GQA group %u unsupported (1, 2, 4, 8)", G);
    }
#undef AD_LAUNCH
#undef AD_LAUNCH1
#undef AD_K
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

static uint32_t *attn_counters(float *partials, uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_seq) {
    return (uint32_t *)((char *)partials + (uint64_t)nh * attn_n_chunks(max_seq, attn_nd(nkv, 256)) * (hd + 2) * 4);
}

// Partials of the C-ABI decode attention (the DMA ring kernel): nh x nd
// chunk partials of 130 f32, then two merge counters per kv head.
static uint64_t ring_partials_bytes(uint32_t nh, uint32_t nkv, int cu_count) {
    return (uint64_t)nh * attn_nd(nkv, cu_count) * (FD_HD + 2) * 4 + 8ull * nkv;
}
static uint32_t *ring_counters(float *partials, uint32_t nh, uint32_t nkv, int cu_count) {
    return (uint32_t *)(partials + (uint64_t)nh * attn_nd(nkv, cu_count) * (FD_HD + 2));
}

int zhk_flash_decode(zh_ctx *c, const float *q, const uint16_t *kc, const uint16_t *vc, const uint32_t *pages,
                     uint32_t n_pages, uint32_t cache_tokens, float *out, void *xq_out, uint32_t nh, uint32_t nkv,
                     uint32_t hd, zh_pos_src seq_len, uint32_t max_seq, float scale, float *partials) {
    AttnP p = {};
    p.q = q; p.kc = (uint16_t *)kc; p.vc = (uint16_t *)vc; p.pages = pages; p.n_pages = n_pages;
    p.cache_tokens = cache_tokens; p.pos = seq_len; p.scale = scale; p.part = partials;
    p.counters = ring_counters(partials, nh, nkv, c->cu_count); p.out = out; p.xq = (uint8_t *)xq_out; p.nq = nh;
    p.ident = 0;
    (void)hd;
    return zhk_attn_ring(c, p, nkv, max_seq, false);
}

// RoPE table: cs[pos][i] = (cos, sin) of (float)pos * inv_freq[i], i < 64,
// the same f32 expression the per-position kernels evaluate.
__global__ void k_rope_table(const float *inv_freq, uint32_t n_pos, float *cs) {
    const uint32_t idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= n_pos * 64) return;
    const uint32_t pos = idx / 64, i = idx % 64;
    float sn, co;
    sincosf((float)pos * inv_freq[i], &sn, &co);
    cs[2 * idx] = co;
    cs[2 * idx + 1] = sn;
}
int zhk_rope_table(zh_ctx *c, const float *inv_freq, uint32_t n_pos, float *cs) {
    hipLaunchKernelGGL(k_rope_table, dim3((n_pos * 64 + 255) / 256), dim3(256), 0, c->stream, inv_freq, n_pos, cs);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

int zhk_attn_decode_fused(zh_ctx *c, const float *q, const float *k, const float *v, const float *qw, const float *kw,
                          const float *rope_cs, uint16_t *kc, uint16_t *vc, const uint32_t *pages, uint32_t n_pages,
                          uint32_t cache_tokens, float *out, void *xq_out, uint32_t nh, uint32_t nkv, zh_pos_src pos,
                          uint32_t max_seq, float scale, float eps, float *partials, bool ident_pages) {
    AttnP p = {};
    p.q = q; p.k_new = k; p.v_new = v; p.q_norm = qw; p.k_norm = kw; p.rope_cs = rope_cs;
    p.kc = kc; p.vc = vc; p.pages = pages; p.n_pages = n_pages; p.cache_tokens = cache_tokens; p.pos = pos;
    p.scale = scale; p.eps = eps; p.part = partials; p.counters = attn_counters(partials, nh, nkv, FD_HD, max_seq);
    p.out = out; p.xq = (uint8_t *)xq_out; p.nq = nh;
    // identity page table: the register-pipelined kernel (measured faster at a
    // 4K context); any other table: the DMA ring kernel, which looks pages up
    if (ident_pages) return attn_launch(c, p, nkv, nh / nkv, max_seq, true, true);
    p.ident = 0;
    return zhk_attn_ring(c, p, nkv, max_seq, true);
}

// zhk_attn_decode_fused for n <= 4 sequences at one position in one launch
// (grid z = sequence), identity pages, the no-wait merge. Array arguments hold
// one entry per sequence; the weights, RoPE table and page table are shared.
int zhk_attn_decode_fused_z(zh_ctx *c, uint32_t n, const float *const *q, const float *const *k,
                            const float *const *v, const float *qw, const float *kw, const float *rope_cs,
                            uint16_t *const *kc, uint16_t *const *vc, const uint32_t *pages, uint32_t n_pages,
                            uint32_t cache_tokens, float *const *out, void *const *xq_out, uint32_t nh, uint32_t nkv,
                            const uint32_t *const *pos_dev, uint32_t max_seq, float scale, float eps,
                            float *const *partials) {
    const uint32_t G = nkv ? nh / nkv : 0;
    if (n == 0 || n > (uint32_t)AD_MAXZ || G == 0 || G > 4 || (G & (G - 1)))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "batched attention: %u sequences, group %u", n, G);
    AttnP p = {};
    p.q_norm = qw; p.k_norm = kw; p.rope_cs = rope_cs; p.pages = pages; p.n_pages = n_pages;
    p.cache_tokens = cache_tokens; p.pos = zh_pos_src{0, pos_dev[0]}; p.scale = scale; p.eps = eps; p.nq = nh;
    p.nd = attn_nd(nkv, c->cu_count);
    p.no_wait = 1;  // chunks of other sequences share the device: no merger waits
    p.ctl = c->err_dev;
    const uint32_t tw = max_seq <= 8192 ? 24u : 32u;
    p.n_chunks = attn_n_chunks(max_seq, p.nd, AD_W * tw);
    if (p.n_chunks > p.nd) p.n_chunks = p.nd;
    AttnZ z = {};
    for (uint32_t s = 0; s < n; s++) {
        z.q[s] = q[s]; z.k_new[s] = k[s]; z.v_new[s] = v[s]; z.kc[s] = kc[s]; z.vc[s] = vc[s];
        z.pos[s] = pos_dev[s]; z.part[s] = partials[s]; z.out[s] = out[s]; z.xq[s] = (uint8_t *)xq_out[s];
        z.counters[s] = attn_counters(partials[s], nh, nkv, FD_HD, max_seq);
    }
    dim3 grid(nkv, p.n_chunks, n);
#define AZ(GG)                                                                                                   \
    if (tw == 24) hipLaunchKernelGGL((k_attn_decode_z<GG, 24>), grid, dim3(AD_T), 0, c->stream, p, z);           \
    else hipLaunchKernelGGL((k_attn_decode_z<GG, 32>), grid, dim3(AD_T), 0, c->stream, p, z)
    switch (G) {
    case 1: AZ(1); break;
    case 2: AZ(2); break;
    default: AZ(4); break;
    }
#undef AZ
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

extern "C" int zh_flash_decode(zh_ctx *c, const zh_buf *q, const zh_buf *kc, const zh_buf *vc, const zh_buf *pages,
                               uint32_t n_pages, uint32_t cache_tokens, zh_buf *out, uint32_t nh, uint32_t nkv,
                               uint32_t hd, uint32_t seq_len, float attn_scale) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (hd != FD_HD) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "head_dim %u unsupported (128 only)", hd);
    if (nkv == 0 || nh % nkv || nh / nkv > FD_MAXG || ((nh / nkv) & (nh / nkv - 1)) || seq_len == 0)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "heads/seq_len");
    if ((seq_len + 15) / 16 > n_pages) return zh_set_err(c, ZH_ERR_CONTEXT_LENGTH_EXCEEDED, "seq_len %u", seq_len);
    if (!in_range(q, 0, 4ull * nh * hd) || !in_range(out, 0, 4ull * nh * hd) ||
        !in_range(kc, 0, 2ull * nkv * cache_tokens * hd) || !in_range(vc, 0, 2ull * nkv * cache_tokens * hd) ||
        !in_range(pages, 0, 4ull * n_pages))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "flash_decode range");
    void *scr;
    int rc = zh_scratch(c, ring_partials_bytes(nh, nkv, c->cu_count), &scr);
    if (rc) return rc;
    ZH_HIP(c, hipMemsetAsync(ring_counters((float *)scr, nh, nkv, c->cu_count), 0, 8ull * nkv, c->stream));
    float scale = attn_scale != 0.f ? attn_scale : 1.0f / sqrtf((float)hd);
    return zhk_flash_decode(c, (const float *)q->ptr, (const uint16_t *)kc->ptr, (const uint16_t *)vc->ptr,
                            (const uint32_t *)pages->ptr, n_pages, cache_tokens, (float *)out->ptr, nullptr, nh, nkv,
                            hd, zh_pos_src{seq_len, nullptr}, seq_len, scale, (float *)scr);
}

// ---------------------------------------------------------------------------
// zh_flash_decode without allocation: the split-K partials and the merge
// counters live in a file-scope device array (one copy per GPU, held until
// the process ends) instead of the context's growable scratch. In host code
// the array's name is only a stand-in: its device address on the current
// GPU comes from hipGetSymbolAddress, looked up once per device on the first
// call there and kept per device.
// ---------------------------------------------------------------------------
constexpr uint64_t FD_NOALLOC_BYTES = 2ull << 20;  // partials (nh x chunks x 130 f32) + counters
static __device__ __align__(256) uint8_t scratch[FD_NOALLOC_BYTES];

__global__ void k_zero_u32(uint32_t *p, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

static int noalloc_scratch(zh_ctx *c, void **out) {
    static std::mutex mu;
    static void *ptr[64] = {};
    if (c->device < 0 || c->device >= 64) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "device %d", c->device);
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[c->device]) {
        // (the caller's current device is restored afterwards)
        int prev = 0;
        ZH_HIP(c, hipGetDevice(&prev));
        ZH_HIP(c, hipSetDevice(c->device));
        void *p = nullptr;
        const hipError_t ge = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        ZH_HIP(c, hipSetDevice(prev));
        ZH_HIP(c, ge);
        if (!p) return zh_set_err(c, ZH_ERR_HIP, "no device address for the no-alloc scratch");
        ptr[c->device] = p;
    }
    *out = ptr[c->device];
    return ZH_OK;
}

extern "C" int zh_flash_decode_noalloc(zh_ctx *c, const zh_buf *q, const zh_buf *kc, const zh_buf *vc,
                                       const zh_buf *pages, uint32_t n_pages, uint32_t cache_tokens, zh_buf *out,
                                       uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t seq_len, float attn_scale) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (hd != FD_HD) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "head_dim %u unsupported (128 only)", hd);
    if (nkv == 0 || nh % nkv || nh / nkv > FD_MAXG || ((nh / nkv) & (nh / nkv - 1)) || seq_len == 0)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "heads/seq_len");
    if ((seq_len + 15) / 16 > n_pages) return zh_set_err(c, ZH_ERR_CONTEXT_LENGTH_EXCEEDED, "seq_len %u", seq_len);
    if (!in_range(q, 0, 4ull * nh * hd) || !in_range(out, 0, 4ull * nh * hd) ||
        !in_range(kc, 0, 2ull * nkv * cache_tokens * hd) || !in_range(vc, 0, 2ull * nkv * cache_tokens * hd) ||
        !in_range(pages, 0, 4ull * n_pages))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "flash_decode range");
    // the same partials layout as zh_flash_decode's scratch (counters after
    // the partials), which must fit the array
    const uint64_t need = ring_partials_bytes(nh, nkv, c->cu_count);
    if (need > FD_NOALLOC_BYTES)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "flash_decode_noalloc: %llu bytes of partials exceed its %llu",
                          (unsigned long long)need, (unsigned long long)FD_NOALLOC_BYTES);
    void *scr;
    int rc = noalloc_scratch(c, &scr);
    if (rc) return rc;
    // the merge counters start at zero (a fill kernel, not a memset node, so
    // the call may be captured into a graph)
    uint32_t *cnt = ring_counters((float *)scr, nh, nkv, c->cu_count);
    hipLaunchKernelGGL(k_zero_u32, dim3((2 * nkv + 255) / 256), dim3(256), 0, c->stream, cnt, 2 * nkv);
    ZH_LAUNCH_CHECK(c);
    float scale = attn_scale != 0.f ? attn_scale : 1.0f / sqrtf((float)hd);
    return zhk_flash_decode(c, (const float *)q->ptr, (const uint16_t *)kc->ptr, (const uint16_t *)vc->ptr,
                            (const uint32_t *)pages->ptr, n_pages, cache_tokens, (float *)out->ptr, nullptr, nh, nkv,
                            hd, zh_pos_src{seq_len, nullptr}, seq_len, scale, (float *)scr);
}

// ---------------------------------------------------------------------------
// Router top-k + softmax over the selected logits (softmax_topk_v2.comp,
// topKSoftmax forward.zig:496-537). One wave; exact f32 comparisons with the
// lowest index winning ties. routing = [ids u32 x k][weights f32 x k].
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void k_softmax_topk(const float *logits, uint32_t n, uint32_t k, uint32_t *routing) {
    float vals[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t e = threadIdx.x + 64 * i;
        vals[i] = e < n ? logits[e] : -INFINITY;
    }
    topk_softmax_wave(vals, n, k, routing);
}

// f32 weights (a MoE router kept unquantised, as llama.cpp's quantiser leaves
// ffn_gate_inp): y[r] = sum_k W[r][k] x[k], one wave per row, each lane
// summing its 4-element chunks in order, then a fixed DPP reduction.
__global__ __launch_bounds__(256) void k_matvec_f32(const float *__restrict__ W, const float *__restrict__ x,
                                                    float *__restrict__ y, uint32_t M, uint32_t K) {
    const uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= M) return;  // uniform per wave
    const float *w = W + (size_t)r * K;
    float s = 0.f;
    for (uint32_t k = 4 * lane; k < K; k += 256) {
        const f32x4 a = *(const f32x4 *)(w + k), b = *(const f32x4 *)(x + k);
        s = fmaf(a.x, b.x, s);
        s = fmaf(a.y, b.y, s);
        s = fmaf(a.z, b.z, s);
        s = fmaf(a.w, b.w, s);
    }
    s = wave_sum(s);
    if (lane == 0) y[r] = s;
}

int zhk_matvec_f32(zh_ctx *c, const float *W, const float *x, float *y, uint32_t M, uint32_t K) {
    if (M == 0 || K % 4) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "matvec_f32 M %u K %u", M, K);
    hipLaunchKernelGGL(k_matvec_f32, dim3((M + 3) / 4), dim3(256), 0, c->stream, W, x, y, M, K);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

int zhk_softmax_topk(zh_ctx *c, const float *logits, uint32_t n, uint32_t k, uint32_t *routing) {
    hipLaunchKernelGGL(k_softmax_topk, dim3(1), dim3(64), 0, c->stream, logits, n, k, routing);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
extern "C" int zh_softmax_topk(zh_ctx *c, const zh_buf *logits, uint32_t n, uint32_t k, zh_buf *routing) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (n == 0 || n > 256 || k == 0 || k > 16 || k > n || !in_range(logits, 0, 4ull * n) ||
        !in_range(routing, 0, 8ull * k))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "softmax_topk shape");
    return zhk_softmax_topk(c, (const float *)logits->ptr, n, k, (uint32_t *)routing->ptr);
}

// moe_weighted_acc.comp:23-33
__global__ void k_moe_weighted_acc(float *a, const float *b, const uint32_t *routing, uint32_t n, uint32_t n_used,
                                   uint32_t stride) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float s = 0.f;
    for (uint32_t j = 0; j < n_used; j++) s += __uint_as_float(routing[n_used + j]) * b[(size_t)j * stride + i];
    a[i] += s;
}
int zhk_moe_weighted_acc(zh_ctx *c, float *a, const float *b, const uint32_t *routing, uint32_t n, uint32_t n_used,
                         uint32_t stride) {
    hipLaunchKernelGGL(k_moe_weighted_acc, dim3((n + 255) / 256), dim3(256), 0, c->stream, a, b, routing, n, n_used,
                       stride);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
extern "C" int zh_moe_weighted_acc(zh_ctx *c, zh_buf *a, const zh_buf *b, const zh_buf *routing, uint32_t n,
                                   uint32_t n_used, uint32_t src_stride) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (n == 0 || n_used == 0 || src_stride < n || !in_range(a, 0, 4ull * n) ||
        !in_range(b, 0, 4ull * ((uint64_t)(n_used - 1) * src_stride + n)) || !in_range(routing, 0, 8ull * n_used))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "moe_weighted_acc shape");
    return zhk_moe_weighted_acc(c, (float *)a->ptr, (const float *)b->ptr, (const uint32_t *)routing->ptr, n, n_used,
                                src_stride);
}

// ---------------------------------------------------------------------------
// Argmax: first (lowest-index) maximum; NaN never compares greater, as the
// reference's strict `>` scan (forward.zig:10348-10356).
// ---------------------------------------------------------------------------
constexpr int AM_WGS = 256;
__global__ __launch_bounds__(256) void k_argmax0(const float *__restrict__ x, uint32_t n, uint32_t *partials) {
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) am_better(bv, bi, x[i], i);
    am_wave(bv, bi);
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) am_better(bv, bi, sv[w], si[w]);
        partials[2 * blockIdx.x] = __float_as_uint(bv);
        partials[2 * blockIdx.x + 1] = bi;
    }
}
__global__ __launch_bounds__(256) void k_argmax1(const uint32_t *partials, uint32_t np, uint32_t *result,
                                                 uint32_t *ring, const uint32_t *ring_index) {
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t i = threadIdx.x; i < np; i += 256) am_better(bv, bi, __uint_as_float(partials[2 * i]), partials[2 * i + 1]);
    am_wave(bv, bi);
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
    if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = bv; si[threadIdx.x >> 6] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) am_better(bv, bi, sv[w], si[w]);
        if (bi == 0xFFFFFFFFu) bi = 0;  // all NaN: the scan keeps index 0
        result[0] = bi;
        if (ring) ring[ring_index[0]] = bi;
    }
}
int zhk_argmax(zh_ctx *c, const float *logits, uint32_t n, uint32_t *result, uint32_t *partials, uint32_t *ring,
               const uint32_t *ring_index) {
    uint32_t wgs = (n + 255) / 256 < AM_WGS ? (n + 255) / 256 : AM_WGS;
    hipLaunchKernelGGL(k_argmax0, dim3(wgs), dim3(256), 0, c->stream, logits, n, partials);
    ZH_LAUNCH_CHECK(c);
    hipLaunchKernelGGL(k_argmax1, dim3(1), dim3(256), 0, c->stream, (const uint32_t *)partials, wgs, result, ring,
                       ring_index);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
extern "C" int zh_argmax(zh_ctx *c, const zh_buf *logits, uint32_t n, zh_buf *result, uint64_t result_off) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (n == 0 || !in_range(logits, 0, 4ull * n) || !in_range(result, result_off, 4) || (result_off & 3))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "argmax range");
    void *scr;
    int rc = zh_scratch(c, AM_WGS * 8, &scr);
    if (rc) return rc;
    return zhk_argmax(c, (const float *)logits->ptr, n, DPTR(result, result_off, uint32_t), (uint32_t *)scr, nullptr,
                      nullptr);
}
