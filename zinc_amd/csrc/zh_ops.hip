// zh_ops.hip — RMSNorm, fused QK-norm/RoPE/KV write, split-context
// flash-decode with LSE merge, SwiGLU, MoE routing and argmax for gfx950.
#include "zh_device.h"
#include "zh_internal.h"

static bool in_range(const zh_buf *b, uint64_t off, uint64_t n) { return b && off <= b->size && n <= b->size - off; }
#define DPTR(b, off, T) ((T *)((char *)(b)->ptr + (off)))

// Quantise one 32-element block held one value per lane across a 32-lane
// group (l = lane index within the group) into XQ block `blk`.
ZH_DEV uint32_t read_pos(zh_pos_src p) { return p.dev ? (*p.dev + p.value) : p.value; }

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
#ifdef ZH_EXP_TRACE
__device__ uint64_t g_exp_trace_ops[16384 * 16];
#define TRACE_OPS(slot) do { const uint32_t bl_ = blockIdx.x + blockIdx.y * gridDim.x; \
    if (threadIdx.x == 0 && bl_ < 8192) g_exp_trace_ops[bl_ * 16 + (slot)] = __builtin_amdgcn_s_memrealtime(); } while (0)
extern "C" int zh_exp_trace_ops_dump(uint64_t *host, uint32_t n) {
    int rc = (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_exp_trace_ops), (size_t)n * 8, 0, hipMemcpyDeviceToHost);
    static uint64_t zeros[16384 * 16];
    return rc | (int)hipMemcpyToSymbol(HIP_SYMBOL(g_exp_trace_ops), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice);
}
#else
#define TRACE_OPS(slot) do { } while (0)
#endif
constexpr int FD_MAXG = 8;   // q heads per kv head
constexpr int FD_HD = 128;   // head_dim supported
// 4 waves x TW tokens: one wave per SIMD, and the 8 kv heads map one per XCD
// (workgroups go round robin over the 8 XCDs), so the chunks of a kv head
// spread over its XCD's 32 CUs. TW (tokens per wave per sub-chunk) is a
// template parameter chosen at launch:
//  * 24 when the context capacity is at most 8192 tokens: a 4K context then
//    runs 2 pipelined 96-token sub-chunks per workgroup over 22 chunks per
//    kv head (15.6 us per layer against 16.4 us for one 136-token chunk over
//    32 chunks: the second sub-chunk's K/V loads are in flight while the
//    first is computed, and fewer partials are merged);
//  * 32 for longer contexts: 128-token sub-chunks (32K context: 36.9 us
//    against 38.8 us with 96 and 40.2 us with 160);
//  * 40 for 8 q heads per kv head, which has no sub-chunk loop.
constexpr int AD_W = 4;      // waves per workgroup
constexpr int AD_T = AD_W * 64;
constexpr int AD_TC_MIN = AD_W * 24;  // the shortest sub-chunk: sizes the partials
// Chunk geometry modes: page-table lookups with chunk = blockIdx.y, the same
// dispatched newest-first (grids larger than the device), or an identity page
// table (physical token = logical token), where nothing waits on page entries
// and the chunk length follows the context: ceil(seq / nd) rounded up to 8
// tokens (at least TW) while that fits TC = 4 TW, with nd = CUs / kv heads, so
// the chunks of all kv heads cover the device once (32 per head for 8 kv
// heads: one XCD each).
enum { AD_PAGED = 0, AD_PAGED_REV = 1, AD_IDENT = 2 };
// Longer contexts: chunks of nsub consecutive TC-token sub-chunks (a
// workgroup runs them in turn with an online softmax), so a kv head never has
// more than nd chunks: the grid stays one round of one workgroup per CU (the
// kernel's registers allow one) and the merge reads at most nd partials.
ZH_DEV uint32_t attn_nsub(uint32_t seq, uint32_t nd, uint32_t tc) {
    const uint32_t span = nd * tc;
    return seq > span ? (seq + span - 1) / span : 1u;
}
ZH_DEV uint32_t attn_chunk_tokens(uint32_t seq, uint32_t nd, bool sub, uint32_t tw) {
    const uint32_t tc = AD_W * tw, ct = ((seq + nd - 1) / nd + 7) / 8 * 8;
    return seq > nd * tc ? tc * (sub ? attn_nsub(seq, nd, tc) : 1u) : max(ct, tw);
}
// Sub-chunks are compiled for up to 4 q heads per kv head (G = 8 would spill
// its loop-carried state); G = 8 keeps TC-token chunks at long contexts.
template <int G> constexpr bool attn_sub_ok() { return G <= 4; }
static uint32_t attn_nd(uint32_t nkv, int cu_count) {
    const uint32_t cu = cu_count > 0 && cu_count < 256 ? (uint32_t)cu_count : 256u;
    const uint32_t nd = cu / nkv > 0 ? cu / nkv : 1u;
    return nd < 256u ? nd : 256u;  // the merge keeps at most 256 chunk statistics in LDS
}
// chunk slots per head for sub-chunks of tc tokens (the partials, sized with
// the shortest, hold any; a device with at most 256 CUs fits)
static uint32_t attn_n_chunks(uint32_t max_seq, uint32_t nd, uint32_t tc = AD_TC_MIN) {
    const uint32_t n = (max_seq + tc - 1) / tc;
    return n > nd ? n : nd;
}

uint64_t zhk_flash_decode_partials_bytes(uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_seq) {
    // partials + two counter words per kv head (at most nh words)
    return (uint64_t)nh * attn_n_chunks(max_seq, attn_nd(nkv, 256)) * (hd + 2) * 4 + 4ull * nh + 256;
}

struct AttnP {
    const float *q;                // FUSED: raw Q projection; else prepared (normed, roped) q
    const float *k_new, *v_new;    // FUSED: raw K/V projection of the new token
    const float *q_norm, *k_norm;  // FUSED: per-head RMSNorm weights (128)
    const float *rope_cs;          // FUSED: [position][64] (cos, sin) pairs of pos * inv_freq
    uint16_t *kc, *vc;
    const uint32_t *pages;
    uint32_t n_pages, cache_tokens;
    zh_pos_src pos;  // FUSED: position of the new token (seq = pos + 1); else seq_len
    float scale, eps;
    float *part;     // [nq][n_chunks][130]
    uint32_t n_chunks;
    uint32_t *counters;  // [nkv], zero between launches
    float *out;          // [nq * 128]
    uint8_t *xq;         // optional XQ image of out
    uint32_t nq;
    uint32_t nd;         // AD_IDENT: target chunks per kv head
    uint32_t no_wait;    // the last arrival merges every q head (no merger waits for others)
};

ZH_DEV float sum8(float v) { return row8_sum(v); }  // over the 8 lanes of a token group

// RMSNorm (weights w) + NeoX RoPE on one head held as lo[e] = x[sub*8+e],
// hi[e] = x[64+sub*8+e] (qk_norm_rope_kv_write.comp:67-171 arithmetic).
ZH_DEV void norm_rope16(float (&lo)[8], float (&hi)[8], const float (&wlo)[8], const float (&whi)[8],
                        const float (&co)[8], const float (&sn)[8], float eps) {
    float sq = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) sq = fmaf(lo[e], lo[e], fmaf(hi[e], hi[e], sq));
    sq = sum8(sq);
    const float rms_inv = 1.0f / sqrtf(sq / (float)FD_HD + eps);
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float a = wlo[e] * (lo[e] * rms_inv);
        const float b = whi[e] * (hi[e] * rms_inv);
        lo[e] = a * co[e] - b * sn[e];
        hi[e] = a * sn[e] + b * co[e];
    }
}


// Two f32 -> packed f16 with the hardware conversion (round to nearest
// even; fp16 denormals are kept in this build's default FP mode), as the
// cache write's @floatCast.
ZH_DEV uint32_t pack_h2(float a, float b) {
    const _Float16 ha = (_Float16)a, hb = (_Float16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, ha) | ((uint32_t)__builtin_bit_cast(uint16_t, hb) << 16);
}

// Row o (0..47) of the three pages a wave reads, page bases pa, pb, pc.
ZH_DEV const uint16_t *kv_row(const uint16_t *h, size_t pa, size_t pb, size_t pc, uint32_t o) {
    const uint32_t pi = o >> 4;
    const size_t pg = pi == 0 ? pa : pi == 1 ? pb : pc;
    return h + (pg * 16 + (o & 15)) * FD_HD;
}

// Merges the chunk partials of q heads h0 .. h0+GM-1: O = sum_c exp(m_c - M) O_c
// / sum_c exp(m_c - M) l_c (the split-K combine of flash_decode.comp's
// reduction). NBAT chunks per round of O loads (every load is issued, with
// clamped addresses, so the wait counts stay static). Reads partials published at device scope; `poison` (a wait that
// timed out) turns the outputs into NaN.
template <int GM, int NBAT>
ZH_DEV void attn_merge(const AttnP &p, uint32_t h0, uint32_t nv, bool poison) {
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    TRACE_OPS(11);
    // Chunk merge. The first batch of each thread's O dims (NBAT chunks) is
    // requested before the chunk statistics, so both arrive in about one
    // round trip; the statistics pass leaves m_c in LDS for the weights.
    // dims per thread: power of two with G*128/OPT <= AD_T
    constexpr int OPT = GM * FD_HD <= AD_T ? 1 : GM * FD_HD <= 2 * AD_T ? 2 : GM * FD_HD <= 4 * AD_T ? 4 : 8;
    constexpr int NTH = GM * FD_HD / OPT;
    constexpr int MB = 256;                 // chunk statistics kept in LDS
    __shared__ __align__(16) float sm[GM][MB];
    __shared__ float hM[GM], hL[GM];
    __shared__ float ob[GM * FD_HD];
    float O[OPT];
#pragma unroll
    for (int k = 0; k < OPT; k++) O[k] = 0.f;
    const uint32_t g_t = min(tid * OPT / FD_HD, (uint32_t)GM - 1), d0 = (tid * OPT) % FD_HD;
    const float *pt = p.part + (size_t)(h0 + g_t) * p.n_chunks * (FD_HD + 2);
    float v[NBAT][OPT];
    auto load_o = [&](uint32_t cb) {
#pragma unroll
        for (int u = 0; u < NBAT; u++) {
            const float *pc = pt + (size_t)min(cb + u, nv - 1) * (FD_HD + 2) + d0;
            if (OPT == 1) {
                v[u][0] = ld_dev(pc);
            } else {
#pragma unroll
                for (int w = 0; w < OPT / 2; w++) {
                    const uint64_t x = ld_dev64(pc + 2 * w);
                    v[u][2 * w] = __uint_as_float((uint32_t)x);
                    v[u][2 * w + 1] = __uint_as_float((uint32_t)(x >> 32));
                }
            }
        }
    };
    const bool one_batch = nv <= (uint32_t)NBAT;  // uniform
    if (one_batch) load_o(0);
    asm volatile("" ::: "memory");  // the O loads go out before the statistics loads
    for (uint32_t g = wave; g < (uint32_t)GM; g += AD_W) {
        const float *pp = p.part + (size_t)(h0 + g) * p.n_chunks * (FD_HD + 2);
        float m = -INFINITY, l = 0.f;
        for (uint32_t c = lane; c < nv; c += 64) {
            const uint64_t ml = ld_dev64(pp + (size_t)c * (FD_HD + 2) + FD_HD);
            const float mc = __uint_as_float((uint32_t)ml), lc = __uint_as_float((uint32_t)(ml >> 32));
            if (c < MB) sm[g][c] = mc;
            const float mn = fmaxf(m, mc);
            l = fmaf(l, m == -INFINITY ? 0.f : expf(m - mn), lc * expf(mc - mn));
            m = mn;
        }
        const float M = wave_max(m);
        l = wave_sum(m == -INFINITY ? 0.f : l * expf(m - M));
        if (lane == 0) { hM[g] = M; hL[g] = l; }
    }
    TRACE_OPS(12);
    __syncthreads();
    TRACE_OPS(13);
    const float Mt = hM[g_t];
    if (one_batch) {
        // weights exp(m_c - M) once per (head, chunk), in place in LDS
        for (uint32_t i = tid; i < (uint32_t)GM * NBAT; i += AD_T) {
            const uint32_t g = i / NBAT, c = i % NBAT;
            sm[g][c] = c < nv ? expf(sm[g][c] - hM[g]) : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int u4 = 0; u4 < NBAT; u4 += 4) {
            const f32x4 w4 = *(const f32x4 *)&sm[g_t][u4];
#pragma unroll
            for (int k = 0; k < OPT; k++) {
                O[k] = fmaf(v[u4][k], w4.x, O[k]);
                O[k] = fmaf(v[u4 + 1][k], w4.y, O[k]);
                O[k] = fmaf(v[u4 + 2][k], w4.z, O[k]);
                O[k] = fmaf(v[u4 + 3][k], w4.w, O[k]);
            }
        }
    } else {
        // long contexts: one round of loads per NBAT chunks
        for (uint32_t cb = 0; cb < nv; cb += NBAT) {
            load_o(cb);
#pragma unroll
            for (int u = 0; u < NBAT; u++) {
                const uint32_t c = cb + u;
                const float mc = c < MB ? sm[g_t][c < MB ? c : 0] : ld_dev(pt + (size_t)min(c, nv - 1) * (FD_HD + 2) + FD_HD);
                const float wgt = c < nv ? expf(mc - Mt) : 0.f;
#pragma unroll
                for (int k = 0; k < OPT; k++) O[k] = fmaf(v[u][k], wgt, O[k]);
            }
        }
    }
    TRACE_OPS(6);
    if (tid < (uint32_t)NTH) {
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            const float r = poison ? __builtin_nanf("") : hL[g_t] > 0.f ? O[k] / hL[g_t] : 0.f;
            ob[tid * OPT + k] = r;
            if (p.out) p.out[(size_t)h0 * FD_HD + tid * OPT + k] = r;
        }
    }
    TRACE_OPS(7);
    if (p.xq) {
        __syncthreads();
        XQView v = xq_view(p.xq, p.nq * FD_HD / 32);
        for (uint32_t o = tid; o < (uint32_t)GM * FD_HD; o += AD_T)  // whole 32-lane groups (GM*128 % 32 == 0)
            xq_store_block32(ob[o], o & 31, v, (h0 * FD_HD + o) / 32);
    }
    TRACE_OPS(5);
}

template <int G, bool FUSED, int MODE, int TW>
__global__ __launch_bounds__(AD_T, 1) void k_attn_decode(AttnP p) {
    constexpr int TC = AD_W * TW;  // tokens per sub-chunk
    const uint32_t kvh = blockIdx.x, tid = threadIdx.x;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, sub = lane & 7, grp = lane >> 3;
    TRACE_OPS(0);
    static_assert(TW % 8 == 0 && TW + 8 <= 48, "a wave's tokens must fit 3 pages from an 8-aligned start");
    // Position: a branch-free read (a branch would wait for the load at its
    // join). AD_PAGED: the chunk is blockIdx.y, so the page entries (scalar
    // loads), the position and the q loads all go out at once. AD_PAGED_REV:
    // chunks are dispatched last-first so the chunk holding the newest tokens
    // (and, FUSED, the KV write) never waits in the dispatch tail; that order
    // needs the position first. AD_IDENT: no page entries; the geometry
    // follows the position (and is reversed the same way).
    const uint32_t pos_raw = *(p.pos.dev ? p.pos.dev : p.pages);
    const uint32_t posv = p.pos.dev ? pos_raw + p.pos.value : p.pos.value;
    const uint32_t seq = FUSED ? posv + 1 : posv;
    constexpr bool SUB = MODE == AD_IDENT && attn_sub_ok<G>();
    const uint32_t CT = MODE == AD_IDENT ? attn_chunk_tokens(seq, p.nd, SUB, TW) : (uint32_t)TC;
    const uint32_t nsub = SUB ? attn_nsub(seq, p.nd, TC) : 1u;  // TC-token sub-chunks per chunk
    uint32_t chunk = blockIdx.y;
    if (MODE != AD_PAGED) {
        const uint32_t nv_hint = (seq + CT - 1) / CT;
        chunk = blockIdx.y < nv_hint ? nv_hint - 1 - blockIdx.y : blockIdx.y;
    }
    const uint32_t t0 = chunk * CT, tw0 = t0 + wave * TW;
    // this wave's tokens within (each sub-chunk of) the chunk: a chunk
    // shorter than TC leaves the last waves fewer, or none
    const uint32_t wtok = CT > wave * TW ? min(CT - wave * TW, (uint32_t)TW) : 0u;
    const uint32_t pgb = tw0 / 16, o16 = tw0 & 15;
    uint32_t page0, page1, page2;
    if (MODE == AD_IDENT) {
        page0 = pgb; page1 = pgb + 1; page2 = pgb + 2;
    } else {
        page0 = p.pages[min(pgb, p.n_pages - 1)];
        page1 = p.pages[min(pgb + 1, p.n_pages - 1)];
        page2 = p.pages[min(pgb + 2, p.n_pages - 1)];
    }
    const uint16_t *kh = p.kc + (size_t)kvh * p.cache_tokens * FD_HD;
    const uint16_t *vh = p.vc + (size_t)kvh * p.cache_tokens * FD_HD;

    // ---- loads: q (and the new token's raw k/v) first, then K, then V
    float qlo[G][8], qhi[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float *qp = p.q + (size_t)(kvh * G + g) * FD_HD;
        const f32x4 a = *(const f32x4 *)(qp + sub * 8), b = *(const f32x4 *)(qp + sub * 8 + 4);
        const f32x4 c = *(const f32x4 *)(qp + 64 + sub * 8), d = *(const f32x4 *)(qp + 64 + sub * 8 + 4);
        qlo[g][0] = a.x; qlo[g][1] = a.y; qlo[g][2] = a.z; qlo[g][3] = a.w;
        qlo[g][4] = b.x; qlo[g][5] = b.y; qlo[g][6] = b.z; qlo[g][7] = b.w;
        qhi[g][0] = c.x; qhi[g][1] = c.y; qhi[g][2] = c.z; qhi[g][3] = c.w;
        qhi[g][4] = d.x; qhi[g][5] = d.y; qhi[g][6] = d.z; qhi[g][7] = d.w;
    }
    float klo[8], khi[8], vn0 = 0.f, vn1 = 0.f, vn8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (FUSED) {
        const float *kp = p.k_new + (size_t)kvh * FD_HD;
        const f32x4 a = *(const f32x4 *)(kp + sub * 8), b = *(const f32x4 *)(kp + sub * 8 + 4);
        const f32x4 c = *(const f32x4 *)(kp + 64 + sub * 8), d = *(const f32x4 *)(kp + 64 + sub * 8 + 4);
        klo[0] = a.x; klo[1] = a.y; klo[2] = a.z; klo[3] = a.w; klo[4] = b.x; klo[5] = b.y; klo[6] = b.z; klo[7] = b.w;
        khi[0] = c.x; khi[1] = c.y; khi[2] = c.z; khi[3] = c.w; khi[4] = d.x; khi[5] = d.y; khi[6] = d.z; khi[7] = d.w;
        const float2 vv = *(const float2 *)(p.v_new + (size_t)kvh * FD_HD + 2 * lane);
        vn0 = vv.x;
        vn1 = vv.y;
        const f32x4 va = *(const f32x4 *)(p.v_new + (size_t)kvh * FD_HD + 8 * (lane & 15));
        const f32x4 vb = *(const f32x4 *)(p.v_new + (size_t)kvh * FD_HD + 8 * (lane & 15) + 4);
        vn8[0] = va.x; vn8[1] = va.y; vn8[2] = va.z; vn8[3] = va.w;
        vn8[4] = vb.x; vn8[5] = vb.y; vn8[6] = vb.z; vn8[7] = vb.w;
    }
    float co[8], sn[8], qwl[8], qwh[8], kwl[8], kwh[8];
    if (FUSED) {
        const f32x4 *w4 = (const f32x4 *)(p.q_norm + sub * 8), *w5 = (const f32x4 *)(p.q_norm + 64 + sub * 8);
        const f32x4 *w6 = (const f32x4 *)(p.k_norm + sub * 8), *w7 = (const f32x4 *)(p.k_norm + 64 + sub * 8);
#pragma unroll
        for (int h2 = 0; h2 < 2; h2++) {
            const f32x4 a = w4[h2], b = w5[h2], c = w6[h2], d = w7[h2];
            qwl[4 * h2] = a.x; qwl[4 * h2 + 1] = a.y; qwl[4 * h2 + 2] = a.z; qwl[4 * h2 + 3] = a.w;
            qwh[4 * h2] = b.x; qwh[4 * h2 + 1] = b.y; qwh[4 * h2 + 2] = b.z; qwh[4 * h2 + 3] = b.w;
            kwl[4 * h2] = c.x; kwl[4 * h2 + 1] = c.y; kwl[4 * h2 + 2] = c.z; kwl[4 * h2 + 3] = c.w;
            kwh[4 * h2] = d.x; kwh[4 * h2 + 1] = d.y; kwh[4 * h2 + 2] = d.z; kwh[4 * h2 + 3] = d.w;
        }
    }
    // The loads above need neither the position nor the page entries (both
    // scalar loads in flight meanwhile); a chunk past the sequence ends here.
    asm volatile("" ::: "memory");
    if (t0 >= seq) return;  // uniform over the workgroup
    const uint32_t nt = seq > tw0 ? min(seq - tw0, wtok) : 0u;
    if (FUSED) {
        const f32x4 *cs = (const f32x4 *)(p.rope_cs + ((size_t)posv * 64 + sub * 8) * 2);
#pragma unroll
        for (int e2 = 0; e2 < 4; e2++) {
            const f32x4 t = cs[e2];
            co[2 * e2] = t.x; sn[2 * e2] = t.y; co[2 * e2 + 1] = t.z; sn[2 * e2 + 1] = t.w;
        }
    }
    // Memory returns in issue order: keep the compiler from interleaving or
    // sinking the groups (q / new token / RoPE first, then K, then V), so the
    // q preparation (after the K and V loads are issued) waits only for its
    // own loads.
    asm volatile("" ::: "memory");
    __shared__ float ps[AD_W][G][TW];
    __shared__ float wm[AD_W][G], wl[AD_W][G];
    __shared__ float wo[AD_W][4][G][FD_HD];  // per wave and token row
    const uint32_t vrow = lane >> 4, vcol = lane & 15;
    const uint32_t ptok = p.cache_tokens / 16;
    // online softmax state of this wave over its sub-chunks (per q head):
    // running maximum, sum of exp and P*V (lane = token row vrow, dims 8 vcol..)
    float m_run[G], l_run[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m_run[g] = -INFINITY;
        l_run[g] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.f;
    }
    // K/V rows of this wave's tokens in sub-chunk i (sub-chunk 0: the page
    // entries computed above; later sub-chunks exist only with the identity
    // page table): up to three 16-token pages, each a contiguous 4 KB run, so
    // every row is an offset from a page base that is uniform per 8-token
    // pass. Rows past the end of the sequence are read (in-bounds) and masked.
    // V: lane = (vrow = lane / 16, vcol = lane % 16) holds dims 8 vcol ..
    // 8 vcol + 7 of the wave's tokens vrow, vrow + 4, .., 36 + vrow: 16-byte
    // loads, one instruction covering 4 tokens x 256 B (4 tokens from a
    // 4-aligned offset never straddle a 16-token page). Sub-chunk i + 1's K
    // loads go out once sub-chunk i's scores are computed, its V loads once
    // sub-chunk i's P*V is done, in the same registers.
    u32x4 kr[TW / 8][2];
    u32x4 vr[TW / 4];
    auto pages_of = [&](uint32_t i, uint32_t &pg0, uint32_t &pg1, uint32_t &pg2, uint32_t &pgbs)
        __attribute__((always_inline)) {
        pg0 = page0; pg1 = page1; pg2 = page2; pgbs = pgb;
        if (i) {
            pgbs = (tw0 + i * TC) / 16;
            pg0 = pgbs; pg1 = pgbs + 1; pg2 = pgbs + 2;
        }
    };
    auto load_k = [&](uint32_t i) __attribute__((always_inline)) {
        uint32_t g0, g1, g2, gb;
        pages_of(i, g0, g1, g2, gb);
        const size_t pa = g0 < ptok ? g0 : 0u, pb = g1 < ptok ? g1 : 0u, pc = g2 < ptok ? g2 : 0u;
#pragma unroll
        for (int j = 0; j < TW / 8; j++) {
            // o16 + 8j is 8-aligned: the pass stays in one page
            const uint16_t *kp = kv_row(kh, pa, pb, pc, o16 + 8 * j) + grp * FD_HD;
            kr[j][0] = *(const u32x4 *)(kp + sub * 8);
            kr[j][1] = *(const u32x4 *)(kp + 64 + sub * 8);
        }
    };
    auto load_v = [&](uint32_t i) __attribute__((always_inline)) {
        uint32_t g0, g1, g2, gb;
        pages_of(i, g0, g1, g2, gb);
        const size_t pa = g0 < ptok ? g0 : 0u, pb = g1 < ptok ? g1 : 0u, pc = g2 < ptok ? g2 : 0u;
#pragma unroll
        for (int k = 0; k < TW / 4; k++)
            vr[k] = *(const u32x4 *)(kv_row(vh, pa, pb, pc, o16 + 4 * k + vrow) + 8 * vcol);
    };
    load_k(0);
    asm volatile("" ::: "memory");
    load_v(0);
    asm volatile("" ::: "memory");
    // ---- q preparation (once per workgroup), while K and V are in flight
    if (FUSED) {
#pragma unroll
        for (int g = 0; g < G; g++) norm_rope16(qlo[g], qhi[g], qwl, qwh, co, sn, p.eps);
    }

    // ---- the new token: its position lies in exactly one wave's range of
    // one sub-chunk (s_own); that wave writes it to the cache here, once, and
    // its scores and P*V select these values for it instead of the cache rows
    // loaded for that position (which predate the write)
    uint32_t s_own = ~0u, inew = 0;  // uniform per wave
    u32x4 n0 = {0, 0, 0, 0}, n1 = {0, 0, 0, 0}, vnew4 = {0, 0, 0, 0};
    if (FUSED && posv >= tw0) {
        const uint32_t rel = posv - tw0;
        if (rel % TC < wtok && rel / TC < nsub) {
            s_own = rel / TC;
            inew = rel % TC;
            norm_rope16(klo, khi, kwl, kwh, co, sn, p.eps);
            n0 = u32x4{pack_h2(klo[0], klo[1]), pack_h2(klo[2], klo[3]), pack_h2(klo[4], klo[5]),
                       pack_h2(klo[6], klo[7])};
            n1 = u32x4{pack_h2(khi[0], khi[1]), pack_h2(khi[2], khi[3]), pack_h2(khi[4], khi[5]),
                       pack_h2(khi[6], khi[7])};
            const uint32_t vnew = pack_h2(vn0, vn1);
            vnew4 = u32x4{pack_h2(vn8[0], vn8[1]), pack_h2(vn8[2], vn8[3]), pack_h2(vn8[4], vn8[5]),
                          pack_h2(vn8[6], vn8[7])};
            // logicalTokenToPhysicalToken for the new position, from the page
            // entries of its sub-chunk (the position lies in page pgbs + 0..2);
            // the host has checked the context length, an unmapped slot is
            // skipped
            uint32_t pg0, pg1, pg2, pgbs;
            pages_of(s_own, pg0, pg1, pg2, pgbs);
            const uint32_t slot = posv / 16, pi = slot - pgbs;
            const uint32_t pg = pi == 0 ? pg0 : pi == 1 ? pg1 : pg2;
            const uint32_t ph = slot < p.n_pages ? pg * 16 + posv % 16 : p.cache_tokens;
            if (ph < p.cache_tokens) {
                if (grp == (inew & 7)) {
                    *(u32x4 *)(p.kc + ((size_t)kvh * p.cache_tokens + ph) * FD_HD + sub * 8) = n0;
                    *(u32x4 *)(p.kc + ((size_t)kvh * p.cache_tokens + ph) * FD_HD + 64 + sub * 8) = n1;
                }
                *(uint32_t *)(p.vc + ((size_t)kvh * p.cache_tokens + ph) * FD_HD + 2 * lane) = vnew;
            }
        }
    }
    TRACE_OPS(1);

    // One sub-chunk. PF: the next sub-chunk's K loads go out once this one's
    // scores are computed, its V loads once this one's P*V is done. The loads
    // are unconditional inside the loop (the last sub-chunk is peeled off), so
    // the compiler's waits count exactly the loads in flight: the scores wait
    // for this sub-chunk's K only, P*V for its V only.
    auto body = [&](uint32_t sc_i, auto pf) __attribute__((always_inline)) {
        constexpr bool PF = decltype(pf)::value;
        const uint32_t tws = tw0 + sc_i * TC;
        const uint32_t nts = seq > tws ? min(seq - tws, wtok) : 0u;
        const bool owner = sc_i == s_own;  // uniform per wave

        // ---- scores: token 8j + grp, 16 dims per lane, reduced over 8 lanes
        float sc[TW / 8][G];
#pragma unroll
        for (int j = 0; j < TW / 8; j++) {
            const bool sel = owner && (uint32_t)(8 * j) + grp == inew;
            const u32x4 k0 = sel ? n0 : kr[j][0], k1 = sel ? n1 : kr[j][1];
            const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
            float kf[16];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                kf[2 * e] = h2f(kw[e]);
                kf[2 * e + 1] = h2f(kw[e] >> 16);
            }
            const bool valid = (uint32_t)(8 * j) + grp < nts;
#pragma unroll
            for (int g = 0; g < G; g++) {
                float sacc = 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    sacc = fmaf(qlo[g][e], kf[e], sacc);
                    sacc = fmaf(qhi[g][e], kf[8 + e], sacc);
                }
                sacc = sum8(sacc) * p.scale;  // dot * scale, as cpuAttention
                sc[j][g] = valid ? sacc : -INFINITY;
            }
        }
        if (sc_i == 0) TRACE_OPS(2);
        if (PF) {
            asm volatile("" ::: "memory");
            load_k(sc_i + 1);
            asm volatile("" ::: "memory");
        }
        // ---- online softmax: new running maximum, rescale the old state
#pragma unroll
        for (int g = 0; g < G; g++) {
            float m = sc[0][g];
#pragma unroll
            for (int j = 1; j < TW / 8; j++) m = fmaxf(m, sc[j][g]);
            m = rows_max(fmaxf(m, dpp_f<0x140>(m)));  // m is uniform within each 8-lane token group
            const float mn = fmaxf(m_run[g], m);
            const float ms = mn == -INFINITY ? 0.f : mn;  // no valid token yet
            const float f = m_run[g] == -INFINITY ? 0.f : expf(m_run[g] - ms);
            float l = 0.f;
#pragma unroll
            for (int j = 0; j < TW / 8; j++) {
                const float pr = expf(sc[j][g] - ms);
                if (sub == 0) ps[wave][g][8 * j + grp] = pr;
                l += pr;
            }
            l = rows_sum(l + dpp_f<0x140>(l));
            l_run[g] = fmaf(l_run[g], f, l);
            m_run[g] = mn;
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] *= f;
        }
        __syncthreads();
        if (sc_i == 0) TRACE_OPS(8);
#pragma unroll
        for (int k = 0; k < TW / 4; k++) {
            const uint32_t i = 4 * k + vrow;
            u32x4 v = owner && i == inew ? vnew4 : vr[k];
            if (i >= nts) v = u32x4{0, 0, 0, 0};  // rows past the end may hold anything
            const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
            float vf[8];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                vf[2 * e] = h2f(vw[e]);
                vf[2 * e + 1] = h2f(vw[e] >> 16);
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float q = ps[wave][g][i];
#pragma unroll
                for (int e = 0; e < 8; e++) acc[g][e] = fmaf(q, vf[e], acc[g][e]);
            }
        }
        if (PF) {
            asm volatile("" ::: "memory");
            load_v(sc_i + 1);
            asm volatile("" ::: "memory");
        }
        __syncthreads();  // ps is rewritten by the next sub-chunk
    };
    if (SUB) {
        for (uint32_t sc_i = 0; sc_i + 1 < nsub; sc_i++) body(sc_i, std::true_type{});  // uniform
    }
    body(nsub - 1, std::false_type{});
#pragma unroll
    for (int g = 0; g < G; g++) {
        if (lane == 0) { wm[wave][g] = m_run[g]; wl[wave][g] = l_run[g]; }
        *(f32x4 *)&wo[wave][vrow][g][8 * vcol] = f32x4{acc[g][0], acc[g][1], acc[g][2], acc[g][3]};
        *(f32x4 *)&wo[wave][vrow][g][8 * vcol + 4] = f32x4{acc[g][4], acc[g][5], acc[g][6], acc[g][7]};
    }
    __syncthreads();
    TRACE_OPS(9);
    // ---- combine the 4 waves: per-head weights once, then thread -> (head, dim)
    __shared__ float cf[AD_W][G], cM[G], cL[G];
    if (tid < (uint32_t)G) {
        const uint32_t g = tid;
        float M = wm[0][g];
#pragma unroll
        for (int w = 1; w < AD_W; w++) M = fmaxf(M, wm[w][g]);
        const float Ms = M == -INFINITY ? 0.f : M;
        float L = 0.f;
#pragma unroll
        for (int w = 0; w < AD_W; w++) {
            const float f = wm[w][g] == -INFINITY ? 0.f : expf(wm[w][g] - Ms);
            cf[w][g] = f;
            L = fmaf(wl[w][g], f, L);
        }
        cM[g] = M;
        cL[g] = L;
    }
    __syncthreads();
    TRACE_OPS(10);
    for (uint32_t o = tid; o < (uint32_t)G * FD_HD; o += AD_T) {
        const uint32_t g = o / FD_HD, d = o % FD_HD;
        float O = 0.f;
#pragma unroll
        for (int w = 0; w < AD_W; w++)
            O = fmaf((wo[w][0][g][d] + wo[w][1][g][d]) + (wo[w][2][g][d] + wo[w][3][g][d]), cf[w][g], O);
        float *pp = p.part + ((size_t)(kvh * G + g) * p.n_chunks + chunk) * (FD_HD + 2);
        st_dev(pp + d, O);
        if (d == 0) { st_dev(pp + FD_HD, cM[g]); st_dev(pp + FD_HD + 1, cL[g]); }
    }
    TRACE_OPS(3);
    // ---- the last arrivals of this kv head merge the chunks
    const uint32_t nv = (seq + CT - 1) / CT;
    __shared__ uint32_t s_prev;
    // The partials went out as device-scope stores, coherent across the
    // XCDs' L2s. Waiting for them to complete (s_waitcnt 0 in every wave,
    // then the barrier) before a relaxed device-scope counter increment
    // publishes them without the full L2 write-back / invalidate that
    // agent-scope release / acquire fences imply; the readers use
    // device-scope loads.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) s_prev = __hip_atomic_fetch_add(p.counters + kvh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    TRACE_OPS(4);
    const uint32_t prev = s_prev;
    // With at least G chunks the last G arrivals merge one q head each (a
    // merger reads 1/G of the partials); otherwise the last arrival merges all.
    // (no_wait: other kernels share the device, so the earlier mergers'
    // bounded wait could wait on chunks that are not resident.)
    const bool split = G > 1 && nv >= (uint32_t)G && !p.no_wait;
    const uint32_t nm = split ? (uint32_t)G : 1u;
    if (prev + nm < nv) return;
    const uint32_t slot = prev + nm - nv;  // nm - 1: the last arrival
    if (!split) {
        attn_merge<G, G <= 4 ? 40 : 12>(p, kvh * G, nv, false);
        if (tid == 0) __hip_atomic_store(p.counters + kvh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // earlier mergers wait until every chunk has arrived; the wait is bounded
    // (50 ms) and a timeout poisons this head's output instead of hanging
    __shared__ uint32_t s_ok;
    if (tid == 0) {
        uint32_t ok = 1;
        if (slot != nm - 1) {
            const uint64_t t_0 = __builtin_amdgcn_s_memrealtime();
            while (__hip_atomic_load(p.counters + kvh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < nv) {
                if (__builtin_amdgcn_s_memrealtime() - t_0 > 5000000ull) { ok = 0; break; }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        s_ok = ok;
        // counters[nkv + kvh] counts mergers past the wait; the last one
        // clears both words for the next launch (no one reads them after)
        uint32_t *done = p.counters + gridDim.x + kvh;
        if (__hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nm - 1) {
            __hip_atomic_store(p.counters + kvh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __syncthreads();
    if (nv <= 32) attn_merge<1, 32>(p, kvh * G + slot, nv, !s_ok);
    else attn_merge<1, 64>(p, kvh * G + slot, nv, !s_ok);
}

// partials: zhk_flash_decode_partials_bytes(nh, nkv, hd, max_seq) bytes; the
// counter words at its end must be zero before the first launch (each
// launch leaves them zero).
static int attn_launch(zh_ctx *c, const AttnP &p0, uint32_t nkv, uint32_t G, uint32_t max_seq, bool fused,
                       bool ident) {
    AttnP p = p0;
    p.nd = attn_nd(nkv, c->cu_count);
    p.no_wait = c->concurrent ? 1u : 0u;
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

int zhk_flash_decode(zh_ctx *c, const float *q, const uint16_t *kc, const uint16_t *vc, const uint32_t *pages,
                     uint32_t n_pages, uint32_t cache_tokens, float *out, void *xq_out, uint32_t nh, uint32_t nkv,
                     uint32_t hd, zh_pos_src seq_len, uint32_t max_seq, float scale, float *partials) {
    AttnP p = {};
    p.q = q; p.kc = (uint16_t *)kc; p.vc = (uint16_t *)vc; p.pages = pages; p.n_pages = n_pages;
    p.cache_tokens = cache_tokens; p.pos = seq_len; p.scale = scale; p.part = partials;
    p.counters = attn_counters(partials, nh, nkv, hd, max_seq); p.out = out; p.xq = (uint8_t *)xq_out; p.nq = nh;
    return attn_launch(c, p, nkv, nh / nkv, max_seq, false, false);
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
    return attn_launch(c, p, nkv, nh / nkv, max_seq, true, ident_pages);
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
    int rc = zh_scratch(c, zhk_flash_decode_partials_bytes(nh, nkv, hd, seq_len), &scr);
    if (rc) return rc;
    ZH_HIP(c, hipMemsetAsync(attn_counters((float *)scr, nh, nkv, hd, seq_len), 0, 4ull * nh, c->stream));
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
ZH_DEV void am_better(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}
ZH_DEV void am_wave(float &bv, uint32_t &bi) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(bv, o, 64);
        uint32_t oi = (uint32_t)__shfl_xor((int)bi, o, 64);
        am_better(bv, bi, ov, oi);
    }
}
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
