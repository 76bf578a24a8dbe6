// zh_ops.hip — RMSNorm, fused QK-norm/RoPE/KV write, split-context
// flash-decode with LSE merge, SwiGLU, MoE routing and argmax for gfx950.
#include "zh_device.h"
#include "zh_internal.h"

static bool in_range(const zh_buf *b, uint64_t off, uint64_t n) { return b && off <= b->size && n <= b->size - off; }
#define DPTR(b, off, T) ((T *)((char *)(b)->ptr + (off)))

// Quantise one 32-element block held one value per lane across a 32-lane
// group (l = lane index within the group) into XQ block `blk`.
ZH_DEV void xq_store_block32(float xi, int l, XQView v, uint32_t blk) {
    float a = fabsf(xi);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 32));
    float inv, sc;
    xq_scales(a, inv, sc);
    int X = xq_quant(xi, inv);
    int l0, l1, l2;
    xq_limbs(X, l0, l1, l2);
    v.limb[blk * 96 + l] = (int8_t)l0;
    v.limb[blk * 96 + 32 + l] = (int8_t)l1;
    v.limb[blk * 96 + 64 + l] = (int8_t)l2;
    int s = X;
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 32);
    if (l == 0) v.xs[blk] = sc;
    if ((l & 15) == 0) v.xsum[blk * 2 + (l >> 4)] = (float)s * sc;
}

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
                                                        zh_pos_src pos_src, float eps) {
    const uint32_t wg = blockIdx.x, lane = threadIdx.x;
    const bool is_q = wg < nq;
    const uint32_t head = is_q ? wg : wg - nq;
    const float *src = is_q ? q + (size_t)head * hd : k + (size_t)head * hd;
    const float *wt = is_q ? qw : kw;
    const uint32_t pos = read_pos(pos_src);
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
                        uint32_t cache_tokens, uint32_t nq, uint32_t nkv, uint32_t hd, zh_pos_src pos, float eps) {
    hipLaunchKernelGGL(k_qk_norm_rope_kv, dim3(nq + nkv), dim3(64), 0, c->stream, q, qw, k, kw, v, inv_freq, kc, vc,
                       pages, n_pages, cache_tokens, nq, hd, pos, eps);
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
// Flash-decode. Grid (n_kv_heads, n_chunks): workgroup (h, c) handles the
// GQA group of kv head h over tokens [c*C, c*C+C) and writes, per q head,
// the chunk's unnormalised output O, running max m and denominator l.
// A merge kernel combines chunks with log-sum-exp weights.
// Cache layout [kv_head][token][head_dim] fp16, read through 16-token pages.
// ---------------------------------------------------------------------------
constexpr int FD_MAXG = 8;     // q heads per kv head (GQA group) handled per wave
constexpr int FD_HD = 128;     // head_dim supported by the kernel
constexpr int FD_T = 32;       // tokens per chunk; one wave per (kv head, chunk)

uint64_t zhk_flash_decode_partials_bytes(uint32_t nh, uint32_t hd, uint32_t max_seq) {
    return (uint64_t)nh * ((max_seq + FD_T - 1) / FD_T) * (hd + 2) * 4 + 256;
}

// One wave = one (kv head, 32-token chunk): all K and V loads are issued up
// front (16 KB per wave, one memory latency), scores use 8 lanes per token
// (16 dims each), the chunk softmax stays in registers, and P*V runs with
// lane = 2 output dims. Writes unnormalised O, chunk max m and sum l per q head.
template <int G>
__global__ __launch_bounds__(64) void k_flash_decode(const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                                     const uint16_t *__restrict__ vc,
                                                     const uint32_t *__restrict__ pages, uint32_t n_pages,
                                                     uint32_t cache_tokens, uint32_t n_chunks, zh_pos_src seq_src,
                                                     float scale, float *__restrict__ part) {
    const uint32_t kvh = blockIdx.x, chunk = blockIdx.y, lane = threadIdx.x;
    const uint32_t seq_len = read_pos(seq_src);
    const uint32_t t0 = chunk * FD_T;
    if (t0 >= seq_len) return;
    const uint32_t nt = min(t0 + FD_T, seq_len) - t0;
    const uint32_t sub = lane & 7, grp = lane >> 3;
    const uint16_t *kh = kc + (size_t)kvh * cache_tokens * FD_HD;
    const uint16_t *vh = vc + (size_t)kvh * cache_tokens * FD_HD;
    auto phys_of = [&](uint32_t i) -> uint32_t {
        uint32_t t = t0 + (i < nt ? i : nt - 1), pg = t / 16;
        uint32_t ph = (pg < n_pages) ? pages[pg] * 16 + t % 16 : 0;
        return ph < cache_tokens ? ph : 0;
    };
    // K: pass j covers tokens 8j + grp; lane reads dims sub*16 .. +15 (32 B)
    u32x4 kr[FD_T / 8][2];
#pragma unroll
    for (int j = 0; j < FD_T / 8; j++) {
        const u32x4 *kp = (const u32x4 *)(kh + (size_t)phys_of(8 * j + grp) * FD_HD + sub * 16);
        kr[j][0] = kp[0];
        kr[j][1] = kp[1];
    }
    // V: token i, dims 2*lane, 2*lane+1
    uint32_t vr[FD_T];
#pragma unroll
    for (int i = 0; i < FD_T; i++) vr[i] = *(const uint32_t *)(vh + (size_t)phys_of(i) * FD_HD + 2 * lane);
    // q for this lane's 16 dims, pre-scaled
    float qf[G][16];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const f32x4 *qp = (const f32x4 *)(q + (size_t)(kvh * G + g) * FD_HD + sub * 16);
#pragma unroll
        for (int e4 = 0; e4 < 4; e4++) {
            f32x4 t = qp[e4];
            qf[g][4 * e4 + 0] = t.x * scale; qf[g][4 * e4 + 1] = t.y * scale;
            qf[g][4 * e4 + 2] = t.z * scale; qf[g][4 * e4 + 3] = t.w * scale;
        }
    }
    // scores s[j][g] for token 8j + grp (replicated over the 8 lanes of grp)
    float sc[FD_T / 8][G];
#pragma unroll
    for (int j = 0; j < FD_T / 8; j++) {
        uint32_t kw[8] = {kr[j][0].x, kr[j][0].y, kr[j][0].z, kr[j][0].w,
                          kr[j][1].x, kr[j][1].y, kr[j][1].z, kr[j][1].w};
        float kf[16];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            kf[2 * e] = h2f(kw[e]);
            kf[2 * e + 1] = h2f(kw[e] >> 16);
        }
        const bool valid = (uint32_t)(8 * j) + grp < nt;
#pragma unroll
        for (int g = 0; g < G; g++) {
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < 16; e++) s = fmaf(qf[g][e], kf[e], s);
            s += __shfl_xor(s, 1, 64);
            s += __shfl_xor(s, 2, 64);
            s += __shfl_xor(s, 4, 64);
            sc[j][g] = valid ? s : -INFINITY;
        }
    }
    // chunk softmax per head: max and sum over passes and the 8 groups
    __shared__ float ps[G][FD_T];
    float mx[G], ls[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        float m = sc[0][g];
#pragma unroll
        for (int j = 1; j < FD_T / 8; j++) m = fmaxf(m, sc[j][g]);
        m = fmaxf(m, __shfl_xor(m, 8, 64));
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        float l = 0.f;
#pragma unroll
        for (int j = 0; j < FD_T / 8; j++) {
            float p = expf(sc[j][g] - m);  // exp(-inf) = 0 for invalid tokens
            if (sub == 0) ps[g][8 * j + grp] = p;
            l += p;
        }
        l += __shfl_xor(l, 8, 64);
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        mx[g] = m;
        ls[g] = l;
    }
    __syncthreads();  // single wave: orders the LDS probability writes
    float acc[G][2];
#pragma unroll
    for (int g = 0; g < G; g++) acc[g][0] = acc[g][1] = 0.f;
#pragma unroll
    for (int i = 0; i < FD_T; i++) {
        const float v0 = h2f(vr[i]), v1 = h2f(vr[i] >> 16);
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float p = ps[g][i];
            acc[g][0] = fmaf(p, v0, acc[g][0]);
            acc[g][1] = fmaf(p, v1, acc[g][1]);
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
        float *pp = part + ((size_t)(kvh * G + g) * n_chunks + chunk) * (FD_HD + 2);
        *(float2 *)(pp + 2 * lane) = make_float2(acc[g][0], acc[g][1]);
        if (lane == 0) { pp[FD_HD] = mx[g]; pp[FD_HD + 1] = ls[g]; }
    }
}

// LSE merge: one 256-thread workgroup per q head. Chunk statistics are read
// in parallel, then each (dim, chunk-quarter) thread accumulates its share.
__global__ __launch_bounds__(256) void k_flash_merge(const float *__restrict__ part, uint32_t n_chunks, uint32_t C,
                                                     zh_pos_src seq_src, float *__restrict__ out, uint8_t *xq) {
    const uint32_t h = blockIdx.x, tid = threadIdx.x;
    const uint32_t seq_len = read_pos(seq_src);
    const uint32_t nv = min(n_chunks, (seq_len + C - 1) / C);
    const float *pp = part + (size_t)h * n_chunks * (FD_HD + 2);
    __shared__ float wsh[1024];
    __shared__ float red[4];
    __shared__ float osum[2][FD_HD];
    // chunk maxima
    float m = -INFINITY;
    for (uint32_t c = tid; c < nv; c += 256) m = fmaxf(m, pp[c * (FD_HD + 2) + FD_HD]);
    m = wave_max(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float l = 0.f;
    for (uint32_t c = tid; c < nv; c += 256) {
        float w = expf(pp[c * (FD_HD + 2) + FD_HD] - M);
        wsh[c] = w;
        l = fmaf(pp[c * (FD_HD + 2) + FD_HD + 1], w, l);
    }
    l = wave_sum(l);
    if ((tid & 63) == 0) red[tid >> 6] = l;
    __syncthreads();
    const float L = red[0] + red[1] + red[2] + red[3];
    // O: thread (d, half) sums chunks c = half, half+2, ...
    const uint32_t d = tid & (FD_HD - 1), half = tid >> 7;
    float O = 0.f;
#pragma unroll 8
    for (uint32_t c = half; c < nv; c += 2) O = fmaf(pp[c * (FD_HD + 2) + d], wsh[c], O);
    osum[half][d] = O;
    __syncthreads();
    if (tid < FD_HD) {
        float o = L > 0.f ? (osum[0][tid] + osum[1][tid]) / L : 0.f;
        out[(size_t)h * FD_HD + tid] = o;
        if (xq) {
            XQView v = xq_view(xq, gridDim.x * FD_HD / 32);
            xq_store_block32(o, tid & 31, v, (h * FD_HD + tid) / 32);
        }
    }
}

int zhk_flash_decode(zh_ctx *c, const float *q, const uint16_t *kc, const uint16_t *vc, const uint32_t *pages,
                     uint32_t n_pages, uint32_t cache_tokens, float *out, void *xq_out, uint32_t nh, uint32_t nkv,
                     uint32_t hd, zh_pos_src seq_len, uint32_t max_seq, float scale, float *partials) {
    const uint32_t G = nh / nkv;
    const uint32_t C = FD_T;
    const uint32_t n_chunks = (max_seq + C - 1) / C;
    if (n_chunks > 1024) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "context too long for merge (%u chunks)", n_chunks);
    dim3 grid(nkv, n_chunks);
#define FD_LAUNCH(GG)                                                                                              \
    hipLaunchKernelGGL(k_flash_decode<GG>, grid, dim3(64), 0, c->stream, q, kc, vc, pages, n_pages, cache_tokens, \
                       n_chunks, seq_len, scale, partials)
    switch (G) {
    case 1: FD_LAUNCH(1); break;
    case 2: FD_LAUNCH(2); break;
    case 4: FD_LAUNCH(4); break;
    case 8: FD_LAUNCH(8); break;
    default: return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "GQA group %u unsupported (1, 2, 4, 8)", G);
    }
#undef FD_LAUNCH
    ZH_LAUNCH_CHECK(c);
    hipLaunchKernelGGL(k_flash_merge, dim3(nh), dim3(256), 0, c->stream, (const float *)partials, n_chunks, C,
                       seq_len, out, (uint8_t *)xq_out);
    ZH_LAUNCH_CHECK(c);
    (void)hd;
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
    int rc = zh_scratch(c, zhk_flash_decode_partials_bytes(nh, hd, seq_len), &scr);
    if (rc) return rc;
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
    const uint32_t lane = threadIdx.x;
    float vals[4];
    bool avail[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t e = lane + 64 * i;
        avail[i] = e < n;
        vals[i] = avail[i] ? logits[e] : -INFINITY;
    }
    __shared__ float sel[16];
    for (uint32_t j = 0; j < k; j++) {
        // best remaining (value desc, index asc) in this lane
        float bv = -INFINITY;
        uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (avail[i] && (bi == 0xFFFFFFFFu || vals[i] > bv)) { bv = vals[i]; bi = lane + 64 * i; }
        float m = bv;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            float ov = __shfl_xor(m, o, 64);
            m = (ov > m || m != m) ? ov : m;
        }
        uint32_t cand = (bi != 0xFFFFFFFFu && bv == m) ? bi : 0xFFFFFFFFu;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) cand = min(cand, (uint32_t)__shfl_xor((int)cand, o, 64));
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (lane + 64 * i == cand) avail[i] = false;
        if (lane == 0) {
            routing[j] = cand;
            sel[j] = m;
        }
    }
    __syncthreads();
    float mx = sel[0];
    float my = lane < k ? expf(sel[lane] - mx) : 0.f;
    float s = wave_sum(my);
    if (lane < k) ((float *)routing)[k + lane] = my / s;
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
