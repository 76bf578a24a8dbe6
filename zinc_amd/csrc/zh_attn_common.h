// zh_attn_common.h — decode-attention pieces shared by the attention
// kernels (zh_ops.hip) and the persistent decode-layers kernel
// (zh_step.hip): geometry, the kernel parameter block, the per-head
// norm + RoPE, the chunk merge, and the DMA-ring attention body.
#pragma once
#include "zh_device.h"
#include "zh_internal.h"

#pragma clang diagnostic ignored "-Winline-asm"

ZH_DEV uint32_t read_pos(zh_pos_src p) { return p.dev ? (*p.dev + p.value) : p.value; }

#ifndef TRACE_OPS
#define TRACE_OPS(slot) ZH_TRACE_POINT(slot)
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
static inline uint32_t attn_nd(uint32_t nkv, int cu_count) {
    const uint32_t cu = cu_count > 0 && cu_count < 256 ? (uint32_t)cu_count : 256u;
    const uint32_t nd = cu / nkv > 0 ? cu / nkv : 1u;
    return nd < 256u ? nd : 256u;  // the merge keeps at most 256 chunk statistics in LDS
}
// chunk slots per head for sub-chunks of tc tokens (the partials, sized with
// the shortest, hold any; a device with at most 256 CUs fits)
static inline uint32_t attn_n_chunks(uint32_t max_seq, uint32_t nd, uint32_t tc = AD_TC_MIN) {
    const uint32_t n = (max_seq + tc - 1) / tc;
    return n > nd ? n : nd;
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
    uint32_t ident;      // k_attn_ring: the page table is the identity (no lookups)
    uint32_t *ctl;       // device control words: [0] error word, [1] merge wait limit (ticks)
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
// LOCAL: every partial was written by a workgroup on this XCD (plain stores,
// held in the XCD's L2) and this workgroup has not read them before in this
// launch (its L1 holds no copy): plain loads, which hit the L2.
template <int GM, int NBAT, bool COH = false, bool LOCAL = false, int NT = AD_T>
ZH_DEV void attn_merge(const AttnP &p, uint32_t h0, uint32_t nv, bool poison, float *lds_out = nullptr) {
    auto ld1 = [](const float *q) { return LOCAL ? *q : ld_dev(q); };
    auto ld2 = [](const float *q) { return LOCAL ? *(const uint64_t *)q : ld_dev64(q); };
    // any workgroup size of at least NT threads (every thread calls it)
    const uint32_t tid = COH ? phase_tid() : threadIdx.x, wave = tid >> 6, lane = tid & 63, nthr = blockDim.x;
    TRACE_OPS(11);
    // Chunk merge. The first batch of each thread's O dims (NBAT chunks) is
    // requested before the chunk statistics, so both arrive in about one
    // round trip; the statistics pass leaves m_c in LDS for the weights.
    // dims per thread: the smallest power of two with G*128/OPT <= NT (more
    // threads means more partial loads in flight; the merge waits on them)
    constexpr int OPT = GM * FD_HD <= NT ? 1 : GM * FD_HD <= 2 * NT ? 2 : GM * FD_HD <= 4 * NT ? 4 : 8;
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
                v[u][0] = ld1(pc);
            } else {
#pragma unroll
                for (int w = 0; w < OPT / 2; w++) {
                    const uint64_t x = ld2(pc + 2 * w);
                    v[u][2 * w] = __uint_as_float((uint32_t)x);
                    v[u][2 * w + 1] = __uint_as_float((uint32_t)(x >> 32));
                }
            }
        }
    };
    const bool one_batch = nv <= (uint32_t)NBAT;  // uniform
    if (one_batch) load_o(0);
    asm volatile("" ::: "memory");  // the O loads go out before the statistics loads
    for (uint32_t g = wave; g < (uint32_t)GM; g += nthr / 64) {
        const float *pp = p.part + (size_t)(h0 + g) * p.n_chunks * (FD_HD + 2);
        float m = -INFINITY, l = 0.f;
        for (uint32_t c = lane; c < nv; c += 64) {
            const uint64_t ml = ld2(pp + (size_t)c * (FD_HD + 2) + FD_HD);
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
        for (uint32_t i = tid; i < (uint32_t)GM * NBAT; i += nthr) {
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
                const float mc = c < MB ? sm[g_t][c < MB ? c : 0] : ld1(pt + (size_t)min(c, nv - 1) * (FD_HD + 2) + FD_HD);
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
            if (lds_out) lds_out[tid * OPT + k] = r;  // (the caller's LDS copy of heads h0 ..)
            if (p.out) {
                if (COH) st_dev(p.out + (size_t)h0 * FD_HD + tid * OPT + k, r);
                else p.out[(size_t)h0 * FD_HD + tid * OPT + k] = r;
            }
        }
    }
    TRACE_OPS(7);
    if (p.xq) {
        __syncthreads();
        XQView v = xq_view(p.xq, p.nq * FD_HD / 32);
        for (uint32_t o = tid; o < (uint32_t)GM * FD_HD; o += nthr) {  // whole 32-lane groups (GM*128 % 32 == 0)
            const uint32_t blk = (h0 * FD_HD + o) / 32;
            if (COH) xq_store_block32_dev(ob[o], o & 31, v, blk);
            else xq_store_block32(ob[o], o & 31, v, blk);
            // the quantiser's max drops NaN: a poisoned head's blocks get NaN
            // scales so that the consumer's sums are NaN too
            if (poison && (o & 15) == 0) {
                float *xs = v.xs + blk, *xz = v.xsum + blk * 2 + ((o >> 4) & 1);
                if (COH) {
                    if ((o & 31) == 0) st_dev(xs, __builtin_nanf(""));
                    st_dev(xz, __builtin_nanf(""));
                } else {
                    if ((o & 31) == 0) *xs = __builtin_nanf("");
                    *xz = __builtin_nanf("");
                }
            }
        }
    }
    TRACE_OPS(5);
}


// The DMA-ring decode attention over a paged fp16 KV cache with the
// chunk's K/V streamed HBM -> LDS by asynchronous DMA (included by
// zh_ops.hip, after AttnP, norm_rope16, pack_h2 and attn_merge).
//
// Split-K flash decode (attention.zig:199-316, flash_decode.comp's split +
// merge) for one token: workgroup (kv head h, chunk c) of a grid of nkv x nd
// (nd = CUs / nkv, one workgroup per CU) owns the logical tokens
// [c CT, (c+1) CT) with CT = ceil(seq / nd) rounded up to a 16-token page.
// The chunk is cut into 64-token sub-chunks (4 pages: 16 KB of K and 16 KB
// of V) that stream through a ring of AR_D LDS slots: every 1 KB copy is 4
// tokens of one page, so each lane's address is page base + offset and any
// page table costs nothing per token (logicalTokenToPhysicalToken,
// forward.zig:677-698; the chunk's page entries are read once into LDS). All
// sub-chunks up to the ring depth are requested at once, before any compute.
//
// FUSED (the engine's step): q and the new token's k get the per-head
// RMSNorm and NeoX RoPE (qk_norm_rope_kv_write.comp), the new K/V row is
// written to the cache, and the workgroup holding the position substitutes
// it for the row its copy read (which predates the write).
//
// Each workgroup publishes one partial (O, m, l) per q head; the last of the
// kv head's workgroups to arrive (a device-scope counter) merges them
// (attn_merge) into the output and its XQ image, and resets the counter.
// No workgroup waits for another.
constexpr int AR_TS = 64;                            // tokens per sub-chunk
constexpr uint32_t AR_SLOT = AR_TS * 2 * FD_HD * 2;  // K then V: 32 KB
constexpr int AR_D = 4;                              // ring slots
constexpr uint32_t AR_MAXPG = 256;                   // page entries per chunk (CT <= 4096 tokens)
// waves per workgroup: two groups of four, each taking alternate sub-chunks
template <int G> constexpr int ar_waves() { return 8; }
// small copies, 1 KB each: q of the group (G / 2 KB), [k_new | v_new],
// [q_norm | k_norm], [RoPE row | -]; then the new K / V row as f16 (512 B)
template <int G> constexpr uint32_t ar_qc() { return (G * FD_HD * 4 + 1023) / 1024; }
template <int G> constexpr uint32_t ar_small() { return (ar_qc<G>() + 3) * 1024 + 512; }
// q's MFMA fragments (8 steps x 64 lanes x (hi, lo) 8 bytes) and the
// heads' 1 / rms
constexpr uint32_t AR_QFRAG = 8 * 64 * 16 + 64 * 4;
template <int G, int AW = ar_waves<G>()>
constexpr uint32_t ar_lds_bytes() {
    return AR_D * AR_SLOT + ar_small<G>() + AR_MAXPG * 4 + AR_QFRAG;
}

// Chunk geometry of workgroup (kv head, chunk c) at the position p.pos:
// chunk length CT = ceil(seq / nd) rounded up to a 16-token page, the chunk's
// tokens [t0, t1), its nsub 64-token sub-chunks (nv chunks hold tokens).
struct AttnGeom {
    uint32_t posv, seq, CT, nv, t0, t1, nsub;
    ZH_DEVM AttnGeom(const AttnP &p, uint32_t c, bool fused) {
        posv = p.pos.dev ? *p.pos.dev + p.pos.value : p.pos.value;
        seq = fused ? posv + 1 : posv;
        CT = ((seq + p.nd - 1) / p.nd + 15) / 16 * 16;
        nv = (seq + CT - 1) / CT;
        t0 = c * CT;
        t1 = min(seq, t0 + CT);
        nsub = c < nv ? (t1 - t0 + AR_TS - 1) / AR_TS : 0u;
    }
};

// K/V copies of sub-chunk s into slot s % AR_D: 32 chunks of 1 KB (4 tokens
// of one page; K then V), 32 / AW per wave. Rows past the chunk re-read its
// last row (masked). 16-byte piece q of LDS row rr holds the row's piece
// q ^ (rr % 16) (the MFMA fragment reads of 16 rows at one dim then hit 16
// different bank groups). pgl: the chunk's page entries (unless identity).
template <int AW>
ZH_DEV void attn_issue_kv(const AttnP &p, const AttnGeom &g, uint32_t kvh, uint32_t s, uint32_t wave,
                          uint32_t lane, uint32_t lds0, const uint32_t *pgl) {
    const uint16_t *kbase = p.kc + (size_t)kvh * p.cache_tokens * FD_HD;
    const uint16_t *vbase = p.vc + (size_t)kvh * p.cache_tokens * FD_HD;
    const uint32_t slot = s % AR_D;
#pragma unroll
    for (uint32_t i = 0; i < 32 / AW; i++) {
        const uint32_t j = wave + AW * i, kv = j >> 4;
        const uint32_t rr = 4 * (j & 15) + (lane >> 4);  // row within the slot
        const uint32_t t = min(g.t0 + s * AR_TS + rr, g.t1 - 1);
        const uint32_t ph = p.ident ? t : pgl[(t - g.t0) >> 4] * 16u + (t & 15u);
        const uint16_t *row = (kv ? vbase : kbase) + (size_t)ph * FD_HD;
        dma16(row + ((lane & 15) ^ (rr & 15)) * 8, lds0 + slot * AR_SLOT + j * 1024);
    }
}

// The chunk's page entries into LDS (a compiler-tracked load) and its first
// sub-chunks' K/V copies, issued while the persistent kernel waits at the
// grid barrier before the attention phase (the cache rows before the
// position do not depend on the Q/K/V phase); returns the count (the body's
// `pre`). Every thread of the workgroup calls it.
template <int G, int AW>
ZH_DEV uint32_t attn_ring_prefetch(const AttnP &p, uint32_t kvh, uint32_t c, uint8_t *lds, bool fused) {
    const uint32_t tid = phase_tid(), lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const AttnGeom g(p, c, fused);
    if (g.nsub == 0) return 0;
    uint32_t *pgl = (uint32_t *)(lds + AR_D * AR_SLOT + ar_small<G>());
    if (!p.ident) {
        for (uint32_t i = tid; i < (g.t1 - g.t0 + 15) / 16; i += AW * 64)
            pgl[i] = p.pages[min(g.t0 / 16 + i, p.n_pages - 1)];
        __syncthreads();
    }
    const uint32_t n = min(g.nsub, (uint32_t)AR_D);
    for (uint32_t s = 0; s < n; s++) attn_issue_kv<AW>(p, g, kvh, s, wave, lane, lds_addr(lds), pgl);
    return n;
}

// AW waves (4 or 8: one or two groups of four taking alternate sub-chunks);
// COH: q and the new token's k / v were written by other workgroups of the
// same launch (read at system scope), and the merged output is read by other
// workgroups of it (stored at device scope). pre: sub-chunks 0 .. pre-1
// already copied (attn_ring_prefetch, page entries included).
template <int G, bool FUSED, int AW, bool COH>
ZH_DEV void attn_ring_body(const AttnP &p, uint32_t kvh, uint32_t c, uint8_t *lds, uint32_t pre = 0) {
    constexpr int AT = AW * 64, NG = AW / 4;  // threads, groups
    constexpr uint32_t QC = ar_qc<G>();
    constexpr uint32_t NSM = QC + (FUSED ? 2 : 0);  // position-independent small copies
    constexpr uint32_t KVW = 32 / AW;               // K/V copies per wave and sub-chunk
    uint8_t *sm = lds + AR_D * AR_SLOT;
    uint32_t *pgl = (uint32_t *)(sm + ar_small<G>());
    const uint32_t tid = COH ? phase_tid() : threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6), sub = lane & 7;
    const uint32_t gq = wave / 4, w4 = wave % 4;  // group, wave within the group
    const uint32_t lds0 = lds_addr(lds);
    TRACE_OPS(0);
    // ---- position-independent small copies first (q, the new token's raw k
    // and v, the norm weights), while the position is read
    {
        const uint32_t l16 = lane * 16, half = lane >> 5, o = (lane & 31) * 16;
        for (uint32_t k = wave; k < NSM; k += AW) {  // uniform per wave
            const uint8_t *src;
            if (k < QC) {
                src = (const uint8_t *)(p.q + (size_t)kvh * G * FD_HD) + min(k * 1024 + l16, (uint32_t)G * 512 - 16);
            } else if (k == QC) {
                src = half ? (const uint8_t *)(p.v_new + (size_t)kvh * FD_HD) + o
                           : (const uint8_t *)(p.k_new + (size_t)kvh * FD_HD) + o;
            } else {
                src = half ? (const uint8_t *)p.k_norm + o : (const uint8_t *)p.q_norm + o;
            }
            if (k <= QC) dma16_act<COH>(src, lds0 + AR_D * AR_SLOT + k * 1024);
            else dma16(src, lds0 + AR_D * AR_SLOT + k * 1024);
        }
    }
    // ---- position and chunk geometry
    const AttnGeom geo(p, c, FUSED);
    const uint32_t posv = geo.posv, nv = geo.nv, t0 = geo.t0, t1 = geo.t1, nsub = geo.nsub;
    if (nsub == 0) {  // uniform: no token of this chunk
        wait_vm<0>();
        return;
    }
    if (!p.ident && pre == 0) {
        // the chunk's page entries (a compiler-tracked load: its wait also
        // drains the small copies, which are needed first anyway)
        for (uint32_t i = tid; i < (t1 - t0 + 15) / 16; i += AT) pgl[i] = p.pages[min(t0 / 16 + i, p.n_pages - 1)];
        __syncthreads();
    }
    if (FUSED && wave == AW - 1)  // the RoPE row of the position
        dma16((const uint8_t *)(p.rope_cs + (size_t)posv * FD_HD) + min(lane * 16, 496u),
              lds0 + AR_D * AR_SLOT + (QC + 2) * 1024);
    auto phys = [&](uint32_t t) __attribute__((always_inline)) {  // logical token in [t0, t1)
        return p.ident ? t : pgl[(t - t0) >> 4] * 16u + (t & 15u);
    };
    auto issue_kv = [&](uint32_t s) __attribute__((always_inline)) {
        attn_issue_kv<AW>(p, geo, kvh, s, wave, lane, lds0, pgl);
    };
    const uint32_t npro = min(nsub, (uint32_t)AR_D);
    for (uint32_t s = pre; s < npro; s++) issue_kv(s);
    // the small copies and the RoPE row (issued before the K/V copies of
    // this call, after the prefetched ones)
    wait_vm_dyn((npro - pre) * KVW);
    lds_bar();
    TRACE_OPS(1);

    // ---- q as MFMA operand fragments: lane l holds head fg = l % 16 (zero
    // rows for fg >= G), dims 16 s + 4 fq + 0..3 (fq = l / 16) for the eight
    // 16-dim steps s, RMS-normalised and roped in place (the RoPE partner of
    // dim d < 64, d + 64, is step s + 4 of the same lane), then split into
    // f16 hi + lo parts so that the f16 products carry the f32 q exactly
    // enough (|q - hi - lo| <= 2^-22 |q|).
    const uint32_t fg = lane & 15, fq = lane >> 4;
    half4 qh[8], ql[8];
    {
        // computed once per workgroup and shared through LDS: the heads' RMS
        // (wave g: head g), then group 0's wave w the dims of steps w and
        // w + 4 (the RoPE pairs), then every wave reads its fragments
        uint8_t *frag = (uint8_t *)(pgl + AR_MAXPG);
        float *rinv = (float *)(frag + 8 * 64 * 16);
        if (FUSED) {
            for (uint32_t g = wave; g < (uint32_t)G; g += AW) {
                const float *qs = (const float *)sm + g * FD_HD;
                const float a = qs[lane], b = qs[lane + 64];
                const float sq = wave_sum(fmaf(a, a, b * b));
                if (lane == 0) rinv[g] = 1.0f / sqrtf(sq / (float)FD_HD + p.eps);
            }
            lds_bar();
        }
        if (wave < 4) {
            const uint32_t pi = wave;  // steps pi (dims < 64) and pi + 4 (their RoPE partners)
            const float *qs = (const float *)sm + min(fg, (uint32_t)G - 1) * FD_HD;
            const f32x4 va = *(const f32x4 *)(qs + 16 * pi + 4 * fq), vb = *(const f32x4 *)(qs + 64 + 16 * pi + 4 * fq);
            float lo[4] = {va.x, va.y, va.z, va.w}, hi[4] = {vb.x, vb.y, vb.z, vb.w};
            if (FUSED) {
                const float *qw = (const float *)(sm + (QC + 1) * 1024);
                const float *cs = (const float *)(sm + (QC + 2) * 1024);
                const float ri = rinv[min(fg, (uint32_t)G - 1)];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t i = 16 * pi + 4 * fq + j;  // dims i and i + 64
                    const float a = qw[i] * (lo[j] * ri);
                    const float b = qw[i + 64] * (hi[j] * ri);
                    const float co = cs[2 * i], sn = cs[2 * i + 1];
                    lo[j] = a * co - b * sn;
                    hi[j] = a * sn + b * co;
                }
            }
            half4 h0, l0, h1, l1;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float x = fg < (uint32_t)G ? lo[j] : 0.f, y = fg < (uint32_t)G ? hi[j] : 0.f;
                h0[j] = (_Float16)x;
                l0[j] = (_Float16)(x - (float)h0[j]);
                h1[j] = (_Float16)y;
                l1[j] = (_Float16)(y - (float)h1[j]);
            }
            *(half4 *)(frag + (pi * 64 + lane) * 16) = h0;
            *(half4 *)(frag + (pi * 64 + lane) * 16 + 8) = l0;
            *(half4 *)(frag + ((pi + 4) * 64 + lane) * 16) = h1;
            *(half4 *)(frag + ((pi + 4) * 64 + lane) * 16 + 8) = l1;
        }
        lds_bar();
#pragma unroll
        for (int s8 = 0; s8 < 8; s8++) {
            qh[s8] = *(const half4 *)(frag + (s8 * 64 + lane) * 16);
            ql[s8] = *(const half4 *)(frag + (s8 * 64 + lane) * 16 + 8);
        }
    }
    TRACE_OPS(9);
    // ---- the new token's k / v (the owner only)
    const bool owner = FUSED && posv >= t0 && posv < t1;  // uniform
    uint16_t *knew16 = (uint16_t *)(sm + (QC + 3) * 1024), *vnew16 = knew16 + FD_HD;
    if (FUSED && owner && wave == 0) {
        const float *kn = (const float *)(sm + QC * 1024), *vn = kn + FD_HD;
        const float *kw = (const float *)(sm + (QC + 1) * 1024) + FD_HD;
        const float *cs = (const float *)(sm + (QC + 2) * 1024);
        float klo[8], khi[8], wlo[8], whi[8], co[8], sn[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            klo[e] = kn[sub * 8 + e];
            khi[e] = kn[64 + sub * 8 + e];
            wlo[e] = kw[sub * 8 + e];
            whi[e] = kw[64 + sub * 8 + e];
            co[e] = cs[2 * (sub * 8 + e)];
            sn[e] = cs[2 * (sub * 8 + e) + 1];
        }
        norm_rope16(klo, khi, wlo, whi, co, sn, p.eps);  // all 64 lanes (8 copies of the head)
        if (lane < 8) {
            *(u32x4 *)(knew16 + sub * 8) = u32x4{pack_h2(klo[0], klo[1]), pack_h2(klo[2], klo[3]),
                                                 pack_h2(klo[4], klo[5]), pack_h2(klo[6], klo[7])};
            *(u32x4 *)(knew16 + 64 + sub * 8) = u32x4{pack_h2(khi[0], khi[1]), pack_h2(khi[2], khi[3]),
                                                      pack_h2(khi[4], khi[5]), pack_h2(khi[6], khi[7])};
        }
        *(uint32_t *)(vnew16 + 2 * lane) = pack_h2(vn[2 * lane], vn[2 * lane + 1]);
    }
    const uint32_t s_own = owner ? (posv - t0) / AR_TS : ~0u, r_own = owner ? (posv - t0) % AR_TS : 0u;
    TRACE_OPS(10);

    // ---- the ring, NG sub-chunks per step (group gq takes sub-chunk
    // NG k + gq); wave w4 of a group takes its tokens 16 w4 .. 16 w4 + 15.
    // Scores: S^T (16 tokens x 16 heads) = K (16 x 128) q^T over eight
    // 16x16x16 MFMA steps (hi and lo q): lane l ends with tokens 4 fq + r of
    // head fg. Online softmax per head over the wave's tokens (the waves
    // are combined at the end). P V: O (16 heads x 128) += P (16 x 16
    // tokens) V (16 tokens x 128), eight 16-dim tiles: the score layout is
    // the P operand's (row = head fg, k = token 4 fq + r); lane l holds O
    // rows 4 fq + r (heads), dim 16 n + fg of tile n.
    float m_run = -INFINITY, l_run = 0.f;  // head fg (every fq copy)
    floatx4 acc[8];
#pragma unroll
    for (int n = 0; n < 8; n++) acc[n] = floatx4{0.f, 0.f, 0.f, 0.f};
    const uint32_t nstep = (nsub + NG - 1) / NG;
    for (uint32_t k = 0; k < nstep; k++) {
        // sub-chunks up to NG k + NG - 1 must have landed; later ones stay in
        // flight (issued so far: the prologue's AR_D, then NG per step from
        // step 1 on, after its wait)
        const uint32_t last = min(NG * k + NG, nsub) - 1;
        const uint32_t issued = min(nsub, k ? NG * k + AR_D - NG : (uint32_t)AR_D);
        wait_vm_dyn((issued - 1 - last) * KVW);
        lds_bar();
        if (k < 2) TRACE_OPS(5 + 2 * k);
        if (k) {  // refill the slots of step k - 1
            for (uint32_t s = NG * k + AR_D - NG; s < NG * k + AR_D && s < nsub; s++) issue_kv(s);
        }
        if (s_own >= NG * k && s_own < NG * k + NG) {  // uniform: substitute the new token's K and V rows
            uint8_t *Ks = lds + (s_own % AR_D) * AR_SLOT;
            const uint32_t pc = ((tid & 15) ^ (r_own & 15)) * 16;  // the row's swizzled 16-byte piece
            if (tid < 16) *(u32x4 *)(Ks + r_own * 256 + pc) = *(const u32x4 *)((const uint8_t *)knew16 + tid * 16);
            else if (tid < 32)
                *(u32x4 *)(Ks + AR_SLOT / 2 + r_own * 256 + pc) =
                    *(const u32x4 *)((const uint8_t *)vnew16 + (tid - 16) * 16);
            lds_bar();
        }
        const uint32_t s = NG * k + gq;
        if (s < nsub) {  // uniform per wave
            const uint8_t *Ks = lds + (s % AR_D) * AR_SLOT, *Vs = Ks + AR_SLOT / 2;
            const uint32_t ts = t0 + s * AR_TS, tb = w4 * 16;
            // every fragment read first (one LDS round trip): K rows of the
            // wave's tokens tb + fg, V of its tokens tb + 4 fq + r. Rows past
            // the chunk hold a copy of its last row: their probabilities are
            // 0 and their V values are zeroed below.
            half4 kf[8], vf[8];
            {
                const uint32_t t = tb + fg;
#pragma unroll
                for (int s8 = 0; s8 < 8; s8++)
                    kf[s8] = *(const half4 *)(Ks + t * 256 + (((2 * s8 + (fq >> 1)) ^ (t & 15)) * 16) + 8 * (fq & 1));
                // P V's column j of MFMA tile n is dim 8 j + n, so a lane's
                // operands are dims 8 fg .. 8 fg + 7 of its 4 tokens: one
                // 16-byte piece of each token's row. V rows past the chunk are
                // zeroed, not only weighted 0: they copy the cache's row of the
                // new token, which this launch has not written yet and may hold
                // anything (NaN after a step whose waits gave up), and 0 x NaN
                // is NaN
                const uint32_t tv = tb + 4 * fq;
                const uint32_t tvalid = t1 - ts;  // tokens of the sub-chunk in the chunk
                u32x4 pv[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const uint32_t t2 = tv + r;
                    const u32x4 w = *(const u32x4 *)(Vs + t2 * 256 + (fg ^ (t2 & 15)) * 16);
                    pv[r] = t2 < tvalid ? w : u32x4{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int n = 0; n < 8; n++) {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const uint32_t d = pv[r][n >> 1];
                        vf[n][r] = __builtin_bit_cast(_Float16, (uint16_t)((n & 1) ? d >> 16 : d));
                    }
                }
            }
            // scores
            floatx4 d1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s8 = 0; s8 < 8; s8++) {
                d1 = __builtin_amdgcn_mfma_f32_16x16x16f16(kf[s8], qh[s8], d1, 0, 0, 0);
                d1 = __builtin_amdgcn_mfma_f32_16x16x16f16(kf[s8], ql[s8], d1, 0, 0, 0);
            }
            float sc[4];
#pragma unroll
            for (int r = 0; r < 4; r++) sc[r] = ts + tb + 4 * fq + r < t1 ? d1[r] * p.scale : -INFINITY;  // dot * scale
            float m = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
            m = xor16_max(m);
            m = xor32_max(m);
            const float mn = fmaxf(m_run, m);
            const float ms = mn == -INFINITY ? 0.f : mn;
            const float f = m_run == -INFINITY ? 0.f : expf(m_run - ms);
            float pr[4], lsum = 0.f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                pr[r] = fg < (uint32_t)G ? expf(sc[r] - ms) : 0.f;
                lsum += pr[r];
            }
            lsum = xor16_sum(lsum);
            lsum = xor32_sum(lsum);
            l_run = fmaf(l_run, f, lsum);
            m_run = mn;
            half4 ph, pl;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const _Float16 h = (_Float16)pr[r];
                ph[r] = h;
                pl[r] = (_Float16)(pr[r] - (float)h);
            }
            // rescale the output rows (heads 4 fq + r) by their heads' factors
            // (lane h, fq = 0, holds head h's)
            float fr[4];
#pragma unroll
            for (int r = 0; r < 4; r++) fr[r] = G > 4 && fq ? lane_f(f, 4 + r) : lane_f(f, r);
#pragma unroll
            for (int n = 0; n < 8; n++) {
#pragma unroll
                for (int r = 0; r < 4; r++) acc[n][r] *= fr[r];
                acc[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(ph, vf[n], acc[n], 0, 0, 0);
                acc[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(pl, vf[n], acc[n], 0, 0, 0);
            }
        }
        if (k < 2) TRACE_OPS(6 + 2 * k);
    }
    TRACE_OPS(2);
    // ---- the new row to the cache (after every copy of this workgroup)
    if (owner && tid < 32) {
        const uint32_t ph = phys(posv);
        uint16_t *dst = (tid < 16 ? p.kc : p.vc) + ((size_t)kvh * p.cache_tokens + ph) * FD_HD + (tid & 15) * 8;
        *(u32x4 *)dst = *(const u32x4 *)((const uint8_t *)(tid < 16 ? knew16 : vnew16) + (tid & 15) * 16);
    }
    // ---- combine the waves (in the ring's LDS, free now): token rows within
    // a wave, then waves
    float *wm = (float *)lds, *wl = wm + AW * G, *wo = wl + AW * G;  // [AW][G], [AW][G], [AW][G][128]
    lds_bar();  // every wave is done with the ring
    // lane l: heads 4 fq + r, dims 8 fg + n (two 16-byte stores per head);
    // the running statistics of head fg are in the lanes with fq = 0
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint32_t g = 4 * fq + r;
        if (g < (uint32_t)G) {
            f32x4 *o = (f32x4 *)(wo + (wave * G + g) * FD_HD + 8 * fg);
            o[0] = f32x4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
            o[1] = f32x4{acc[4][r], acc[5][r], acc[6][r], acc[7][r]};
        }
    }
    if (fq == 0 && fg < (uint32_t)G) {
        wm[wave * G + fg] = m_run;
        wl[wave * G + fg] = l_run;
    }
    __syncthreads();
    for (uint32_t o = tid; o < (uint32_t)G * FD_HD; o += AT) {
        const uint32_t g = o / FD_HD, d = o % FD_HD;
        float M = wm[g];
#pragma unroll
        for (int w = 1; w < AW; w++) M = fmaxf(M, wm[w * G + g]);
        const float Ms = M == -INFINITY ? 0.f : M;
        float O = 0.f, L = 0.f;
#pragma unroll
        for (int w = 0; w < AW; w++) {
            const float f = wm[w * G + g] == -INFINITY ? 0.f : expf(wm[w * G + g] - Ms);
            O = fmaf(wo[(w * G + g) * FD_HD + d], f, O);
            L = fmaf(wl[w * G + g], f, L);
        }
        float *pp = p.part + ((size_t)(kvh * G + g) * p.n_chunks + c) * (FD_HD + 2);
        st_dev(pp + d, O);
        if (d == 0) {
            st_dev(pp + FD_HD, M);
            st_dev(pp + FD_HD + 1, L);
        }
    }
    TRACE_OPS(3);
    // ---- publish; the last arrival of this kv head merges. The partials
    // went out as device-scope stores (coherent across the XCDs' L2s);
    // s_waitcnt 0 in every wave and the barrier make them complete before the
    // counter increment, and the merger reads them with device-scope loads.
    __shared__ uint32_t s_prev, s_ok;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) s_prev = __hip_atomic_fetch_add(p.counters + kvh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (!COH && p.no_wait) {
        if (s_prev != nv - 1) return;
        TRACE_OPS(4);
        if (tid == 0) __hip_atomic_store(p.counters + kvh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        attn_merge<G, G <= 4 ? 40 : 12, COH, false, AT>(p, kvh * G, nv, false);
        return;
    }
    // Every workgroup resident (the persistent kernel, or a launch with the
    // device to itself: one workgroup per CU, grid <= CUs): the last G
    // arrivals merge one q head each; all but the last wait (bounded by
    // p.ctl[1] ticks, ZH_DEVERR_ATTN_WAIT on giving up) for the kv head's
    // other chunks. counters[nkv + kvh] counts mergers past the wait; the
    // last one clears both words (nothing reads them after).
    const uint32_t nm = nv >= (uint32_t)G ? (uint32_t)G : 1u, prev = s_prev;
    if (prev + nm < nv) return;
    const uint32_t slot = prev + nm - nv;
    TRACE_OPS(4);
    if (tid == 0) {
        uint32_t ok = 1;
        if (slot != nm - 1) {
            const uint64_t t_0 = __builtin_amdgcn_s_memrealtime();
            const uint64_t limit = __hip_atomic_load(p.ctl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            while (limit == 0 || __hip_atomic_load(p.counters + kvh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < nv) {
                if (__builtin_amdgcn_s_memrealtime() - t_0 >= limit) {
                    ok = 0;
                    __hip_atomic_fetch_or(p.ctl, ZH_DEVERR_ATTN_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        s_ok = ok;
        uint32_t *done = p.counters + p.nq / G + kvh;
        if (__hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nm - 1) {
            __hip_atomic_store(p.counters + kvh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __syncthreads();
    if (nm == 1) attn_merge<G, G <= 4 ? 40 : 12, COH, false, AT>(p, kvh * G, nv, !s_ok);
    else attn_merge<1, 32, COH>(p, kvh * G + slot, nv, !s_ok);
}

