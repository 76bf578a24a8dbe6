// zh_qkv_attn.hip — the decode step's Q/K/V projection and attention in one
// launch, for models with 8 kv heads on a device of 8 XCDs x 32 CUs.
//
// Replaces two dispatches of the reference's decode step: the Q/K/V DMMVs
// (forward.zig:4776-4800, dmmv_q4k.comp) and the fused q/k norm + RoPE + KV
// write + flash decode (qk_norm_rope_kv_write.comp, attention.zig:199-316,
// flash_decode.comp with its split-K merge).
//
// The dispatcher deals the workgroups of a launch round robin over the 8
// XCDs, starting where the previous launch stopped (measured: workgroup w
// lands on XCD (w + s) % 8 for a launch-dependent s; the engine checks this
// once per context with zhk_xcd_round_robin). Each workgroup reads its XCD
// from the XCC_ID register and takes kv head h = XCD, slice j = w / 8: every
// run of 8 consecutive workgroups covers the 8 XCDs once, so the (h, j) are
// all distinct. The 32 workgroups of XCD h
//   1. compute the (G + 2) * 128 Q/K/V rows of kv head h (its G q heads, its
//      k and v head), R = 4 (G + 2) rows each, from attn_norm(x) as XQ
//      limbs (the arithmetic of the ring DMMV, zh_ring_q4k.h, row for row);
//   2. meet at an XCD-local flag barrier;
//   3. run the split-K attention over chunk j of the context (norm + RoPE of
//      q and the new k, MFMA scores and P V, the new K/V row written to the
//      cache by its chunk's owner), publish a partial (O, m, l) per q head;
//   4. meet again: workgroups j < G merge q head h G + j into the attention
//      output and its XQ image for the O projection.
// Everything exchanged between steps stays inside XCD h, so it is exchanged
// through that XCD's L2: the producer's plain stores land in its L2, the
// consumers read with device-scope (sc1) loads, which return the L2's copy
// (measured: a flag round trip 0.5 us against 1.0 us for device-scope
// stores and 3.5-4.5 us for a flag barrier over all 256 workgroups). The
// next kernel sees the outputs after the end-of-kernel L2 write-back.
//
// Flags carry an epoch instead of being reset: at the start every
// workgroup of XCD h reads the epoch word ep[h] and publishes E = ep[h] + 1;
// merger 0 stores E into ep[h] once every chunk of the head has published,
// i.e. after all 32 workgroups read it. Every wait is bounded (the attention
// merge's limit, ctl[1]); one that gives up sets ZH_DEVERR_ATTN_WAIT and the
// head's output is NaN, as in the two-kernel path.
//
// LDS (155.6 KB of 160): K/V sub-chunks 0 and 1 (64 tokens of K then V,
// 32 KB each), the workgroup's weight rows (R x 2304 B; afterwards the
// attention's q, new k / v rows and q fragments), the f32 x and norm weight
// (then its XQ image, then K/V sub-chunk 2), norm weights and the RoPE row.
// The weight rows, x, the norm weights and (after the position) the K/V
// sub-chunks are all requested at the start, so the K/V stream overlaps the
// projection and the barrier. Longer chunks stream their 64-token sub-chunks
// through a ring of four slots (the x region and the weight region join it
// once the projection is done), two sub-chunks ahead of the wave groups:
// contexts up to 32 x 2048 tokens.
#define TRACE_OPS(slot) ZH_TRACE_POINT((slot) == 11 ? 14 : (slot) == 13 ? 15 : 99)  // merge start, merge stats done
#include "zh_attn_common.h"
#include "zh_lpb_common.h"
#include "zh_xcd.h"

namespace {

constexpr int QA_T = 512;                       // 8 waves, two per SIMD
constexpr uint32_t RG_SEG = 400;                // XQ image: bytes per 128-element half super-block (padded)
constexpr int QA_AW = 8, QA_KVW = 32 / QA_AW;   // K/V copies per wave and sub-chunk
constexpr uint32_t QA_MAXR = 24;                // rows per workgroup (4 q heads + k + v: 768 rows / 32)
constexpr uint32_t QA_W = 2 * AR_SLOT;          // weight rows
constexpr uint32_t QA_NXCD = 8, QA_PER = 32;    // XCDs, workgroups per XCD

// The two model shapes the kernel is built for:
//   SH 3 (config 3): hidden 4096, 8 kv heads = one per XCD, Q4_K Q/K/V/O,
//        contexts up to 65536;
//   SH 4 (config 4): hidden 2048, 4 kv heads of 8 q heads: kv head h / 2 on
//        XCD h, which takes its q heads 4 (h % 2) .. + 3 (both XCDs of a
//        pair compute the kv head's k and v rows, identically); Q8_0
//        Q/K/V/O; contexts up to 65536.
// Either way an XCD owns 4 q heads, 24 projection rows per workgroup and the
// O projection's columns of its 4 heads.
template <int SH>
struct QaS {
    static constexpr uint32_t H = SH == 3 ? 4096 : 2048;
    static constexpr bool Q8 = SH == 4;                     // Q8_0 rows, else Q4_K
    static constexpr uint32_t KVX = SH == 3 ? 1 : 2;        // XCDs per kv head
    static constexpr uint32_t MAXSUB = 32;                  // K/V sub-chunks per chunk (contexts up to 65536)
    static constexpr uint32_t NB = H / 256;                 // 256-element super-blocks of x
    static constexpr uint32_t ROWB = Q8 ? H / 32 * 34 : NB * 144;
    static constexpr uint32_t X = QA_W + QA_MAXR * ROWB;    // x | norm weight, XQ image, K/V sub-chunk 2
    static constexpr uint32_t NRM = X + AR_SLOT;            // q_norm | k_norm (1 KB)
    static constexpr uint32_t ROPE = NRM + 1024;            // the position's (cos, sin) row (1 KB copy)
    static constexpr uint32_t YL = ROPE + 1024;             // row results [32], RMS partials [8]
    static constexpr uint32_t LDS = YL + 256;
    static constexpr uint32_t OROWS = H / QA_PER;           // O-projection rows per workgroup
    static constexpr uint32_t OROWB = Q8 ? 16 * 34 : 2 * 144;  // a row's columns of the XCD's 4 heads
    static constexpr uint32_t OW = QA_W + 16384;            // the O rows' LDS copy
    static constexpr uint32_t SUB3 = QA_W + 16384;          // K/V sub-chunk 3 (SH 4; the weight region, after the rows)
    static constexpr uint32_t RROWS = H / (QA_NXCD * QA_PER);  // residual rows each workgroup stores / zeroes
    static_assert(NB * 2 * RG_SEG + NB * 8 * 12 <= AR_SLOT && 2 * H * 4 <= AR_SLOT, "x | norm and the XQ image fit the x region");
    static_assert(OW + OROWS * OROWB <= X && SUB3 + AR_SLOT <= X, "O rows / sub-chunk slot 3 fit");
    static_assert(QA_MAXR * ROWB % 1024 == 0, "whole 1 KB copies of the rows");
};

}  // namespace

// Flag words (zero when the engine is created): [0, 256) unused (the Q/K/V
// rows carry epoch tags), [256, 512) partials published (head h at h * 32:
// one 128-byte line per XCD), [512, 520) epochs.
constexpr uint32_t QA_FLAG_WORDS = 2 * QA_NXCD * QA_PER + QA_NXCD;
constexpr uint32_t QA_XROWS = 4 * FD_HD + 2 * FD_HD;  // an XCD's q | k | v rows (at most 4 q heads)

struct QaP {
    AttnP a;                      // q / k_new / v_new: the projection outputs (written here)
    const uint8_t *wq, *wk, *wv;  // Q4_K [nq * 128 | 8 * 128 | 8 * 128][4096]
    const float *x, *norm_w;      // residual stream, attn_norm weight
    uint32_t *flags;              // QA_FLAG_WORDS
    uint32_t kv_defer;            // K/V copies issued at the start (0), after x landed (1), after the rows landed (2)
    // WITH_O: the O projection of the XCD's G heads (Q4_K W_o [4096][4096],
    // super-blocks 2h and 2h + 1 of every row) added to x_acc with device
    // atomics; x (the Q/K/V input) is then not x_acc, which changes during
    // the launch (a copy of it taken before, or the split residual below).
    const uint8_t *wo;
    void *x_acc;                  // f32 (no split residual) or zh_fix (split residual: zh_xcd.h fix_add)
    uint64_t *xrows;              // [8][QA_XROWS] epoch-tagged Q/K/V rows (exchanged inside each XCD)
    // Split residual (with the O phase): the layer input is x + xb (xb: the
    // previous launch's atomic sums in fixed point, staged in K/V sub-chunk
    // 0's slot, whose copy then waits until x is in registers); every
    // workgroup stores its 16 rows of x + xb into x_out and zeroes its 16
    // rows of `zero`.
    const zh_fix *xb;
    float *x_out;
    zh_fix *zero;
};

// LDS offset of K/V sub-chunk s: a ring of four slots (the third is the x
// region, free once the XQ image is in registers; the fourth the weight
// region, free once the rows are computed)
template <int SH>
ZH_DEV uint32_t qa_slot(uint32_t s) {
    const uint32_t r = s & 3;
    return r == 0 ? 0u : r == 1 ? AR_SLOT : r == 2 ? QaS<SH>::X : QaS<SH>::SUB3;
}

template <int G, bool WITH_O, int SH>
__global__ __launch_bounds__(QA_T, 1) void k_qkv_attn(QaP P) {
    using S = QaS<SH>;
    constexpr uint32_t QA_X = S::X, QA_NRM = S::NRM, QA_ROPE = S::ROPE, QA_YL = S::YL, QA_OW = S::OW;
    constexpr uint32_t QA_OROWS = S::OROWS, QA_OROWB = S::OROWB, QA_NB = S::NB, QA_ROWB = S::ROWB;
    constexpr uint32_t QA_MAXSUB = S::MAXSUB, H = S::H;
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr uint32_t R = 4 * (G + 2);          // weight rows per workgroup
    constexpr uint32_t NCH = R * QA_ROWB / 1024;  // their 1 KB copies
    constexpr uint32_t NP = (R + 15) / 16;        // passes of 16 rows
    constexpr uint32_t QC = ar_qc<G>();           // 1 KB copies of the group's q
    constexpr uint32_t QR = G * FD_HD;            // q rows of a kv head
    static_assert(R * QA_ROWB % 1024 == 0 && R <= QA_MAXR && R % 4 == 0, "row slice");
    static_assert(!WITH_O || G == 4, "the O phase takes 4 heads = 2 super-blocks of columns per XCD");
    const AttnP &p = P.a;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // kv head = this workgroup's XCD; slice j = blockIdx / 8 (each run of 8
    // consecutive workgroups covers the 8 XCDs once)
    const uint32_t h = min(xcc_id(), QA_NXCD - 1), j = blockIdx.x / QA_NXCD, kvh = h / S::KVX;
    const uint32_t lds0 = lds_addr(lds);
    uint32_t *fl_p = P.flags + QA_NXCD * QA_PER + h * QA_PER;
    uint32_t *ep = P.flags + 2 * QA_NXCD * QA_PER + h;
    // position and epoch through the scalar cache (no vector-memory count)
    const uint32_t posv = *(const __attribute__((address_space(4))) uint32_t *)p.pos.dev + p.pos.value;
    const uint32_t E = *(const __attribute__((address_space(4))) uint32_t *)ep + 1u;
    ZH_TRACE_POINT(0);
    ZH_TRACE_VALUE(h + 1);  // (the XCD, + 1: a slot of 0 reads as unset)

    // ---- copies. Waves 0-3 copy what the projection needs (x | attn_norm
    // weight, then the slice's weight rows); waves 4-7 the attention's (K/V
    // sub-chunks, q_norm | k_norm, the RoPE row), so that no wave that waits
    // for the projection's data also waits for K/V, and the row publication
    // below waits only for its own stores.
    const bool wa = wave < 4;  // uniform
    const uint32_t wl4 = wave & 3;
    const uint32_t nw = wl4 < NCH % 4 ? NCH / 4 + 1 : NCH / 4;  // weight copies of an A wave
    if (wa) {
#pragma unroll
        for (uint32_t i = 0; i < H / 1024; i++) {  // H / 256 copies of 1 KB per vector over 4 waves
            const uint32_t c = wl4 + 4 * i;
            dma16((const uint8_t *)P.x + c * 1024 + lane * 16, lds0 + QA_X + c * 1024);
            dma16((const uint8_t *)P.norm_w + c * 1024 + lane * 16, lds0 + QA_X + H * 4 + c * 1024);
        }
        if (P.xb)  // (8 bytes per element: H / 128 copies of 1 KB)
#pragma unroll
            for (uint32_t i = 0; i < H / 512; i++) {
                const uint32_t c = wl4 + 4 * i;
                dma16((const uint8_t *)P.xb + c * 1024 + lane * 16, lds0 + qa_slot<SH>(0) + c * 1024);
            }
#pragma unroll
        for (uint32_t i = 0; i < (NCH + 3) / 4; i++) {
            const uint32_t c = wl4 + 4 * i;
            if (c < NCH) {  // uniform per wave
                const uint32_t o = c * 1024 + lane * 16, r = o / QA_ROWB, within = o - r * QA_ROWB;
                const uint32_t rr = j * R + r;  // row of the kv head's q | k | v rows
                const uint8_t *src = rr < QR ? P.wq + (size_t)(h * QR + rr) * QA_ROWB
                                   : rr < QR + FD_HD ? P.wk + (size_t)(kvh * FD_HD + rr - QR) * QA_ROWB
                                                     : P.wv + (size_t)(kvh * FD_HD + rr - QR - FD_HD) * QA_ROWB;
                dma16(src + within, lds0 + QA_W + c * 1024);
            }
        }
    } else if (wave == 4) {
        dma16((const uint8_t *)(lane < 32 ? p.q_norm : p.k_norm) + (lane & 31) * 16, lds0 + QA_NRM);
    }

    // ---- chunk geometry (chunk j of 32)
    const uint32_t seq = posv + 1;
    const uint32_t CT = ((seq + QA_PER - 1) / QA_PER + 15) / 16 * 16;
    const uint32_t nv = (seq + CT - 1) / CT;  // chunks holding tokens
    const uint32_t t0 = j * CT, t1 = min(seq, t0 + CT);
    uint32_t nsub = j < nv ? (t1 - t0 + AR_TS - 1) / AR_TS : 0u;
    if (nsub > QA_MAXSUB) {  // (the engine keeps the context within 32 x 2048 tokens)
        if (tid == 0) __hip_atomic_fetch_or(p.ctl, ZH_DEVERR_ATTN_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        nsub = QA_MAXSUB;
    }
    const uint16_t *kbase = p.kc + (size_t)kvh * p.cache_tokens * FD_HD;
    const uint16_t *vbase = p.vc + (size_t)kvh * p.cache_tokens * FD_HD;
    // sub-chunk s (B waves): 32 copies of 1 KB (4 token rows of K, then of
    // V); rows past the chunk re-read its last row (masked). 16-byte piece q
    // of LDS row rr holds the row's piece q ^ (rr % 16).
    auto issue_kv = [&](uint32_t s) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) {
            const uint32_t jj = wl4 + 4 * i, kv = jj >> 4;
            const uint32_t rr = 4 * (jj & 15) + (lane >> 4);
            const uint32_t t = min(t0 + s * AR_TS + rr, t1 - 1);
            const uint16_t *row = (kv ? vbase : kbase) + (size_t)t * FD_HD;
            dma16(row + ((lane & 15) ^ (rr & 15)) * 8, lds0 + qa_slot<SH>(s) + jj * 1024);
        }
    };
    const uint32_t n01 = min(nsub, 2u);
    if (!wa) {
        if (wave == 5)
            dma16((const uint8_t *)(p.rope_cs + (size_t)posv * FD_HD) + min(lane * 16, 496u), lds0 + QA_ROPE);
        if (P.kv_defer == 0)
            for (uint32_t s = P.xb ? 1u : 0u; s < n01; s++) issue_kv(s);
    }

    // ---- attn_norm(x) as XQ limbs (the ring DMMV's staging, in place)
    if (wa) wait_vm_dyn(nw);
    lds_bar();
    ZH_TRACE_POINT(1);
    if (!wa && P.kv_defer == 1)
        for (uint32_t s = 0; s < n01; s++) issue_kv(s);
    float *yl = (float *)(lds + QA_YL), *red = yl + 32;
    uint32_t L[4][24];
    float xs[4], xz[4];
    const uint32_t team = tid / 32, tl = tid % 32, b = tl >> 1, hh = tl & 1;
    {
        constexpr int NIT = H / (4 * QA_T);  // 4 elements per thread and pass
        const float *xr = (const float *)(lds + QA_X), *wr = xr + H;
        f32x4 v[NIT], w[NIT];
        float sq = 0.f;
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            v[it] = *(const f32x4 *)(xr + (it * QA_T + tid) * 4);
            if (P.xb) {
                const zh_fix *dq = (const zh_fix *)(lds + qa_slot<SH>(0)) + (it * QA_T + tid) * 4;
                v[it].x += fix_to_f(dq[0]); v[it].y += fix_to_f(dq[1]);
                v[it].z += fix_to_f(dq[2]); v[it].w += fix_to_f(dq[3]);
                if ((it * QA_T + tid) * 4 / S::RROWS == blockIdx.x)  // this workgroup's rows
                    *(f32x4 *)(P.x_out + (it * QA_T + tid) * 4) = v[it];
            }
            w[it] = *(const f32x4 *)(wr + (it * QA_T + tid) * 4);
            sq = fmaf(v[it].x, v[it].x, sq); sq = fmaf(v[it].y, v[it].y, sq);
            sq = fmaf(v[it].z, v[it].z, sq); sq = fmaf(v[it].w, v[it].w, sq);
        }
        sq = wave_sum(sq);
        if (lane == 0) red[wave] = sq;
        lds_bar();  // (also: every x / weight value is in registers before the image overwrites them)
        if (!wa && P.xb && P.kv_defer == 0 && n01 > 0) issue_kv(0);  // xb is read: sub-chunk 0's slot is free
        if (P.zero && tid < S::RROWS) P.zero[blockIdx.x * S::RROWS + tid] = 0;
        float tot = 0.f;
#pragma unroll
        for (int w8 = 0; w8 < 8; w8++) tot += red[w8];
        const float rms_inv = 1.0f / sqrtf(tot / (float)H + p.eps);
        uint8_t *xqa = lds + QA_X;
        float *ixs = (float *)(xqa + QA_NB * 2 * RG_SEG), *ixz = ixs + QA_NB * 8;
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const uint32_t e0 = (it * QA_T + tid) * 4;
            f32x4 u = v[it];
            u.x = w[it].x * (u.x * rms_inv); u.y = w[it].y * (u.y * rms_inv);
            u.z = w[it].z * (u.z * rms_inv); u.w = w[it].w * (u.w * rms_inv);
            const float a = row8_max(fmaxf(fmaxf(fabsf(u.x), fabsf(u.y)), fmaxf(fabsf(u.z), fabsf(u.w))));
            float inv, sc;
            xq_scales(a, inv, sc);
            int X[4] = {xq_quant(u.x, inv), xq_quant(u.y, inv), xq_quant(u.z, inv), xq_quant(u.w, inv)};
            int l0[4], l1[4], l2[4];
#pragma unroll
            for (int q = 0; q < 4; q++) xq_limbs(X[q], l0[q], l1[q], l2[q]);
            const uint32_t blk = e0 / 32, lo = e0 % 32;
            uint8_t *dst = xqa + (blk / 4) * RG_SEG + (blk % 4) * 96 + lo;
            *(uint32_t *)(dst) = pack4(l0[0], l0[1], l0[2], l0[3]);
            *(uint32_t *)(dst + 32) = pack4(l1[0], l1[1], l1[2], l1[3]);
            *(uint32_t *)(dst + 64) = pack4(l2[0], l2[1], l2[2], l2[3]);
            int sm = X[0] + X[1] + X[2] + X[3];
            sm += __builtin_amdgcn_update_dpp(0, sm, 0xB1, 0xF, 0xF, false);
            sm += __builtin_amdgcn_update_dpp(0, sm, 0x4E, 0xF, 0xF, false);
            const uint32_t sub = tid & 7;
            if (sub == 0) ixs[blk] = sc;
            if ((sub & 3) == 0) ixz[blk * 2 + (sub >> 2)] = (float)sm * sc;
        }
        lds_bar();
        if (!S::Q8) {
            // this lane's half super-block: limbs, block scales and sums
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t jb = b * 8 + 4 * hh + q;
                lds_load_limbs(L[q], xqa + tl * RG_SEG + q * 96);
                xs[q] = ixs[jb];
                xz[q] = ixz[2 * jb] + ixz[2 * jb + 1];
            }
        } else {
            // Q8_0 (K = 2048): this lane's blocks 2 tl and 2 tl + 1
#pragma unroll
            for (int q = 0; q < 2; q++) {
                lds_load_limbs(L[q], xqa + (tl / 2) * RG_SEG + (tl % 2) * 192 + q * 96);
                xs[q] = ixs[2 * tl + q];
            }
        }
        lds_bar();  // the image is read: the region takes K/V sub-chunk 2
    }
    ZH_TRACE_POINT(2);
    if (!wa && P.kv_defer < 2 && nsub > 2) issue_kv(2);

    // ---- the slice's rows (the ring DMMV's per-row arithmetic)
    if (wa) wait_vm<0>();
    lds_bar();
    if (!wa && P.kv_defer == 2)
        for (uint32_t s = 0; s < nsub; s++) issue_kv(s);
    ZH_TRACE_POINT(3);
#pragma unroll
    for (uint32_t ps = 0; ps < NP; ps++) {
        const uint32_t r = ps * 16 + team;
        if (r < R) {  // uniform per wave (R % 4 == 0)
            float res;
            if constexpr (S::Q8) {
                // Q8_0 blocks 2 tl and 2 tl + 1 of the row: 68 bytes from a
                // 4-byte aligned start (f16 d, 32 int8; f16 d, 32 int8)
                const uint32_t *wp = (const uint32_t *)(lds + QA_W + r * QA_ROWB + tl * 68);
                uint32_t wd[17];
#pragma unroll
                for (int i = 0; i < 17; i++) wd[i] = wp[i];
                int D0[3] = {0, 0, 0}, D1[3] = {0, 0, 0};
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const uint32_t q0 = __builtin_amdgcn_alignbyte(wd[i + 1], wd[i], 2), q1 = wd[9 + i];
#pragma unroll
                    for (int k = 0; k < 3; k++) {
                        D0[k] = sdot4(q0, L[0][k * 8 + i], D0[k]);
                        D1[k] = sdot4(q1, L[1][k * 8 + i], D1[k]);
                    }
                }
                res = fmaf(h2f(wd[0]) * xs[0], comb_f(D0[0], D0[1], D0[2]),
                           h2f(wd[8] >> 16) * xs[1] * comb_f(D1[0], D1[1], D1[2]));
            } else {
                const uint8_t *blk = lds + QA_W + r * QA_ROWB + b * 144;
                uint32_t hd[4], qs[16];
                {
                    const u32x4 v = *(const u32x4 *)blk;
                    hd[0] = v.x; hd[1] = v.y; hd[2] = v.z; hd[3] = v.w;
    #pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const u32x4 w = *(const u32x4 *)(blk + 16 + 64 * hh + 16 * i);
                        qs[4 * i] = w.x; qs[4 * i + 1] = w.y; qs[4 * i + 2] = w.z; qs[4 * i + 3] = w.w;
                    }
                }
                const LpbQ4K::Hdr hdr = LpbQ4K::header(hd);
                const uint32_t scw = hh ? hdr.scB : hdr.scA, mw = hh ? hdr.mB : hdr.mA;
                float accd = 0.f, accm = 0.f;
    #pragma unroll
                for (int pl = 0; pl < 2; pl++) {
                    int D[2][3] = {{0, 0, 0}, {0, 0, 0}};
    #pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const uint32_t w = qs[8 * pl + i];
                        const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    #pragma unroll
                        for (int k = 0; k < 3; k++) {
                            D[0][k] = sdot4(lo, L[2 * pl][k * 8 + i], D[0][k]);
                            D[1][k] = sdot4(hi, L[2 * pl + 1][k * 8 + i], D[1][k]);
                        }
                    }
                    const float sc0 = ubyte_f(scw, 2 * pl), sc1 = ubyte_f(scw, 2 * pl + 1);
                    const float m0 = ubyte_f(mw, 2 * pl), m1 = ubyte_f(mw, 2 * pl + 1);
                    const float S0 = (float)comb_i(D[0][0], D[0][1], D[0][2]);
                    const float S1 = (float)comb_i(D[1][0], D[1][1], D[1][2]);
                    accd = fmaf(sc0 * xs[2 * pl], S0, accd);
                    accd = fmaf(sc1 * xs[2 * pl + 1], S1, accd);
                    accm = fmaf(m0, xz[2 * pl], accm);
                    accm = fmaf(m1, xz[2 * pl + 1], accm);
                }
                res = fmaf(hdr.d, accd, -hdr.dmin * accm);
            }
            res = team_sum_dpp<32>(res);
            if (tl == 0) yl[r] = res;
        }
    }
    lds_bar();
    ZH_TRACE_POINT(4);
    if (!wa && nsub > 3) issue_kv(3);  // the weight rows are read: their region takes sub-chunk 3
    // ---- publish the rows as epoch-tagged words (wave 0): word rr of XCD h
    // is row rr of its q | k | v rows (zh_xcd.h tag_store)
    uint64_t *xr = P.xrows + (size_t)h * QA_XROWS;
    if (wave == 0 && lane < R) tag_store(xr + j * R + lane, yl[lane], E);
    ZH_TRACE_POINT(5);
    // ---- the attention's inputs: the XCD's q, the new k | v, polled from
    // the L2 as they arrive (waves 0 .. NXW - 1, 128 words each) into LDS
    uint8_t *sm = lds + QA_W;  // q [G][128] f32 (QC KB), k_new | v_new (1 KB), new K / V rows f16, q fragments
    constexpr uint32_t NXW = (QR + 2 * FD_HD) / 128;
    __shared__ uint32_t s_okw[QA_AW];
    if (wave < NXW) {
        float v2[2];
        const bool okw = tag_wait<2>(xr + wave * 128, E, p.ctl, v2);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint32_t rr = wave * 128 + 64 * i + lane;
            ((float *)sm)[rr < QR ? rr : QC * 256 + rr - QR] = v2[i];
        }
        if (lane == 0) s_okw[wave] = okw ? 1u : 0u;
    }
    ZH_TRACE_POINT(6);
    wait_vm<0>();  // every K/V sub-chunk
    lds_bar();
    bool ok_rows = true;
#pragma unroll
    for (uint32_t w = 0; w < NXW; w++) ok_rows = ok_rows && s_okw[w] != 0;
    ZH_TRACE_POINT(7);
    // ---- WITH_O: this workgroup's O rows (128 rows x the XCD's two
    // super-blocks, 36 KB) into the weight region's free part, by waves 4-7
    // while the attention runs (HBM is idle from here on)
    // (SH 4: after the attention, its sub-chunk 3 occupies the region)
    auto issue_o = [&]() __attribute__((always_inline)) {
        constexpr uint32_t WO_ROWB = S::Q8 ? 4 * QA_NXCD * FD_HD / 32 * 34 : 16 * 144;  // a W_o row (4096 columns)
        constexpr uint32_t PCS = QA_OROWB / 16;  // 16-byte pieces of a row's columns of the XCD
        static_assert(QA_OROWS * QA_OROWB % 1024 == 0 && QA_OROWB % 16 == 0, "whole copies");
        for (uint32_t c = wl4; c < QA_OROWS * QA_OROWB / 1024; c += 4) {
            const uint32_t pc = c * 64 + lane, row = pc / PCS, within = pc - row * PCS;
            dma16(P.wo + (size_t)(j * QA_OROWS + row) * WO_ROWB + h * QA_OROWB + within * 16, lds0 + QA_OW + c * 1024);
        }
    };
    if (WITH_O && nsub <= 3 && !wa) issue_o();  // (more sub-chunks: after the attention, see below)
    // ---- q as MFMA fragments (RMSNorm, RoPE, f16 hi + lo), shared through LDS
    const uint32_t sub = lane & 7, fg = lane & 15, fq = lane >> 4;
    const uint32_t gq = wave / 4, w4 = wave % 4;
    const float *qw = (const float *)(lds + QA_NRM), *kw = qw + FD_HD;
    const float *cs = (const float *)(lds + QA_ROPE);
    uint16_t *knew16 = (uint16_t *)(sm + (QC + 1) * 1024), *vnew16 = knew16 + FD_HD;
    uint8_t *frag = sm + (QC + 2) * 1024;
    float *rinv = (float *)(frag + 8 * 64 * 16);
    half4 qh[8], ql[8];
    {
        for (uint32_t g = wave; g < (uint32_t)G; g += QA_AW) {
            const float *qs = (const float *)sm + g * FD_HD;
            const float a = qs[lane], bb = qs[lane + 64];
            const float sq = wave_sum(fmaf(a, a, bb * bb));
            if (lane == 0) rinv[g] = 1.0f / sqrtf(sq / (float)FD_HD + p.eps);
        }
        lds_bar();
        if (wave < 4) {
            const uint32_t pi = wave;  // steps pi (dims < 64) and pi + 4 (their RoPE partners)
            const float *qs = (const float *)sm + min(fg, (uint32_t)G - 1) * FD_HD;
            const f32x4 va = *(const f32x4 *)(qs + 16 * pi + 4 * fq), vb = *(const f32x4 *)(qs + 64 + 16 * pi + 4 * fq);
            float lo[4] = {va.x, va.y, va.z, va.w}, hi[4] = {vb.x, vb.y, vb.z, vb.w};
            const float ri = rinv[min(fg, (uint32_t)G - 1)];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t i = 16 * pi + 4 * fq + e;  // dims i and i + 64
                const float a = qw[i] * (lo[e] * ri);
                const float bb = qw[i + 64] * (hi[e] * ri);
                const float co = cs[2 * i], sn = cs[2 * i + 1];
                lo[e] = a * co - bb * sn;
                hi[e] = a * sn + bb * co;
            }
            half4 h0, l0, h1, l1;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float x0 = fg < (uint32_t)G ? lo[e] : 0.f, y0 = fg < (uint32_t)G ? hi[e] : 0.f;
                h0[e] = (_Float16)x0;
                l0[e] = (_Float16)(x0 - (float)h0[e]);
                h1[e] = (_Float16)y0;
                l1[e] = (_Float16)(y0 - (float)h1[e]);
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
    ZH_TRACE_POINT(8);
    // ---- the new token's k (norm + RoPE) and v as f16 rows (the owner only)
    const bool owner = posv >= t0 && posv < t1;  // uniform
    if (owner && wave == 0) {
        const float *kn = (const float *)(sm + QC * 1024), *vn = kn + FD_HD;
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
        norm_rope16(klo, khi, wlo, whi, co, sn, p.eps);
        if (lane < 8) {
            *(u32x4 *)(knew16 + sub * 8) = u32x4{pack_h2(klo[0], klo[1]), pack_h2(klo[2], klo[3]),
                                                 pack_h2(klo[4], klo[5]), pack_h2(klo[6], klo[7])};
            *(u32x4 *)(knew16 + 64 + sub * 8) = u32x4{pack_h2(khi[0], khi[1]), pack_h2(khi[2], khi[3]),
                                                      pack_h2(khi[4], khi[5]), pack_h2(khi[6], khi[7])};
        }
        *(uint32_t *)(vnew16 + 2 * lane) = pack_h2(vn[2 * lane], vn[2 * lane + 1]);
    }
    const uint32_t s_own = owner ? (posv - t0) / AR_TS : ~0u, r_own = owner ? (posv - t0) % AR_TS : 0u;
    lds_bar();
    // substitute the new row for the copy (which predates it); sub-chunk 4
    // is copied later, into sub-chunk 0's slot
    auto substitute = [&]() __attribute__((always_inline)) {
        uint8_t *Ks = lds + qa_slot<SH>(s_own);
        const uint32_t pc = ((tid & 15) ^ (r_own & 15)) * 16;
        if (tid < 16) *(u32x4 *)(Ks + r_own * 256 + pc) = *(const u32x4 *)((const uint8_t *)knew16 + tid * 16);
        else if (tid < 32)
            *(u32x4 *)(Ks + AR_SLOT / 2 + r_own * 256 + pc) = *(const u32x4 *)((const uint8_t *)vnew16 + (tid - 16) * 16);
    };
    if (owner && s_own < nsub && s_own < 4) substitute();  // (later sub-chunks: once copied)
    lds_bar();

    // ---- scores and P V over the landed sub-chunks: group gq (4 waves) takes
    // sub-chunks gq, gq + 2 (, 4); wave w4 of a group tokens 16 w4 .. 16 w4 + 15
    float m_run = -INFINITY, l_run = 0.f;
    floatx4 acc[8];
#pragma unroll
    for (int n = 0; n < 8; n++) acc[n] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t it = 0; 2 * it < nsub; it++) {  // uniform: group gq takes sub-chunk 2 it + gq
        if (nsub > 4 && it >= 1) {  // (at most four sub-chunks: all copied before the loop)
            // sub-chunks 2 it - 2 and 2 it - 1 are read: their slots take 2 it
            // + 2 and 2 it + 3; from step 2 on, wait for this step's 2 it and
            // 2 it + 1 (copied one step earlier)
            const uint32_t nnew = nsub > 2 * it + 2 ? min(nsub - (2 * it + 2), 2u) : 0u;
            if (nnew) {
                lds_bar();
                if (!wa)
                    for (uint32_t s2 = 2 * it + 2; s2 < 2 * it + 2 + nnew; s2++) issue_kv(s2);
            }
            if (it >= 2) {
                if (!wa) wait_vm_dyn(nnew * 8);
                lds_bar();
                if (owner && s_own >= 4 && s_own / 2 == it) {
                    substitute();
                    lds_bar();
                }
            }
        }
        const uint32_t s = 2 * it + gq;
        if (s >= nsub) continue;  // uniform per wave
        const uint8_t *Ks = lds + qa_slot<SH>(s), *Vs = Ks + AR_SLOT / 2;
        const uint32_t ts = t0 + s * AR_TS, tb = w4 * 16;
        half4 kf[8], vf[8];
        {
            const uint32_t t = tb + fg;
#pragma unroll
            for (int s8 = 0; s8 < 8; s8++)
                kf[s8] = *(const half4 *)(Ks + t * 256 + (((2 * s8 + (fq >> 1)) ^ (t & 15)) * 16) + 8 * (fq & 1));
            // P V's column j of MFMA tile n is dim 8 j + n, so a lane's
            // operands are dims 8 fg .. 8 fg + 7 of its 4 tokens: one 16-byte
            // piece of each token's row. V rows past the chunk are zeroed,
            // not only weighted 0: they copy the cache's row of the new token,
            // which this launch has not written yet and may hold anything
            // (NaN after a step whose waits gave up), and 0 x NaN is NaN
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
        floatx4 d1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s8 = 0; s8 < 8; s8++) {
            d1 = __builtin_amdgcn_mfma_f32_16x16x16f16(kf[s8], qh[s8], d1, 0, 0, 0);
            d1 = __builtin_amdgcn_mfma_f32_16x16x16f16(kf[s8], ql[s8], d1, 0, 0, 0);
        }
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; r++) sc[r] = ts + tb + 4 * fq + r < t1 ? d1[r] * p.scale : -INFINITY;
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
            const _Float16 hv = (_Float16)pr[r];
            ph[r] = hv;
            pl[r] = (_Float16)(pr[r] - (float)hv);
        }
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
    ZH_TRACE_POINT(9);
    // ---- the new row to the cache
    if (owner && tid < 32) {
        uint16_t *dst = (tid < 16 ? p.kc : p.vc) + ((size_t)kvh * p.cache_tokens + posv) * FD_HD + (tid & 15) * 8;
        *(u32x4 *)dst = *(const u32x4 *)((const uint8_t *)(tid < 16 ? knew16 : vnew16) + (tid & 15) * 16);
    }
    // ---- combine the waves (in sub-chunk 0's slot), publish the partials
    float *wm = (float *)lds, *wl = wm + QA_AW * G, *wo = wl + QA_AW * G;
    lds_bar();
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint32_t g = 4 * fq + r;
        if (g < (uint32_t)G) {  // dims 8 fg .. 8 fg + 7 of head g: two 16-byte stores
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
    if (nsub) {
        for (uint32_t o = tid; o < (uint32_t)G * FD_HD; o += QA_T) {
            const uint32_t g = o / FD_HD, d = o % FD_HD;
            float M = wm[g];
#pragma unroll
            for (int w = 1; w < QA_AW; w++) M = fmaxf(M, wm[w * G + g]);
            const float Ms = M == -INFINITY ? 0.f : M;
            float O = 0.f, Ls = 0.f;
#pragma unroll
            for (int w = 0; w < QA_AW; w++) {
                const float f = wm[w * G + g] == -INFINITY ? 0.f : expf(wm[w * G + g] - Ms);
                O = fmaf(wo[(w * G + g) * FD_HD + d], f, O);
                Ls = fmaf(wl[w * G + g], f, Ls);
            }
            float *pp = p.part + ((size_t)(h * G + g) * p.n_chunks + j) * (FD_HD + 2);
            pp[d] = O;
            if (d == 0) {
                pp[FD_HD] = M;
                pp[FD_HD + 1] = Ls;
            }
        }
        wait_vm<0>();  // every wave's partial stores are in the L2 ...
        __syncthreads();
        if (tid == 0) *(volatile uint32_t *)(fl_p + j) = E;  // ... before the flag
    }
    ZH_TRACE_POINT(10);
    if (!WITH_O) {
        if (j >= (uint32_t)G) return;
        // ---- merger j: q head h G + j, once every chunk of the kv head published
        const bool ok = xcd_wait(fl_p, nv, E, p.ctl, tid);
        ZH_TRACE_POINT(11);
        if (j == 0 && tid == 0 && ok && ok_rows) *(volatile uint32_t *)ep = E;  // every workgroup of the head has read the epoch (a wait that gave up leaves the words to zh_sync's reset)
        attn_merge<1, 32, false, true>(p, h * G + j, nv, !(ok && ok_rows));
        ZH_TRACE_POINT(12);
        return;
    }
    if (nsub > 3 && !wa) issue_o();  // (the O rows' region held sub-chunk slot 3)
    // ---- WITH_O: every workgroup of the XCD merges the XCD's G heads itself
    // (their partials are in this XCD's L2) into LDS, as the XQ image of
    // the O projection's 4 G blocks of 32 (no second publication round)
    const bool ok = xcd_wait(fl_p, nv, E, p.ctl, tid);
    ZH_TRACE_POINT(11);
    if (j == 0 && tid == 0 && ok && ok_rows) *(volatile uint32_t *)ep = E;  // every workgroup of the head has read the epoch (a wait that gave up leaves the words to zh_sync's reset)
    float *mo = (float *)(lds + QA_X + 4096);  // merged heads [G][128]
    {
        AttnP pm = p;
        pm.out = nullptr;
        pm.xq = nullptr;
        attn_merge<G, 32, false, true, QA_T>(pm, h * G, nv, false, mo);
    }
    ZH_TRACE_POINT(12);
    __syncthreads();
    {
        const XQView v = xq_view(lds + QA_X, 4 * G);  // limbs [4G][96], xs [4G], xsum [4G][2]
        if (tid < (uint32_t)G * FD_HD) xq_store_block32(mo[tid], tid & 31, v, tid / 32);
        lds_bar();
        wait_vm<0>();  // the O rows' copies (waves 4-7)
        lds_bar();
    }
    const uint8_t *xlimb = lds + QA_X;
    const float *oxs = (const float *)(lds + QA_X + 4 * G * 96), *oxz = oxs + 4 * G;
    if constexpr (S::Q8) {
        // lane: row r = tid / 8 of the 64, blocks 2 q8 and 2 q8 + 1 of the
        // XCD's 16 (Q8_0: 68 bytes from a 4-byte aligned start)
        const uint32_t q8 = tid & 7, r = tid >> 3;
        uint32_t Lo[2][24];
#pragma unroll
        for (int k = 0; k < 2; k++) lds_load_limbs(Lo[k], xlimb + (2 * q8 + k) * 96);
        const uint32_t *wp = (const uint32_t *)(lds + QA_OW + r * QA_OROWB + q8 * 68);
        uint32_t wd[17];
#pragma unroll
        for (int i = 0; i < 17; i++) wd[i] = wp[i];
        int D0[3] = {0, 0, 0}, D1[3] = {0, 0, 0};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t q0 = __builtin_amdgcn_alignbyte(wd[i + 1], wd[i], 2), q1 = wd[9 + i];
#pragma unroll
            for (int k = 0; k < 3; k++) {
                D0[k] = sdot4(q0, Lo[0][k * 8 + i], D0[k]);
                D1[k] = sdot4(q1, Lo[1][k * 8 + i], D1[k]);
            }
        }
        float res = fmaf(h2f(wd[0]) * oxs[2 * q8], comb_f(D0[0], D0[1], D0[2]),
                         h2f(wd[8] >> 16) * oxs[2 * q8 + 1] * comb_f(D1[0], D1[1], D1[2]));
        res = team_sum_dpp<8>(res);
        if (!(ok && ok_rows)) res = __builtin_nanf("");  // a wait gave up: the rows' sums are poisoned
        if (q8 == 0) {
            if (P.xb) fix_add((zh_fix *)P.x_acc + j * QA_OROWS + r, res);
            else __hip_atomic_fetch_add((float *)P.x_acc + j * QA_OROWS + r, res, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else {
        // lane: row r = tid / 4 of the 128, half super-block q = tid % 4 of the
        // XCD's 4 G half-blocks (G = 4; fewer heads leave lanes idle)
        const uint32_t q = tid & 3, r = tid >> 2;
        const bool act = q < (uint32_t)G;  // 2 G / 2 half-blocks
        const uint32_t qq = act ? q : 0;
        uint32_t Lo[4][24];
        float oxs4[4], oxz4[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t jb = 4 * qq + k;
            lds_load_limbs(Lo[k], xlimb + jb * 96);
            oxs4[k] = oxs[jb];
            oxz4[k] = oxz[2 * jb] + oxz[2 * jb + 1];
        }
        const uint8_t *blk = lds + QA_OW + r * QA_OROWB + (qq >> 1) * 144;
        const uint32_t hh = qq & 1;
        uint32_t hd[4], qs[16];
        {
            const u32x4 v = *(const u32x4 *)blk;
            hd[0] = v.x; hd[1] = v.y; hd[2] = v.z; hd[3] = v.w;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const u32x4 w = *(const u32x4 *)(blk + 16 + 64 * hh + 16 * i);
                qs[4 * i] = w.x; qs[4 * i + 1] = w.y; qs[4 * i + 2] = w.z; qs[4 * i + 3] = w.w;
            }
        }
        const LpbQ4K::Hdr hdr = LpbQ4K::header(hd);
        const uint32_t scw = hh ? hdr.scB : hdr.scA, mw = hh ? hdr.mB : hdr.mA;
        float accd = 0.f, accm = 0.f;
#pragma unroll
        for (int pl = 0; pl < 2; pl++) {
            int D[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t w = qs[8 * pl + i];
                const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                for (int k = 0; k < 3; k++) {
                    D[0][k] = sdot4(lo, Lo[2 * pl][k * 8 + i], D[0][k]);
                    D[1][k] = sdot4(hi, Lo[2 * pl + 1][k * 8 + i], D[1][k]);
                }
            }
            const float sc0 = ubyte_f(scw, 2 * pl), sc1 = ubyte_f(scw, 2 * pl + 1);
            const float m0 = ubyte_f(mw, 2 * pl), m1 = ubyte_f(mw, 2 * pl + 1);
            const float S0 = (float)comb_i(D[0][0], D[0][1], D[0][2]);
            const float S1 = (float)comb_i(D[1][0], D[1][1], D[1][2]);
            accd = fmaf(sc0 * oxs4[2 * pl], S0, accd);
            accd = fmaf(sc1 * oxs4[2 * pl + 1], S1, accd);
            accm = fmaf(m0, oxz4[2 * pl], accm);
            accm = fmaf(m1, oxz4[2 * pl + 1], accm);
        }
        float res = act ? fmaf(hdr.d, accd, -hdr.dmin * accm) : 0.f;
        res = team_sum_dpp<4>(res);
        if (!(ok && ok_rows)) res = __builtin_nanf("");  // a wait gave up: the rows' sums are poisoned
        if (q == 0) {
            if (P.xb) fix_add((zh_fix *)P.x_acc + j * QA_OROWS + r, res);
            else __hip_atomic_fetch_add((float *)P.x_acc + j * QA_OROWS + r, res, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // a wait gave up: the fixed-point sums cannot carry a NaN, so the
    // workgroup's rows of the plain part become NaN instead (written by the
    // threads that stored them above, so in program order after them)
    if (P.x_out && !(ok && ok_rows)) {
#pragma unroll
        for (int it = 0; it < (int)(H / (4 * QA_T)); it++)
            if ((it * QA_T + tid) * 4 / S::RROWS == blockIdx.x)
                *(f32x4 *)(P.x_out + (it * QA_T + tid) * 4) = f32x4{__builtin_nanf(""), __builtin_nanf(""),
                                                                     __builtin_nanf(""), __builtin_nanf("")};
    }
    ZH_TRACE_POINT(13);
}

ZH_TRACE_DUMP_FN(zh_debug_trace_qa)

// Whether the workgroups of a 256-workgroup grid (one per CU) land on XCDs
// (blockIdx + s) % 8 for one s: the placement k_qkv_attn's (kv head, slice)
// assignment relies on (otherwise a slice would be missing and its waits
// would give up).
__global__ __launch_bounds__(64) void k_xcd_probe(uint32_t *out) {
    extern __shared__ uint8_t lds_probe[];
    if (threadIdx.x == 0) {
        lds_probe[0] = 0;
        out[blockIdx.x] = xcc_id();
    }
}

bool zhk_xcd_round_robin(zh_ctx *c) {
    if (c->xcd_rr >= 0) return c->xcd_rr != 0;
    c->xcd_rr = 0;
    if (c->cu_count != (int)(QA_NXCD * QA_PER)) return false;
    uint32_t *d = nullptr, h[QA_NXCD * QA_PER];
    if (hipMalloc((void **)&d, sizeof h) != hipSuccess) return false;
    bool ok = false;
    // 96 KB of LDS: one workgroup per CU, as k_qkv_attn
    if (hipFuncSetAttribute((const void *)k_xcd_probe, hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024) ==
        hipSuccess) {
        hipLaunchKernelGGL(k_xcd_probe, dim3(QA_NXCD * QA_PER), dim3(64), 96 * 1024, c->stream, d);
        if (hipStreamSynchronize(c->stream) == hipSuccess &&
            hipMemcpy(h, d, sizeof h, hipMemcpyDeviceToHost) == hipSuccess) {
            ok = h[0] < QA_NXCD;
            for (uint32_t i = 0; i < QA_NXCD * QA_PER; i++) ok = ok && h[i] == (h[0] + i) % QA_NXCD;
        }
    }
    hipFree(d);
    c->xcd_rr = ok ? 1 : 0;
    return ok;
}

uint32_t zhk_qkv_attn_flag_words() { return QA_FLAG_WORDS; }
uint64_t zhk_qkv_attn_xrows_bytes() { return 8ull * QA_NXCD * QA_XROWS; }

// Whether k_qkv_attn takes a model of this shape on this context.
bool zhk_qkv_attn_supported(zh_ctx *c, uint32_t hidden, uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_ctx) {
    const uint32_t G = nkv ? nh / nkv : 0;
    const bool s3 = hidden == QaS<3>::H && nkv == QA_NXCD && nh == G * nkv && (G == 1 || G == 2 || G == 4) &&
                    max_ctx <= QA_PER * QaS<3>::MAXSUB * AR_TS;  // (the merge's 32 chunks of up to 2048 tokens)
    const bool s4 = hidden == QaS<4>::H && nkv == QA_NXCD / QaS<4>::KVX && nh == 4 * QA_NXCD &&
                    max_ctx <= QA_PER * QaS<4>::MAXSUB * AR_TS;
    return (s3 || s4) && hd == FD_HD && !c->concurrent && zhk_xcd_round_robin(c);
}

int zhk_qkv_attn(zh_ctx *c, const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x,
                 const float *norm_w, float *q, float *k, float *v, const float *qw, const float *kw,
                 const float *rope_cs, uint16_t *kc, uint16_t *vc, uint32_t cache_tokens, float *out, void *xq_out,
                 uint32_t nh, zh_pos_src pos, float scale, float eps, float *partials, uint32_t *flags,
                 const uint8_t *wo, void *x_acc, const zh_fix *xb, float *x_out, zh_fix *zero, uint32_t hidden,
                 uint64_t *xrows) {
    QaP P = {};
    AttnP &p = P.a;
    p.q = q; p.k_new = k; p.v_new = v; p.q_norm = qw; p.k_norm = kw; p.rope_cs = rope_cs;
    p.kc = kc; p.vc = vc; p.pages = nullptr; p.n_pages = 0; p.cache_tokens = cache_tokens; p.pos = pos;
    p.scale = scale; p.eps = eps; p.part = partials; p.n_chunks = QA_PER; p.counters = nullptr;
    p.out = out; p.xq = (uint8_t *)xq_out; p.nq = nh; p.nd = QA_PER; p.no_wait = 0; p.ident = 1; p.ctl = c->err_dev;
    P.wq = wq; P.wk = wk; P.wv = wv; P.x = x; P.norm_w = norm_w; P.flags = flags;
    P.wo = wo; P.x_acc = x_acc; P.xb = xb; P.x_out = x_out; P.zero = zero; P.xrows = xrows;
    P.kv_defer = xb || hidden != QaS<3>::H ? 0u : (uint32_t)zh_knob_int("ZH_QA_DEFER", 0);
    if (xb && (!wo || !x_out || !zero || ((uintptr_t)xb & 15) || ((uintptr_t)x_out & 15)))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "qkv_attn: split residual needs the O phase and aligned rows");
    const uint32_t G = nh / QA_NXCD;
    if (!xrows || (wo && (!x_acc || ((uintptr_t)wo & 15))) || !pos.dev || ((uintptr_t)x & 15) || ((uintptr_t)norm_w & 15) || ((uintptr_t)wq & 15) || ((uintptr_t)wk & 15) ||
        ((uintptr_t)wv & 15))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "qkv_attn: device position and 16-byte aligned operands");
#define QA_L(GG, WO, SS)                                                                                         \
    {                                                                                                            \
        static bool attr = false;                                                                                \
        if (!attr) {                                                                                             \
            ZH_HIP(c, hipFuncSetAttribute((const void *)k_qkv_attn<GG, WO, SS>,                                  \
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)QaS<SS>::LDS));       \
            attr = true;                                                                                         \
        }                                                                                                        \
        hipLaunchKernelGGL((k_qkv_attn<GG, WO, SS>), dim3(QA_NXCD * QA_PER), dim3(QA_T), QaS<SS>::LDS, c->stream, \
                           P);                                                                                   \
        break;                                                                                                   \
    }
    if (wo && G != 4) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "qkv_attn: O phase needs 4 q heads per kv head");
    if (hidden != QaS<3>::H && (hidden != QaS<4>::H || G != 4))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "qkv_attn: hidden %u with %u q heads", hidden, nh);
    switch (G + (wo ? 100 : 0) + (hidden == QaS<4>::H ? 1000 : 0)) {
    case 1: QA_L(1, false, 3)
    case 2: QA_L(2, false, 3)
    case 4: QA_L(4, false, 3)
    case 104: QA_L(4, true, 3)
    case 1004: QA_L(4, false, 4)
    case 1104: QA_L(4, true, 4)
    default: return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "qkv_attn: GQA group %u", G);
    }
#undef QA_L
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
