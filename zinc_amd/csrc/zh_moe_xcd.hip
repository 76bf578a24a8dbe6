// zh_moe_xcd.hip — the sparse-MoE FFN of one decode layer (ffn_norm, router
// + top-k, the selected experts' gate/up + SwiGLU and down, the weighted sum
// added to the residual) in one launch, one selected expert per XCD (hidden
// 2048, 128 experts, top-8, expert FFN 768; Q8_0 router, Q4_K experts).
//
// Replaces five dispatches of the reference's MoE decode step: ffn_norm, the
// router DMMV, softmax_topk, the experts' gate/up/SwiGLU and down DMMVs and
// the weighted accumulation (forward.zig:5958-6500; softmax_topk_v2.comp,
// dmmv_q4k.comp, moe_weighted_acc.comp).
//
// The 32 workgroups of XCD h (zh_xcd.h; slot j):
//   1. stage ffn_norm(x) as XQ limbs and compute router rows [4 j, 4 j + 4)
//      (every XCD computes all 128 logits, bit-identically, from the same
//      bytes) and publish them in the XCD's L2 as epoch-tagged 64-bit words
//      (zh_xcd.h tag_store), which every workgroup polls;
//   2. every workgroup's polling wave takes the top 8 of the 128 logits
//      itself (eight rounds of a wave maximum; the lowest index wins ties)
//      and their weights (softmax over the selected logits) — XCD h takes
//      the h-th selected expert e and its weight;
//   3. workgroup j: gate and up rows [24 j, 24 j + 24) of expert e and their
//      SwiGLU, published to the XCD (tagged words), while expert e's down rows
//      [64 j, 64 j + 64) (the unmodified Q4_K bytes) stream in behind the
//      gate/up tiles;
//   4. every workgroup reads the XCD's 768 SwiGLU values, quantises them as
//      XQ limbs and adds its 64 down rows, times the expert's weight, into the
//      residual with device atomics.
// Every exchange stays inside an XCD; the only device-wide traffic is the
// final atomics (8 per row, one per expert).
//
// x is not y, which changes during the launch: either a copy of the
// residual taken before it (the O projection writes both), or the split
// residual of the fused attention launch (zh_engine.hip): x = xa + xb, this
// workgroup's 8 rows of x stored into xout, 8 rows of `zero` cleared.
#include "zh_ring_q4k.h"
#include "zh_xcd.h"

namespace {
constexpr uint32_t MX_H = 2048, MX_E = 128, MX_K = 8, MX_F = 768;
constexpr uint32_t MX_NB = MX_H / 256;                 // Q4_K super-blocks per gate/up row (8)
constexpr uint32_t MX_RROW = MX_H / 32 * 34;           // router row bytes (Q8_0, 2176)
constexpr uint32_t MX_RPW = MX_E / XCD_PER;            // router rows per workgroup (4)
constexpr uint32_t MX_FR = MX_F / XCD_PER;             // FFN rows per workgroup (24)
constexpr uint32_t MX_DR = MX_H / XCD_PER;             // down rows of each workgroup (64)
constexpr uint32_t MX_DNB = MX_F / 256;                // Q4_K super-blocks per down row (3)
constexpr uint32_t MX_DROWB = MX_DNB * 144;            // a down row (432 B)
constexpr uint32_t MX_DCH = MX_DR * MX_DROWB / 1024;   // the workgroup's down rows as 1 KB copies (27)
constexpr uint32_t MX_GT = 2;                          // gate/up tiles (24 rows, 16 per pass)
constexpr uint32_t MX_RT = (RG_D - 1) * RG_TILE;       // router rows staged in the third ring slot
constexpr uint32_t MX_RAW = RG_D * RG_TILE + RG_XQ_BYTES;  // x | norm staging, then the SwiGLU values
static_assert(MX_RPW * MX_RROW <= 9 * 1024 && MX_DR * MX_DROWB % 1024 == 0 && MX_DCH * 1024 <= RG_TILE,
              "router rows in 9 copies; the down rows in whole copies in one ring slot");
static_assert(MX_DR * 8 == RG_T && MX_F % 64 == 0 && MX_F * 4 <= RG_RAW_BYTES, "down: 8 lanes per row");
}  // namespace

// Flag words (zero when the engine is created): [0, 512) unused (the
// exchanged values carry epoch tags), [512, 520) epochs.
constexpr uint32_t MX_FLAG_WORDS = 2 * XCD_N * XCD_PER + XCD_N;

struct MoeP {
    const float *x;               // residual copy (or its plain part, xa)
    const zh_fix *xb;             // split residual: its atomic part, fixed point (else nullptr)
    float *xout;                  // split residual: x = xa + xb stored
    zh_fix *zero;                 // split residual: the vector to clear
    const float *norm_w;          // ffn_norm weight
    float eps;
    const uint8_t *router;        // Q8_0 [128][2048]
    const uint8_t *egate, *eup;   // Q4_K [128][768][2048]
    const uint8_t *edown;         // Q4_K [128][2048][768]
    void *y;                      // residual: += sum_k w_k down_k (zh_fix with the split residual, else f32)
    uint64_t *logits;             // [8 XCDs][128] tagged router logits (exchanged inside each XCD)
    uint64_t *xsw;                // [8 XCDs][768] tagged SwiGLU values (exchanged inside each XCD)
    uint32_t *routing;            // [ids x 8][weights x 8] of the selection, written by workgroup 0 (for inspection)
    const uint32_t *force;        // test hook: 8 expert ids to run instead of the selection (else nullptr)
    uint32_t *flags;              // MX_FLAG_WORDS
    uint32_t *ctl;                // [0] error word, [1] wait limit
};

__global__ __launch_bounds__(RG_T, 1) void k_moe_xcd(MoeP P) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ uint32_t s_route[2 * MX_K];
    constexpr int NB = MX_NB, MODE = LPB_GATE_UP;
    using TT = Q4Tiles<NB, MODE>;
    constexpr int TL = TT::TL, RPP = TT::RPP;
    constexpr uint32_t NBLK = NB * 8;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t h = min(xcc_id(), XCD_N - 1), j = blockIdx.x / XCD_N, w = h * XCD_PER + j;
    uint32_t *fl_p = P.flags + XCD_N * XCD_PER + h * XCD_PER;
    uint32_t *ep = P.flags + 2 * XCD_N * XCD_PER + h;
    const uint32_t E = *(const __attribute__((address_space(4))) uint32_t *)ep + 1u;
    const uint32_t lds0 = lds_addr(lds);
    uint8_t *ring = lds, *xqa = lds + RG_D * RG_TILE, *raw = lds + MX_RAW;
    float *yl = (float *)(lds + RG_D * RG_TILE + RG_XQ_BYTES + RG_RAW_BYTES), *red = yl + 2 * RG_MAXROWS;
    ZH_TRACE_POINT(0);
    ZH_TRACE_VALUE(h + 1);  // (the XCD, + 1: a slot of 0 reads as unset)

    // ---- x, the norm weight (8 KB each: one copy per wave) and this
    // workgroup's router rows (8.5 KB: 9 copies, the last clamped)
    dma16((const uint8_t *)P.x + wave * 1024 + lane * 16, lds0 + MX_RAW + wave * 1024);
    dma16((const uint8_t *)P.norm_w + wave * 1024 + lane * 16, lds0 + MX_RAW + NB * 1024 + wave * 1024);
    if (P.xb)  // (8 bytes per element: 2 copies per wave)
        for (uint32_t i = 0; i < 2; i++)
            dma16((const uint8_t *)P.xb + (wave + 8 * i) * 1024 + lane * 16,
                  lds0 + MX_RAW + 2 * NB * 1024 + (wave + 8 * i) * 1024);
    {
        const uint8_t *rr = P.router + (size_t)j * MX_RPW * MX_RROW;
        for (uint32_t c = wave; c < 9; c += 8)
            dma16(rr + min(c * 1024 + lane * 16, MX_RPW * MX_RROW - 16), lds0 + MX_RT + c * 1024);
    }
    wait_vm<0>();
    lds_bar();
    ZH_TRACE_POINT(1);
    // ---- ffn_norm(x) as the XQ image (4 elements per thread)
    float *ixs = (float *)(xqa + NB * 2 * RG_SEG), *ixz = ixs + NBLK;
    {
        const float *xr = (const float *)raw, *wr = xr + MX_H;
        const uint32_t e0 = tid * 4;
        f32x4 v = *(const f32x4 *)(xr + e0);
        if (P.xb) {
            const zh_fix *dq = (const zh_fix *)(wr + MX_H) + e0;
            v.x += fix_to_f(dq[0]); v.y += fix_to_f(dq[1]); v.z += fix_to_f(dq[2]); v.w += fix_to_f(dq[3]);
            if (e0 / (MX_H / 256) == blockIdx.x) *(f32x4 *)(P.xout + e0) = v;  // this workgroup's 8 rows
            if (tid < MX_H / 256) P.zero[blockIdx.x * (MX_H / 256) + tid] = 0;
        }
        const f32x4 wn = *(const f32x4 *)(wr + e0);
        float sq = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, v.w * v.w)));
        sq = wave_sum(sq);
        if (lane == 0) red[wave] = sq;
        lds_bar();
        float tot = 0.f;
#pragma unroll
        for (int w8 = 0; w8 < 8; w8++) tot += red[w8];
        const float rms_inv = 1.0f / sqrtf(tot / (float)MX_H + P.eps);
        v.x = wn.x * (v.x * rms_inv); v.y = wn.y * (v.y * rms_inv);
        v.z = wn.z * (v.z * rms_inv); v.w = wn.w * (v.w * rms_inv);
        const float a = row8_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        float inv, sc;
        xq_scales(a, inv, sc);
        int X[4] = {xq_quant(v.x, inv), xq_quant(v.y, inv), xq_quant(v.z, inv), xq_quant(v.w, inv)};
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
        lds_bar();
    }
    // ---- router rows [4 j, 4 j + 4): wave r < 4 takes row r, lane = its
    // 32-element block (Q8_0: f16 d, 32 int8; blocks 34 bytes apart)
    if (wave < MX_RPW) {
        const uint32_t off = MX_RT + wave * MX_RROW + lane * 34, sh = off & 3;
        const uint32_t *wp = (const uint32_t *)(lds + (off & ~3u));
        uint32_t wd[10];
#pragma unroll
        for (int i = 0; i < 10; i++) wd[i] = wp[i];
        const uint32_t dw = __builtin_amdgcn_alignbyte(wd[1], wd[0], sh);
        const uint8_t *lb = xqa + (lane / 4) * RG_SEG + (lane % 4) * 96;
        int D[3] = {0, 0, 0};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // int8 quants i*4 .. i*4+3 at byte off + 2 + 4 i
            const uint32_t q = sh ? wd[i + 1] : __builtin_amdgcn_alignbyte(wd[i + 1], wd[i], 2);
#pragma unroll
            for (int k = 0; k < 3; k++) D[k] = sdot4(q, ((const uint32_t *)(lb + 32 * k))[i], D[k]);
        }
        float v = h2f(dw) * (ixs[lane] * comb_f(D[0], D[1], D[2]));
        v = wave_sum(v);
        if (lane == 0) tag_store(P.logits + h * MX_E + j * MX_RPW + wave, v, E);
    }
    // ---- gate/up lanes: their half super-block of x in registers (before
    // the SwiGLU limbs overwrite anything near the image)
    const uint32_t team = tid / TL, tl = tid % TL, b = tl >> 1, hh = tl & 1;
    uint32_t L[4][24];
    float xs[4], xz[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t jb = b * 8 + 4 * hh + q;
        lds_load_limbs(L[q], xqa + tl * RG_SEG + q * 96);
        xs[q] = ixs[jb];
        xz[q] = ixz[2 * jb] + ixz[2 * jb + 1];
    }
    // ---- the XCD's 128 logits (wave 0, as they arrive); the top 8 in the
    // same wave: eight rounds of a wave maximum over the logits not yet
    // taken, the lowest index among equal values first (the order of
    // topk_softmax_wave: value descending, lowest index first); a NaN logit
    // is never taken (a NaN router leaves ids past the experts: clamped below)
    __shared__ float s_lg[MX_E];
    __shared__ uint32_t s_okr;
    if (wave == 0) {
        float lv[2];
        const bool okr = tag_wait<2>(P.logits + h * MX_E, E, P.ctl, lv);
        s_lg[lane] = lv[0];
        s_lg[lane + 64] = lv[1];
        if (lane == 0) s_okr = okr ? 1u : 0u;
        ZH_TRACE_POINT(2);
        bool t0 = false, t1 = false;  // taken
        uint32_t id = 0xFFFFFFFFu;    // lane k < 8: the k-th selected expert
        float lsel = -INFINITY;       //   and its logit
#pragma unroll
        for (int k = 0; k < (int)MX_K; k++) {
            const float a0 = t0 ? -INFINITY : lv[0], a1 = t1 ? -INFINITY : lv[1];
            const float m = wave_max(fmaxf(a0, a1));
            const uint64_t b0 = __builtin_amdgcn_ballot_w64(!t0 && lv[0] == m);
            const uint64_t b1 = __builtin_amdgcn_ballot_w64(!t1 && lv[1] == m);
            const uint32_t i = b0 ? (uint32_t)__builtin_ctzll(b0) : b1 ? 64u + (uint32_t)__builtin_ctzll(b1) : 0xFFFFFFFFu;
            if (lane == (uint32_t)k) { id = i; lsel = m; }
            t0 = t0 || lane == i;
            t1 = t1 || lane + 64 == i;
        }
        ZH_TRACE_POINT(6);
        // weights: softmax over the selected logits (rank 0 holds the max)
        const float l0 = lane_f(lsel, 0);
        const float ex = lane < MX_K && id < MX_E ? expf(lsel - l0) : 0.f;
        const float sm = wave_sum(ex);
        if (lane < MX_K) {
            s_route[lane] = id;
            ((float *)s_route)[MX_K + lane] = ex / sm;
        }
        __builtin_amdgcn_wave_barrier();  // (one wave: its LDS accesses complete in order)
        if (blockIdx.x == 0 && lane < 2 * MX_K) P.routing[lane] = s_route[lane];
        if (P.force) {
            // run the given experts, weighted by the softmax over their own
            // logits (the selection above stays the recorded one)
            const uint32_t fe = lane < MX_K ? min(P.force[lane], MX_E - 1) : 0u;
            const float fl = lane < MX_K ? s_lg[fe] : -INFINITY;
            const float fm = wave_max(fl);
            const float fx = lane < MX_K ? expf(fl - fm) : 0.f;
            const float fs = wave_sum(fx);
            __builtin_amdgcn_wave_barrier();
            if (lane < MX_K) {
                s_route[lane] = fe;
                ((float *)s_route)[MX_K + lane] = fx / fs;
            }
        }
    }
    lds_bar();
    const bool ok_r = s_okr != 0;
    uint32_t e = s_route[h];
    if (e >= MX_E) {  // a NaN router: clamp, as the per-group kernels do
        if (tid == 0) __hip_atomic_fetch_or(P.ctl, ZH_DEVERR_EXPERT_ID, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        e = MX_E - 1;
    }
    e = __builtin_amdgcn_readfirstlane(e);
    const float wexp = __builtin_bit_cast(float, s_route[MX_K + h]);
    ZH_TRACE_POINT(3);

    // ---- the stream: gate/up tiles 0, 1 of expert e, then its down rows
    // [64 j, +64) (unmodified Q4_K, 27 KB) into the third slot
    RingP p = {};
    p.M = MX_F; p.K = MX_H; p.nseg = 1; p.rpw = MX_FR;
    const size_t gstride = (size_t)MX_F * NB * 144;
    p.segW[0] = P.egate + e * gstride; p.segW[1] = p.segW[0]; p.segW[2] = p.segW[0];
    p.W2 = P.eup + e * gstride;
    p.seg_end[0] = MX_F; p.seg_end[1] = MX_F; p.seg_end[2] = MX_F;
    const TT tiles(p, j, tid, lds);
    const uint32_t tcw = tiles.tcw;
    tiles.issue(0, 0);
    tiles.issue(1, 1);
    const uint32_t dcw = wave < MX_DCH % 8 ? MX_DCH / 8 + 1 : MX_DCH / 8;
    {
        const uint8_t *dr = P.edown + ((size_t)e * MX_H + (size_t)j * MX_DR) * MX_DROWB;
#pragma unroll
        for (uint32_t i = 0; i < (MX_DCH + 7) / 8; i++) {
            const uint32_t c = wave + 8 * i;
            if (c < MX_DCH) dma16(dr + c * 1024 + lane * 16, lds0 + 2 * RG_TILE + c * 1024);
        }
    }
    {
        const uint32_t mrow = team / RPP, trow = team % RPP;
        for (uint32_t u = 0; u < MX_GT; u++) {
            // copies still allowed in flight: tile 1 (u = 0) and the down rows
            wait_vm_dyn(dcw + (u == 0 ? tcw : 0u));
            lds_bar();
            const uint8_t *blk = ring + (u % RG_D) * RG_TILE + team * TT::ROWB + b * 144;
            uint32_t hd[4], qs[16];
            {
                const u32x4 vv = *(const u32x4 *)blk;
                hd[0] = vv.x; hd[1] = vv.y; hd[2] = vv.z; hd[3] = vv.w;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const u32x4 q4 = *(const u32x4 *)(blk + 16 + 64 * hh + 16 * i);
                    qs[4 * i] = q4.x; qs[4 * i + 1] = q4.y; qs[4 * i + 2] = q4.z; qs[4 * i + 3] = q4.w;
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
                    const uint32_t q = qs[8 * pl + i];
                    const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
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
            float res = fmaf(hdr.d, accd, -hdr.dmin * accm);
            res = team_sum_dpp<TL>(res);
            if (tl == 0) yl[mrow * RG_MAXROWS + u * RPP + trow] = res;
        }
    }
    lds_bar();
    ZH_TRACE_POINT(4);
    // ---- SwiGLU of the 24 rows, published to the XCD as epoch-tagged words
    // [XCD][768]; wave 0 then reads the XCD's 768 values into LDS
    float *swv = (float *)(lds + MX_RAW);  // [768]
    __shared__ uint32_t s_oks;
    if (wave == 0) {
        if (lane < MX_FR)
            tag_store(P.xsw + (size_t)h * MX_F + j * MX_FR + lane, silu_mul(yl[lane], yl[RG_MAXROWS + lane]), E);
        float v[MX_F / 64];
        const bool oks = tag_wait<MX_F / 64>(P.xsw + (size_t)h * MX_F, E, P.ctl, v);
#pragma unroll
        for (int i = 0; i < (int)(MX_F / 64); i++) swv[lane + 64 * i] = v[i];
        if (lane == 0) s_oks = oks ? 1u : 0u;
    }
    lds_bar();
    const bool ok_s = s_oks != 0;
    // every workgroup of the XCD published, so every one has read the epoch
    // (a wait that gave up leaves the words to zh_sync's reset)
    if (j == 0 && tid == 0 && ok_r && ok_s) *(volatile uint32_t *)ep = E;
    ZH_TRACE_POINT(5);
    // ---- the 768 values as the XQ image (waves 0-2, 4 elements per thread)
    {
        float *ixs2 = (float *)(xqa + MX_DNB * 2 * RG_SEG), *ixz2 = ixs2 + MX_DNB * 8;
        if (tid < MX_F / 4) {
            const uint32_t e0 = tid * 4;
            const f32x4 u = *(const f32x4 *)(swv + e0);
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
            if (sub == 0) ixs2[blk] = sc;
            if ((sub & 3) == 0) ixz2[blk * 2 + (sub >> 2)] = (float)sm * sc;
        }
        wait_vm<0>();  // the down rows
        lds_bar();
        // ---- down: lane (row r = tid / 8, half super-block hb = tid % 8 < 6)
        const uint32_t r = tid >> 3, hb = tid & 7;
        float res = 0.f;
        if (hb < 2 * MX_DNB) {
            const uint32_t bb = hb >> 1, h2 = hb & 1;
            uint32_t Ld[4][24];
            float dxs[4], dxz[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t jb = bb * 8 + 4 * h2 + q;
                lds_load_limbs(Ld[q], xqa + hb * RG_SEG + q * 96);
                dxs[q] = ixs2[jb];
                dxz[q] = ixz2[2 * jb] + ixz2[2 * jb + 1];
            }
            const uint8_t *blk = lds + 2 * RG_TILE + r * MX_DROWB + bb * 144;
            uint32_t hd[4], qs[16];
            {
                const u32x4 vv = *(const u32x4 *)blk;
                hd[0] = vv.x; hd[1] = vv.y; hd[2] = vv.z; hd[3] = vv.w;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const u32x4 q4 = *(const u32x4 *)(blk + 16 + 64 * h2 + 16 * i);
                    qs[4 * i] = q4.x; qs[4 * i + 1] = q4.y; qs[4 * i + 2] = q4.z; qs[4 * i + 3] = q4.w;
                }
            }
            const LpbQ4K::Hdr hdr = LpbQ4K::header(hd);
            const uint32_t scw = h2 ? hdr.scB : hdr.scA, mw = h2 ? hdr.mB : hdr.mA;
            float accd = 0.f, accm = 0.f;
#pragma unroll
            for (int pl = 0; pl < 2; pl++) {
                int D[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const uint32_t q = qs[8 * pl + i];
                    const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                    for (int k = 0; k < 3; k++) {
                        D[0][k] = sdot4(lo, Ld[2 * pl][k * 8 + i], D[0][k]);
                        D[1][k] = sdot4(hi, Ld[2 * pl + 1][k * 8 + i], D[1][k]);
                    }
                }
                const float sc0 = ubyte_f(scw, 2 * pl), sc1 = ubyte_f(scw, 2 * pl + 1);
                const float m0 = ubyte_f(mw, 2 * pl), m1 = ubyte_f(mw, 2 * pl + 1);
                const float S0 = (float)comb_i(D[0][0], D[0][1], D[0][2]);
                const float S1 = (float)comb_i(D[1][0], D[1][1], D[1][2]);
                accd = fmaf(sc0 * dxs[2 * pl], S0, accd);
                accd = fmaf(sc1 * dxs[2 * pl + 1], S1, accd);
                accm = fmaf(m0, dxz[2 * pl], accm);
                accm = fmaf(m1, dxz[2 * pl + 1], accm);
            }
            res = fmaf(hdr.d, accd, -hdr.dmin * accm);
        }
        res = team_sum_dpp<8>(res) * wexp;
        if (!(ok_r && ok_s)) res = __builtin_nanf("");  // a wait gave up
        if (hb == 0) {
            if (P.xb) fix_add((zh_fix *)P.y + j * MX_DR + r, res);
            else __hip_atomic_fetch_add((float *)P.y + j * MX_DR + r, res, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // a wait gave up: the fixed-point sums cannot carry a NaN, so the
    // workgroup's rows of the plain part become NaN instead (written by the
    // threads that stored them, so in program order after them)
    if (P.xb && !(ok_r && ok_s) && (tid * 4) / (MX_H / 256) == blockIdx.x)
        *(f32x4 *)(P.xout + tid * 4) = f32x4{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""),
                                             __builtin_nanf("")};
    ZH_TRACE_POINT(7);
}

ZH_TRACE_DUMP_FN(zh_debug_trace_moe)

uint32_t zhk_moe_xcd_flag_words() { return MX_FLAG_WORDS; }
uint64_t zhk_moe_part_bytes() { return (uint64_t)XCD_N * (MX_E + MX_F) * 8; }

bool zhk_moe_xcd_supported(zh_ctx *c, uint32_t hidden, uint32_t n_experts, uint32_t n_used, uint32_t expert_ffn) {
    return hidden == MX_H && n_experts == MX_E && n_used == MX_K && expert_ffn == MX_F && !c->concurrent &&
           zhk_xcd_round_robin(c);
}

int zhk_moe_xcd(zh_ctx *c, const float *x, const float *norm_w, float eps, const uint8_t *router,
                const uint8_t *egate, const uint8_t *eup, const uint8_t *edown, void *y, void *scratch,
                uint32_t *routing, uint32_t *flags, const zh_fix *xb, float *xout, zh_fix *zero,
                const uint32_t *force) {
    if (((uintptr_t)x & 15) || ((uintptr_t)norm_w & 15) || ((uintptr_t)router & 15) || ((uintptr_t)egate & 15) ||
        ((uintptr_t)eup & 15) || ((uintptr_t)edown & 15) || ((uintptr_t)scratch & 15) || !y || !routing ||
        (xb && (((uintptr_t)xb & 15) || ((uintptr_t)xout & 15) || !zero)))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "moe_xcd: 16-byte aligned operands");
    MoeP P = {};
    P.x = x; P.xb = xb; P.xout = xout; P.zero = zero; P.norm_w = norm_w; P.eps = eps; P.router = router; P.egate = egate; P.eup = eup; P.edown = edown; P.y = y;
    P.logits = (uint64_t *)scratch; P.xsw = P.logits + XCD_N * MX_E;
    P.routing = routing; P.force = force; P.flags = flags; P.ctl = c->err_dev;
    static bool attr = false;
    if (!attr) {
        ZH_HIP(c, hipFuncSetAttribute((const void *)k_moe_xcd, hipFuncAttributeMaxDynamicSharedMemorySize, (int)RG_LDS));
        attr = true;
    }
    hipLaunchKernelGGL(k_moe_xcd, dim3(XCD_N * XCD_PER), dim3(RG_T), RG_LDS, c->stream, P);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
