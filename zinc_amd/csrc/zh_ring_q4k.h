// zh_ring_q4k.h — the streaming Q4_K DMMV body shared by the one-launch
// kernel (zh_dmmv_ring.hip) and the persistent decode-layers kernel
// (zh_step.hip).
//
// One 512-thread workgroup per CU owns a contiguous range of output rows. Its
// weight rows stream HBM -> LDS through a ring of three 36 KB tiles with the
// asynchronous global_load_lds DMA (16 bytes per lane, one contiguous 1 KB
// run per wave instruction, so every load is fully coalesced and no
// registers hold tile data in flight): two tiles are in flight while the
// third is computed. The activation is staged once per workgroup (DMA into
// LDS, RMS-normalised and quantised to XQ limbs there) and each lane then
// keeps the limbs of its half super-block in registers, so the inner loop
// reads only weight bytes from LDS (80 B per lane and row). Outputs are
// buffered in LDS and written after the loop.
//
// Every global load of the body is a DMA issued from inline assembly, so the
// compiler tracks none of them and each wait is explicit: a wave waits
// (s_waitcnt vmcnt) for its own DMA instructions of the tile it needs, then
// a barrier makes the whole tile visible. A compiler-generated wait would be
// vmcnt(0), draining the ring.
//
// COH (the persistent kernel): the activation was written by other
// workgroups of the same launch, possibly on another XCD, so it is read with
// system-scope DMA (past this XCD's L2), and every output another workgroup
// reads is stored at device scope.
#pragma once
#include "zh_device.h"
#include "zh_internal.h"
#include "zh_lpb_common.h"

#pragma clang diagnostic ignored "-Winline-asm"

namespace {

constexpr int RG_T = 512;                       // threads (8 waves, 2 per SIMD)
constexpr uint32_t RG_TILE = 36864;             // bytes per tile = one pass of the workgroup
constexpr uint32_t RG_CH = RG_TILE / 1024;      // 1 KB DMA chunks per tile
constexpr int RG_D = 3;                         // tiles in the ring
constexpr uint32_t RG_MAXROWS = 128;            // output rows per workgroup
constexpr uint32_t RG_XQ_BYTES = 16384;         // LDS for the XQ image of K <= 4096 (14.3 KB used)
constexpr uint32_t RG_RAW_BYTES = 32768;        // LDS for the f32 activation and norm weights
constexpr uint32_t RG_LDS = RG_D * RG_TILE + RG_XQ_BYTES + RG_RAW_BYTES + 2 * RG_MAXROWS * 4 + 64;
// COH layout: the f32 activation and norm weights are staged in the last
// ring slot, which the ring first fills after the activation is in
// registers (the persistent kernel shares its LDS with other phases)
constexpr uint32_t RG_LDS_COH = RG_D * RG_TILE + RG_XQ_BYTES + 2 * RG_MAXROWS * 4 + 64;
template <bool COH> constexpr uint32_t rg_raw_off() { return COH ? (RG_D - 1) * RG_TILE : RG_D * RG_TILE + RG_XQ_BYTES; }
template <bool COH> constexpr uint32_t rg_yl_off() { return RG_D * RG_TILE + RG_XQ_BYTES + (COH ? 0 : RG_RAW_BYTES); }
static_assert(RG_RAW_BYTES <= RG_TILE, "staging fits a ring slot");

}  // namespace

struct RingP {
    const float *x;        // f32 activation (XIN 0/1)
    const float *norm_w;   // RMSNorm weight (XIN 1)
    float eps;
    const uint8_t *xq;     // XQ activation (XIN 2)
    uint32_t M, K, nseg, acc, rpw;  // output rows, K, segments, y +=, output rows per workgroup
    const uint8_t *segW[3];
    const uint8_t *W2;     // up matrix (gate/up mode)
    float *segY[3];
    uint32_t seg_end[3];
    uint8_t *xq_out;       // gate/up: SwiGLU output also as XQ (optional)
    uint32_t *grp_cnt;
};

// Stacked segments (Q | K | V) addressed by offsets: the address of a row's
// bytes is w0 + row * row_bytes plus 64-bit deltas selected by comparisons.
// An indexed kernel-argument array (or a select the compiler turns into one)
// would be read with vector or scratch loads whose vmcnt(0) wait drains the
// DMA ring.
struct RingSegs {
    uint64_t w0, dw1, dw2, y0, dy1, dy2;
    uint32_t e0, e1;
    ZH_DEVM RingSegs(const RingP &p, uint32_t row_bytes) {
        const uint64_t w1 = (uint64_t)(uintptr_t)p.segW[1] - (uint64_t)p.seg_end[0] * row_bytes;
        const uint64_t w2 = (uint64_t)(uintptr_t)p.segW[2] - (uint64_t)p.seg_end[1] * row_bytes;
        const uint64_t y1 = (uint64_t)(uintptr_t)p.segY[1] - (uint64_t)p.seg_end[0] * 4;
        const uint64_t y2 = (uint64_t)(uintptr_t)p.segY[2] - (uint64_t)p.seg_end[1] * 4;
        w0 = (uint64_t)(uintptr_t)p.segW[0];
        y0 = (uint64_t)(uintptr_t)p.segY[0];
        dw1 = w1 - w0; dw2 = w2 - w1; dy1 = y1 - y0; dy2 = y2 - y1;
        e0 = p.nseg > 1 ? p.seg_end[0] : 0xFFFFFFFFu;
        e1 = p.nseg > 2 ? p.seg_end[1] : 0xFFFFFFFFu;
    }
    ZH_DEVM const uint8_t *w(uint32_t row, uint32_t row_bytes) const {
        const uint64_t a = w0 + (uint64_t)row * row_bytes + (row >= e0 ? dw1 : 0ull) + (row >= e1 ? dw2 : 0ull);
        return (const uint8_t *)(uintptr_t)a;
    }
    ZH_DEVM float *y(uint32_t row) const {
        return (float *)(uintptr_t)(y0 + (uint64_t)row * 4 + (row >= e0 ? dy1 : 0ull) + (row >= e1 ? dy2 : 0ull));
    }
};

// Padded LDS image of the XQ limbs: the 384 limb bytes of each 128-element
// half super-block (four 32-element blocks) at a 400-byte stride, so the 16
// lanes reading 16 consecutive half-blocks hit distinct banks.
constexpr uint32_t RG_SEG = 400;

// The ring's geometry and tile copies for workgroup wg: tile t (output rows
// r0 + t RPP ..) into ring slot s. Chunk c = wave + 8 i (i < 5): waves 0..3
// issue 5 chunks, 4..7 issue 4.
template <int NB, int MODE>
struct Q4Tiles {
    static constexpr int TL = 2 * NB;                  // lanes per row: half a super-block each
    static constexpr int TPP = RG_T / TL;              // rows (teams) per pass
    static constexpr int NM = MODE == LPB_GATE_UP ? 2 : 1;
    static constexpr int RPP = TPP / NM;               // output rows per pass
    static constexpr uint32_t ROWB = NB * 144;
    static_assert(TPP * ROWB == RG_TILE, "one pass covers one tile");
    uint32_t r0, r1, nt, wave, lane, tcw, lds0;
    RingSegs sgs;
    uint64_t dup;
    ZH_DEVM Q4Tiles(const RingP &p, uint32_t wg, uint32_t tid, const uint8_t *lds) : sgs(p, ROWB) {
        lane = tid & 63;
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        r0 = wg * p.rpw;
        r1 = min(p.M, r0 + p.rpw);
        nt = r0 < p.M ? (r1 - r0 + RPP - 1) / RPP : 0u;
        tcw = wave < RG_CH % 8 ? RG_CH / 8 + 1 : RG_CH / 8;
        lds0 = lds_addr(lds);
        dup = (uint64_t)(uintptr_t)p.W2 - (uint64_t)(uintptr_t)p.segW[0];  // gate/up: up - gate
    }
    // tiles copied before the ring's first wait (the others follow as slots free)
    ZH_DEVM uint32_t prologue() const { return min(nt, (uint32_t)RG_D - 1); }
    ZH_DEVM void issue(uint32_t t, uint32_t s) const {
#pragma unroll
        for (uint32_t i = 0; i < (RG_CH + 7) / 8; i++) {
            const uint32_t c = wave + 8 * i;
            if (c < RG_CH) {  // uniform per wave
                const uint32_t o = c * 1024 + lane * 16;
                const uint32_t team = o / ROWB, within = o - team * ROWB;
                const uint32_t m = NM == 2 ? team / RPP : 0;
                // rows past the range re-read the range's last row (discarded)
                const uint32_t row = min(r0 + t * RPP + (NM == 2 ? team % RPP : team), r1 - 1);
                const uint8_t *src;
                if (NM == 2) {
                    src = sgs.w(row, ROWB) + (m ? dup : 0ull) + within;
                } else {
                    src = sgs.w(row, ROWB) + within;
                }
                dma16(src, lds0 + s * RG_TILE + c * 1024);
            }
        }
    }
};

// The persistent kernel copies a phase's first tiles while it waits at the
// grid barrier before the phase (the weights do not depend on the previous
// phase); returns the count, the body's `pre`.
template <int NB, int MODE>
ZH_DEV uint32_t q4k_ring_prefetch(const RingP &p, uint32_t wg, uint8_t *lds) {
    const Q4Tiles<NB, MODE> tl(p, wg, phase_tid(), lds);
    const uint32_t n = tl.prologue();
    for (uint32_t t = 0; t < n; t++) tl.issue(t, t);
    return n;
}

// NB = K / 256 super-blocks per row (8 or 16); MODE LPB_PLAIN or LPB_GATE_UP;
// XIN 0: f32 x, 1: f32 x with fused RMSNorm, 2: XQ x. pre: tiles 0 .. pre-1
// already copied (q4k_ring_prefetch), before the activation's copy.
template <int NB, int MODE, int XIN, bool COH>
ZH_DEV void q4k_ring_body(const RingP &p, uint32_t wg, uint8_t *lds, uint32_t pre = 0) {
    using TT = Q4Tiles<NB, MODE>;
    constexpr int TL = TT::TL, NM = TT::NM, RPP = TT::RPP;
    constexpr uint32_t NBLK = NB * 8;           // 32-element blocks of x
    uint8_t *ring = lds;
    uint8_t *xqa = lds + RG_D * RG_TILE;        // XQ image (global XQ layout)
    uint8_t *raw = lds + rg_raw_off<COH>();     // f32 x [K], norm weight [K]
    float *yl = (float *)(lds + rg_yl_off<COH>());  // [NM][RG_MAXROWS]
    float *red = yl + 2 * RG_MAXROWS;           // [8]
    const uint32_t tid = COH ? phase_tid() : threadIdx.x, lane = tid & 63;
    const TT tiles(p, wg, tid, lds);
    const uint32_t wave = tiles.wave, r0 = tiles.r0, r1 = tiles.r1, nt = tiles.nt, lds0 = tiles.lds0;
    if (nt == 0) return;  // (persistent kernel: more workgroups than row ranges)
    const RingSegs &sgs = tiles.sgs;
    ZH_TRACE_POINT(0);

    // ---- activation DMA (NB chunks of 1 KB per vector: NB / 8 per wave)
    if (XIN == 2) {
        const uint32_t xq_bytes = NBLK * 108;
#pragma unroll
        for (int i = 0; i < NB / 8; i++) {
            const uint32_t c = wave + 8 * i;
            dma16_act<COH>(p.xq + min(c * 1024 + lane * 16, xq_bytes - 16), lds0 + rg_raw_off<COH>() + c * 1024);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NB / 8; i++) {
            const uint32_t c = wave + 8 * i;
            dma16_act<COH>((const uint8_t *)p.x + c * 1024 + lane * 16, lds0 + rg_raw_off<COH>() + c * 1024);
            if (XIN == 1)
                dma16((const uint8_t *)p.norm_w + c * 1024 + lane * 16,
                      lds0 + rg_raw_off<COH>() + NB * 1024 + c * 1024);
        }
    }

    const uint32_t tcw = tiles.tcw;
    auto issue_tile = [&](uint32_t t, uint32_t s) __attribute__((always_inline)) { tiles.issue(t, s); };
    const uint32_t npro = tiles.prologue();
    for (uint32_t t = pre; t < npro; t++) issue_tile(t, t);

    // ---- the activation as XQ in LDS (the tiles it precedes are still in
    // flight; prefetched tiles precede it and have landed with it)
    wait_vm_dyn((npro - pre) * tcw);
    lds_bar();
    ZH_TRACE_POINT(1);
    // image: padded limbs [NB*2][RG_SEG], then xs [NBLK], xsum [NBLK][2]
    float *ixs = (float *)(xqa + NB * 2 * RG_SEG), *ixz = ixs + NBLK;
    if (XIN == 2) {
        const XQView xv = xq_view(raw, NBLK);
        for (uint32_t q = tid; q < NBLK * 6; q += RG_T) {  // 16-byte limb chunks
            const uint32_t j = q / 6, part = q % 6;
            *(u32x4 *)(xqa + (j / 4) * RG_SEG + (j % 4) * 96 + part * 16) = *(const u32x4 *)((const uint8_t *)xv.limb + q * 16);
        }
        for (uint32_t j = tid; j < NBLK; j += RG_T) {
            ixs[j] = xv.xs[j];
            ixz[2 * j] = xv.xsum[2 * j];
            ixz[2 * j + 1] = xv.xsum[2 * j + 1];
        }
        lds_bar();
    } else {
        const float *xr = (const float *)raw, *wr = (const float *)(raw + NB * 1024);
        float rms_inv = 1.f;
        if (XIN == 1) {
            float sq = 0.f;
#pragma unroll
            for (int it = 0; it < NB / 8; it++) {
                const f32x4 v = *(const f32x4 *)(xr + (it * RG_T + tid) * 4);
                sq = fmaf(v.x, v.x, sq); sq = fmaf(v.y, v.y, sq); sq = fmaf(v.z, v.z, sq); sq = fmaf(v.w, v.w, sq);
            }
            sq = wave_sum(sq);
            if (lane == 0) red[wave] = sq;
            lds_bar();
            float tot = 0.f;
#pragma unroll
            for (int w = 0; w < 8; w++) tot += red[w];
            rms_inv = 1.0f / sqrtf(tot / (float)p.K + p.eps);
        }
        // 8 lanes per 32-element block, 4 consecutive elements per lane
#pragma unroll
        for (int it = 0; it < NB / 8; it++) {
            const uint32_t e0 = (it * RG_T + tid) * 4;
            f32x4 v = *(const f32x4 *)(xr + e0);
            if (XIN == 1) {
                const f32x4 w = *(const f32x4 *)(wr + e0);
                v.x = w.x * (v.x * rms_inv); v.y = w.y * (v.y * rms_inv);
                v.z = w.z * (v.z * rms_inv); v.w = w.w * (v.w * rms_inv);
            }
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
            sm += __builtin_amdgcn_update_dpp(0, sm, 0xB1, 0xF, 0xF, false);  // 16 elements = 4 lanes
            sm += __builtin_amdgcn_update_dpp(0, sm, 0x4E, 0xF, 0xF, false);
            const uint32_t sub = tid & 7;
            if (sub == 0) ixs[blk] = sc;
            if ((sub & 3) == 0) ixz[blk * 2 + (sub >> 2)] = (float)sm * sc;
        }
        lds_bar();
    }

    // ---- this lane's half super-block: limbs, block scales and sums in registers
    const uint32_t team = tid / TL, tl = tid % TL, b = tl >> 1, h = tl & 1;
    uint32_t L[4][24];
    float xs[4], xz[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint32_t j = b * 8 + 4 * h + q;
        lds_load_limbs(L[q], xqa + tl * RG_SEG + q * 96);
        xs[q] = ixs[j];
        xz[q] = ixz[2 * j] + ixz[2 * j + 1];
    }
    ZH_TRACE_POINT(2);

    // ---- the ring
    const uint32_t mrow = NM == 2 ? team / RPP : 0, trow = NM == 2 ? team % RPP : team;
    for (uint32_t t = 0; t < nt; t++) {
        wait_vm_dyn(min(nt - 1 - t, (uint32_t)RG_D - 2) * tcw);
        lds_bar();
        if (t + RG_D - 1 < nt) issue_tile(t + RG_D - 1, (t + RG_D - 1) % RG_D);
        const uint8_t *blk = ring + (t % RG_D) * RG_TILE + team * TT::ROWB + b * 144;
        uint32_t hd[4], qs[16];
        {
            const u32x4 v = *(const u32x4 *)blk;
            hd[0] = v.x; hd[1] = v.y; hd[2] = v.z; hd[3] = v.w;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const u32x4 w = *(const u32x4 *)(blk + 16 + 64 * h + 16 * i);
                qs[4 * i] = w.x; qs[4 * i + 1] = w.y; qs[4 * i + 2] = w.z; qs[4 * i + 3] = w.w;
            }
        }
        const LpbQ4K::Hdr hh = LpbQ4K::header(hd);
        const uint32_t scw = h ? hh.scB : hh.scA, mw = h ? hh.mB : hh.mA;
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
        float res = fmaf(hh.d, accd, -hh.dmin * accm);
        res = team_sum_dpp<TL>(res);
        const uint32_t i = t * RPP + trow;
        if (tl == 0 && i < RG_MAXROWS) yl[mrow * RG_MAXROWS + i] = res;
    }
    lds_bar();
    ZH_TRACE_POINT(3);

    // ---- outputs
    const uint32_t nrow = r1 - r0;
    if (MODE == LPB_GATE_UP) {
        float *Y = p.segY[0];
        for (uint32_t i = tid; i < nrow; i += RG_T) {
            const float v = silu_mul(yl[i], yl[RG_MAXROWS + i]);
            if (COH || p.xq_out) st_dev(Y + r0 + i, v);  // device scope: read by other workgroups
            else Y[r0 + i] = v;
        }
        if (p.xq_out) {
            // The SwiGLU output as XQ for the down projection: each 32-row
            // group is counted up to 32 published rows; the workgroup whose
            // rows complete it quantises the group's block. Rows were stored
            // at device scope, so after this workgroup's stores drain they are
            // visible to whichever workgroup's counter increment comes last.
            __shared__ uint32_t s_last[LPB_XQ_MAX_GROUPS];
            const uint32_t g0 = r0 / 32, ng = (r1 - 1) / 32 - g0 + 1;
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (tid < ng) {
                const uint32_t g = g0 + tid;
                const uint32_t n = min(r1, g * 32 + 32) - max(r0, g * 32);
                const uint32_t prev = __hip_atomic_fetch_add(p.grp_cnt + g, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_last[tid] = prev + n == 32 ? 1u : 0u;
            }
            __syncthreads();
            for (uint32_t i = tid / 64; i < ng; i += RG_T / 64) {
                if (!s_last[i]) continue;
                const uint32_t g = g0 + i;
                const float v = ld_dev(Y + g * 32 + (tid & 31));
                if (COH) xq_store_block32_dev(v, tid & 31, xq_view(p.xq_out, p.M / 32), g);
                else xq_store_block32(v, tid & 31, xq_view(p.xq_out, p.M / 32), g);
                if ((tid & 63) == 0) __hip_atomic_store(p.grp_cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    } else {
        for (uint32_t i = tid; i < nrow; i += RG_T) {
            const uint32_t row = r0 + i;
            float *y = sgs.y(row);
            float out = yl[i];
            if (COH) {
                if (p.acc) out += ld_dev(y);
                st_dev(y, out);
            } else {
                if (p.acc) out += *y;
                *y = out;
            }
        }
    }
    ZH_TRACE_POINT(4);
}

