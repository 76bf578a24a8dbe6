// zh_ring_q6k.h — streaming Q6_K DMMV for the FFN down projection (K = the
// FFN width, 256 * NB) in the persistent decode-layers kernel (zh_step.hip).
//
// One 512-thread workgroup owns a contiguous range of output rows, which
// are contiguous in memory (row-major, NB * 210 bytes each). A pass covers
// RPP = 512 / (2 NB) rows: 2 NB lanes per row, one half super-block (128
// elements: ql[64h..], qh[32h..], scales[8h..], d) per lane (capped at 4
// rows). The passes' bytes stream HBM -> LDS through a ring of three slots with the
// asynchronous global_load_lds DMA, two slots in flight while the third is
// computed (the Q4_K ring's scheme, zh_ring_q4k.h). The XQ activation is
// copied once into the last slot (the ring fills it only after the first
// wait) and each lane keeps the limbs of its half super-block in registers.
// Per-row sums: 16-lane DPP sums (a row's lanes start at a multiple of 16),
// then the 2 NB / 16 partials of a row added in LDS after the loop.
//
// Replaces DmmvDispatch.recordDispatch for Q6_K (src/compute/dmmv.zig:806-874,
// dmmv_q6k.comp) where it feeds the residual add (forward.zig:8274-8290).
#pragma once
#include "zh_device.h"
#include "zh_internal.h"
#include "zh_lpb_common.h"

#pragma clang diagnostic ignored "-Winline-asm"

namespace {
constexpr int R6_T = 512;
constexpr int R6_D = 3;
constexpr uint32_t R6_MAXROWS = 64;  // output rows per workgroup
}  // namespace

struct Ring6P {
    const uint8_t *W;   // [M][NB blocks of 210 B]
    const uint8_t *xq;  // XQ activation of K = 256 NB elements
    float *y;           // y = W x, or y += W x with acc
    uint32_t M, acc, rpw;
};

template <int NB>
struct R6 {
    static constexpr uint32_t TL = 2 * NB;                  // lanes per row
    // rows per pass: as many as the lanes allow, at most 4 (three slots of
    // four rows fit the LDS the persistent kernel leaves; 16-row workgroup
    // ranges then take four full passes)
    static constexpr uint32_t RPP = R6_T / TL < 4 ? R6_T / TL : 4;
    static constexpr uint32_t ROWB = NB * 210;              // bytes per row
    static constexpr uint32_t SLOT = (RPP * ROWB + 1023) / 1024 * 1024;
    static constexpr uint32_t CH = SLOT / 1024;             // 1 KB copies per pass
    static constexpr uint32_t NBLK = NB * 8;                // 32-element blocks of x
    static constexpr uint32_t LIMB = NBLK * 96;             // limb bytes of x (a multiple of 1 KB)
    static constexpr uint32_t XQB = NBLK * 108;             // all XQ bytes of x
    static constexpr uint32_t XCH = (XQB + 1023) / 1024;    // 1 KB copies of x
    static constexpr uint32_t SMALL = (NBLK * 12 + 1023) / 1024 * 1024 + 1024;  // xs, xsum (+ copy slack)
    static constexpr uint32_t NPART = TL / 16;              // 16-lane partials per row
    static constexpr uint32_t LDS = R6_D * SLOT + SMALL + R6_MAXROWS * NPART * 4;
    static_assert(NB % 8 == 0 && TL <= (uint32_t)R6_T, "rows start 16-byte aligned, a row fits a workgroup");
    static_assert(LIMB % 1024 == 0 && LIMB <= SLOT, "the limbs fit the last ring slot");
};

// Pass t (rows r0 + t RPP ..) of workgroup wg into slot s. Bytes past the
// range re-read its last 16 bytes (discarded rows).
template <int NB>
struct Q6Tiles {
    using G = R6<NB>;
    uint32_t r0, r1, nt, wave, lane, tcw, lds0, wlim;
    const uint8_t *wbase;
    ZH_DEVM Q6Tiles(const Ring6P &p, uint32_t wg, uint32_t tid, const uint8_t *lds) {
        lane = tid & 63;
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        r0 = wg * p.rpw;
        r1 = min(p.M, r0 + p.rpw);
        nt = r0 < p.M ? (r1 - r0 + G::RPP - 1) / G::RPP : 0u;
        tcw = wave < G::CH % 8 ? G::CH / 8 + 1 : G::CH / 8;
        lds0 = lds_addr(lds);
        wbase = p.W + (size_t)r0 * G::ROWB;
        wlim = nt ? (r1 - r0) * G::ROWB - 16 : 0u;
    }
    ZH_DEVM uint32_t prologue() const { return min(nt, (uint32_t)R6_D - 1); }
    ZH_DEVM void issue(uint32_t t, uint32_t s) const {
#pragma unroll
        for (uint32_t i = 0; i < (G::CH + 7) / 8; i++) {
            const uint32_t c = wave + 8 * i;
            if (c < G::CH) dma16(wbase + min(t * G::RPP * G::ROWB + c * 1024 + lane * 16, wlim), lds0 + s * G::SLOT + c * 1024);
        }
    }
};

// The first passes' copies, issued while the persistent kernel waits at the
// grid barrier before the phase; returns the count (the body's `pre`).
template <int NB>
ZH_DEV uint32_t q6k_ring_prefetch(const Ring6P &p, uint32_t wg, uint8_t *lds) {
    const Q6Tiles<NB> tl(p, wg, phase_tid(), lds);
    const uint32_t n = tl.prologue();
    for (uint32_t t = 0; t < n; t++) tl.issue(t, t);
    return n;
}

// pre: passes 0 .. pre-1 already copied (q6k_ring_prefetch), before the
// activation's copy.
template <int NB, bool COH>
ZH_DEV void q6k_ring_body(const Ring6P &p, uint32_t wg, uint8_t *lds, uint32_t pre = 0) {
    using G = R6<NB>;
    const uint32_t tid = COH ? phase_tid() : threadIdx.x, lane = tid & 63;
    const Q6Tiles<NB> tiles(p, wg, tid, lds);
    const uint32_t wave = tiles.wave, r0 = tiles.r0, r1 = tiles.r1, nt = tiles.nt;
    if (nt == 0) return;  // (persistent kernel: more workgroups than row ranges)
    uint8_t *ring = lds;
    float *sx = (float *)(lds + R6_D * G::SLOT);  // xs [NBLK], xsum [NBLK][2]
    float *sz = sx + G::NBLK;
    float *part = (float *)(lds + R6_D * G::SLOT + G::SMALL);  // [R6_MAXROWS][NPART]
    const uint32_t lds0 = lds_addr(lds);

    // ---- the activation: limbs into the last slot, xs / xsum after the ring
#pragma unroll
    for (uint32_t i = 0; i < (G::XCH + 7) / 8; i++) {
        const uint32_t c = wave + 8 * i;
        if (c < G::XCH) {  // uniform per wave
            const uint32_t dst = c < G::LIMB / 1024 ? (R6_D - 1) * G::SLOT + c * 1024
                                                    : R6_D * G::SLOT + (c - G::LIMB / 1024) * 1024;
            dma16_act<COH>(p.xq + min(c * 1024 + lane * 16, G::XQB - 16), lds0 + dst);
        }
    }
    const uint32_t tcw = tiles.tcw;
    auto issue_tile = [&](uint32_t t, uint32_t s) __attribute__((always_inline)) { tiles.issue(t, s); };
    const uint32_t npro = tiles.prologue();
    for (uint32_t t = pre; t < npro; t++) issue_tile(t, t);
    wait_vm_dyn((npro - pre) * tcw);  // the activation (older than the tiles it precedes) has landed
    lds_bar();

    // ---- this lane's half super-block: limbs, scales, sums in registers
    const uint32_t rt = tid / G::TL, tl = tid % G::TL;
    const bool active = rt < G::RPP;
    const uint32_t rtc = active ? rt : 0u, b = tl >> 1, h = tl & 1, j0 = b * 8 + 4 * h;
    uint32_t L[4][24];
    float xs[4], z0[4], z1[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        lds_load_limbs(L[q], ring + (R6_D - 1) * G::SLOT + (j0 + q) * 96);
        xs[q] = sx[j0 + q];
        z0[q] = -32.f * sz[2 * (j0 + q)];
        z1[q] = -32.f * sz[2 * (j0 + q) + 1];
    }

    // ---- the ring
    for (uint32_t t = 0; t < nt; t++) {
        wait_vm_dyn(min(nt - 1 - t, (uint32_t)R6_D - 2) * tcw);
        lds_bar();
        if (t + R6_D - 1 < nt) issue_tile(t + R6_D - 1, (t + R6_D - 1) % R6_D);
        const uint8_t *slot = ring + (t % R6_D) * G::SLOT;
        const uint32_t boff = rtc * G::ROWB + b * 210;  // 2-byte aligned block start
        const uint32_t sh = boff & 3;
        // ql / qh / this half's 8 scales / d: dword reads realigned by the
        // block start's byte offset (every index below is static, so the
        // words stay in registers)
        uint32_t rq[17], rh[9], rs[3];
        {
            const uint32_t *a = (const uint32_t *)(slot + ((boff + 64 * h) & ~3u));
#pragma unroll
            for (int i = 0; i < 17; i++) rq[i] = a[i];
            const uint32_t *c = (const uint32_t *)(slot + ((boff + 128 + 32 * h) & ~3u));
#pragma unroll
            for (int i = 0; i < 9; i++) rh[i] = c[i];
            const uint32_t *sp = (const uint32_t *)(slot + ((boff + 192 + 8 * h) & ~3u));
#pragma unroll
            for (int i = 0; i < 3; i++) rs[i] = sp[i];
        }
        const uint32_t scw[2] = {__builtin_amdgcn_alignbyte(rs[1], rs[0], sh), __builtin_amdgcn_alignbyte(rs[2], rs[1], sh)};
        const uint32_t dw = *(const uint16_t *)(slot + boff + 208);  // d (2-byte aligned)
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            // element 32 g + 16 grp + 4 i + e of the half: 6-bit code from the
            // low / high nibble of ql (g & 1 selects the 32-byte half of ql,
            // g >> 1 the nibble) and 2 bits of qh
            int D[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int qi = (g & 1) * 8 + i;
                const uint32_t av = __builtin_amdgcn_alignbyte(rq[qi + 1], rq[qi], sh);
                const uint32_t cv = __builtin_amdgcn_alignbyte(rh[i + 1], rh[i], sh);
                const uint32_t lo4 = (g >> 1) ? ((av >> 4) & 0x0F0F0F0Fu) : (av & 0x0F0F0F0Fu);
                const uint32_t hi2 = ((cv >> (2 * g)) << 4) & 0x30303030u;
                const uint32_t q = lo4 | hi2;  // unsigned code; the -32 offset enters through z0 / z1
                const int grp = i >> 2;
#pragma unroll
                for (int k = 0; k < 3; k++) D[grp][k] = sdot4(q, L[g][k * 8 + i], D[grp][k]);
            }
            const int sc0 = (int)(int8_t)((scw[g >> 1] >> (16 * (g & 1))) & 0xFF);  // scales[8h + 2g]
            const int sc1 = (int)(int8_t)((scw[g >> 1] >> (16 * (g & 1) + 8)) & 0xFF);
            const float S0 = comb_f(D[0][0], D[0][1], D[0][2]);
            const float S1 = comb_f(D[1][0], D[1][1], D[1][2]);
            acc = fmaf((float)sc0, fmaf(xs[g], S0, z0[g]), acc);
            acc = fmaf((float)sc1, fmaf(xs[g], S1, z1[g]), acc);
        }
        float res = h2f(dw) * acc;
        res = row16_sum(res);
        const uint32_t row = t * G::RPP + rt;
        if (active && (tid & 15) == 0 && row < R6_MAXROWS) part[row * G::NPART + tl / 16] = res;
    }
    lds_bar();

    // ---- outputs: a row's partials in lane order
    for (uint32_t i = tid; i < r1 - r0; i += R6_T) {
        float out = 0.f;
#pragma unroll
        for (uint32_t k = 0; k < G::NPART; k++) out += part[i * G::NPART + k];
        float *y = p.y + r0 + i;
        if (COH) {
            if (p.acc) out += ld_dev(y);
            st_dev(y, out);
        } else {
            if (p.acc) out += *y;
            *y = out;
        }
    }
}
