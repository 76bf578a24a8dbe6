// zh_ffn_xcd.hip — the dense FFN of one decode layer (ffn_norm, gate/up +
// SwiGLU, down + residual) in one launch, split by XCD (8B shape: hidden
// 4096, FFN 12288, Q4_K gate/up, Q6_K down).
//
// Replaces three dispatches of the reference's decode step: ffn_norm, the
// fused gate/up/SwiGLU DMMV and the down DMMV with its residual add
// (forward.zig:8237-8290; dmmv_q4k.comp, dmmv_q6k.comp).
//
// XCD h owns FFN rows [1536 h, 1536 h + 1536): its 32 workgroups compute those
// gate/up rows and their SwiGLU outputs (48 rows each, the Q4_K ring's
// arithmetic, zh_ring_q4k.h), publish them in the XCD's L2 and meet at an
// XCD-local flag barrier (zh_xcd.h); then every workgroup multiplies the
// 1536 outputs by the down matrix's columns [1536 h, 1536 h + 1536) for its
// 128 rows (six Q6_K super-blocks of each row, 1260 bytes) and adds the 128
// partial sums into the residual with device-scope float atomics (one per
// XCD and row). The down projection thus needs no launch, no global
// exchange of the SwiGLU vector and no staging of the whole 12288-element
// activation: each XCD only ever sees its own slice of it.
//
// The residual is kept as A + D1 + D2 (zh_engine.hip): this launch reads
// x = A + D1 (A: the layer input, D1: the attention's O projection added by
// atomics), adds the down projection into D2 (zeroed by the attention launch
// of this layer) and zeroes D1 of the other parity (its last reader was this
// layer's attention launch; the next layer's attention adds into it).
//
// LDS: phase 1 is the Q4_K ring's layout (three 36 KB slots, XQ image, f32 x
// and norm weight; D1 is staged in the third slot, which the ring fills only
// after the activation work); phase 2 reuses it as three 40 KB slots of 32
// down rows (1280 bytes each: the 1260-byte column segment from its 16-byte
// aligned start), the SwiGLU slice and its XQ image.
#include "zh_ring_q4k.h"
#include "zh_xcd.h"

namespace {
constexpr uint32_t FX_H = 4096, FX_F = 12288;
constexpr uint32_t FX_RA = FX_F / (XCD_N * XCD_PER);   // gate/up rows per workgroup (48)
constexpr uint32_t FX_FS = FX_F / XCD_N;                // SwiGLU outputs per XCD (1536)
constexpr uint32_t FX_NSB = FX_FS / 256;                // down super-blocks per row and XCD (6)
constexpr uint32_t FX_HB = 2 * FX_NSB;                  // half super-blocks (12): lanes per down row
constexpr uint32_t FX_RB = FX_H / XCD_PER;  // down rows per workgroup (128)
constexpr uint32_t FX_DROWB = FX_F / 256 * 210;         // a down row (10080 B)
constexpr uint32_t FX_SEGB = FX_NSB * 210;              // its XCD column segment (1260 B)
constexpr uint32_t FX_SEGP = (FX_SEGB + 15 + 15) / 16;  // 16-byte pieces per row copy (80)
constexpr uint32_t FX_RS = FX_SEGP * 16;                // LDS bytes per down row (1280)
constexpr uint32_t FX_TR = 32;                          // down rows per tile (one pass: 32 teams of 16 lanes)
constexpr uint32_t FX_NT = FX_RB / FX_TR;               // tiles (4)
constexpr uint32_t FX_SLOT = FX_TR * FX_RS;             // 40 KB
constexpr uint32_t FX_TCH = FX_SLOT / 1024;             // 1 KB copies per tile (40: 10 per copying wave)
constexpr uint32_t FX_XQ2 = 3 * FX_SLOT;                // phase 2: XQ image of the slice
constexpr uint32_t FX_SRAW = FX_XQ2 + 8192;             // phase 2: the slice as f32 (6 KB)
static_assert(FX_SRAW + FX_FS * 4 <= RG_LDS, "phase 2 fits phase 1's LDS");
static_assert(FX_TCH % 4 == 0 && FX_HB <= 16, "tile copies over 4 waves; a row's lanes in a 16-lane team");
}  // namespace

// Flag words (zero when the engine is created): [0, 256) SwiGLU slices
// published (XCD h at h * 32), [256, 264) epochs.
constexpr uint32_t FX_FLAG_WORDS = XCD_N * XCD_PER + XCD_N;

struct FfnP {
    const float *xa, *xb;        // x = xa + xb (A + D1 of the residual)
    const float *norm_w;         // ffn_norm weight
    float eps;
    const uint8_t *wg, *wu;      // Q4_K gate, up [12288][4096]
    const uint8_t *wd;           // Q6_K down [4096][12288]
    float *s;                    // SwiGLU outputs [12288] (exchanged inside each XCD)
    float *xout;                 // xa + xb (16 rows per workgroup)
    float *acc;                  // D2: += the down projection (atomics)
    float *zero;                 // D1 of the other parity: zeroed (16 rows per workgroup)
    uint32_t *flags;             // FX_FLAG_WORDS
    uint32_t *ctl;               // device control words: [0] error word, [1] wait limit
    uint32_t plain;
    uint32_t pre, late;          // down tiles copied before the slices' wait (1..3); the rest after it (late 0) or after the slice landed (1)
};

__global__ __launch_bounds__(RG_T, 1) void k_ffn_xcd(FfnP P) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int NB = 16, MODE = LPB_GATE_UP;
    using TT = Q4Tiles<NB, MODE>;
    constexpr int TL = TT::TL, RPP = TT::RPP;
    constexpr uint32_t NBLK = NB * 8;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t h = min(xcc_id(), XCD_N - 1), j = blockIdx.x / XCD_N;
    uint32_t *fl = P.flags + h * XCD_PER, *ep = P.flags + XCD_N * XCD_PER + h;
    const uint32_t E = *(const __attribute__((address_space(4))) uint32_t *)ep + 1u;
    ZH_TRACE_POINT(0);

    // ---- phase 1: gate/up rows [1536 h + 48 j, + 48) (the ring's workgroup
    // h * 32 + j of 48 rows), ffn_norm(xa + xb) as XQ
    RingP p = {};
    p.norm_w = P.norm_w; p.eps = P.eps; p.M = FX_F; p.K = FX_H; p.nseg = 1; p.rpw = FX_RA;
    p.segW[0] = P.wg; p.segW[1] = P.wg; p.segW[2] = P.wg; p.W2 = P.wu;
    p.seg_end[0] = FX_F; p.seg_end[1] = FX_F; p.seg_end[2] = FX_F;
    const TT tiles(p, h * XCD_PER + j, tid, lds);
    const uint32_t wave = tiles.wave, r0 = tiles.r0, nt = tiles.nt, lds0 = tiles.lds0, tcw = tiles.tcw;
    uint8_t *ring = lds, *xqa = lds + RG_D * RG_TILE, *raw = lds + RG_D * RG_TILE + RG_XQ_BYTES;
    float *yl = (float *)(lds + RG_D * RG_TILE + RG_XQ_BYTES + RG_RAW_BYTES), *red = yl + 2 * RG_MAXROWS;
    // the activation: xa and the norm weight into the raw region, xb into
    // the third ring slot (2 + 1 KB copies per wave per vector)
#pragma unroll
    for (int i = 0; i < NB / 8; i++) {
        const uint32_t c = wave + 8 * i;
        dma16((const uint8_t *)P.xa + c * 1024 + lane * 16, lds0 + RG_D * RG_TILE + RG_XQ_BYTES + c * 1024);
        dma16((const uint8_t *)P.norm_w + c * 1024 + lane * 16, lds0 + RG_D * RG_TILE + RG_XQ_BYTES + NB * 1024 + c * 1024);
        dma16((const uint8_t *)P.xb + c * 1024 + lane * 16, lds0 + (RG_D - 1) * RG_TILE + c * 1024);
    }
    const uint32_t npro = tiles.prologue();
    for (uint32_t t = 0; t < npro; t++) tiles.issue(t, t);
    wait_vm_dyn(npro * tcw);
    lds_bar();
    ZH_TRACE_POINT(1);
    float *ixs = (float *)(xqa + NB * 2 * RG_SEG), *ixz = ixs + NBLK;
    {
        const float *xr = (const float *)raw, *wr = (const float *)(raw + NB * 1024);
        const float *xr2 = (const float *)(ring + (RG_D - 1) * RG_TILE);
        f32x4 v[NB / 8], w[NB / 8];
        float sq = 0.f;
#pragma unroll
        for (int it = 0; it < NB / 8; it++) {
            const uint32_t e0 = (it * RG_T + tid) * 4;
            const f32x4 a = *(const f32x4 *)(xr + e0), b = *(const f32x4 *)(xr2 + e0);
            v[it] = f32x4{a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w};
            if ((it * RG_T + tid) / 4 == blockIdx.x) *(f32x4 *)(P.xout + e0) = v[it];  // this workgroup's 16 rows
            w[it] = *(const f32x4 *)(wr + e0);
            sq = fmaf(v[it].x, v[it].x, sq); sq = fmaf(v[it].y, v[it].y, sq);
            sq = fmaf(v[it].z, v[it].z, sq); sq = fmaf(v[it].w, v[it].w, sq);
        }
        sq = wave_sum(sq);
        if (lane == 0) red[wave] = sq;
        lds_bar();
        float tot = 0.f;
#pragma unroll
        for (int w8 = 0; w8 < 8; w8++) tot += red[w8];
        const float rms_inv = 1.0f / sqrtf(tot / (float)FX_H + P.eps);
#pragma unroll
        for (int it = 0; it < NB / 8; it++) {
            const uint32_t e0 = (it * RG_T + tid) * 4;
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
    }
    {
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
        ZH_TRACE_POINT(2);
        const uint32_t mrow = team / RPP, trow = team % RPP;
        for (uint32_t t = 0; t < nt; t++) {
            wait_vm_dyn(min(nt - 1 - t, (uint32_t)RG_D - 2) * tcw);
            lds_bar();  // (t = 0: also every wave done with xb in the third slot)
        if (t == 0) ZH_TRACE_POINT(11);
            if (t + RG_D - 1 < nt) tiles.issue(t + RG_D - 1, (t + RG_D - 1) % RG_D);
            const uint8_t *blk = ring + (t % RG_D) * RG_TILE + team * TT::ROWB + b * 144;
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
            float res = fmaf(hdr.d, accd, -hdr.dmin * accm);
            res = team_sum_dpp<TL>(res);
            const uint32_t i = t * RPP + trow;
            if (tl == 0 && i < RG_MAXROWS) yl[mrow * RG_MAXROWS + i] = res;
        }
    }
    lds_bar();
    ZH_TRACE_POINT(3);
    // ---- publish the 48 SwiGLU outputs in the XCD's L2 (wave 0), then the flag
    if (wave == 0) {
        if (lane < FX_RA) P.s[r0 + lane] = silu_mul(yl[lane], yl[RG_MAXROWS + lane]);
        wait_vm<0>();
        if (lane == 0) *(volatile uint32_t *)(fl + j) = E;
    }
    __syncthreads();  // phase 1's LDS is free

    // ---- phase 2: down rows [128 j, 128 j + 128) x columns [1536 h, + 1536).
    // Waves 0-3 copy the tiles (row segments from their 16-byte aligned
    // start, oh bytes before the segment); waves 4-7 wait for the XCD's
    // SwiGLU slices and copy the slice.
    const uint32_t oh = (h * FX_SEGB) & 15u;
    const uint8_t *dseg = P.wd + (size_t)(j * FX_RB) * FX_DROWB + h * FX_SEGB - oh;
    // the last piece inside the row (XCD 7's segment ends at the row's end)
    const uint32_t klast = (FX_DROWB - (h * FX_SEGB - oh)) / 16 - 1;
    const bool wa = wave < 4;
    const uint32_t wl4 = wave & 3;
    auto issue_d = [&](uint32_t t, uint32_t s) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t i = 0; i < FX_TCH / 4; i++) {
            const uint32_t c = wl4 + 4 * i, pc = c * 64 + lane;  // 16-byte piece of the tile
            const uint32_t row = pc / FX_SEGP, k = min(pc - row * FX_SEGP, klast);
            dma16(dseg + (size_t)(t * FX_TR + row) * FX_DROWB + k * 16, lds0 + s * FX_SLOT + c * 1024);
        }
    };
    const uint32_t pre = P.pre;
    if (wa)  // the first tiles (up to three; the fourth follows into slot 0)
        for (uint32_t t = 0; t < pre; t++) issue_d(t, t);
    if (tid < 16) P.zero[blockIdx.x * 16 + tid] = 0.f;  // D1 of the other parity
    const bool ok = xcd_wait(fl, XCD_PER, E, P.ctl, tid, 4);
    ZH_TRACE_POINT(4);
    if (j == 0 && tid == 256) *(volatile uint32_t *)ep = E;  // every workgroup of the XCD has read the epoch (wave 4: no copies in flight)
    if (wa && !P.late)
        for (uint32_t t = pre; t < 3; t++) issue_d(t, t);
    if (!wa) {  // the slice (6 KB): waves 4-7, 1 KB copies
        for (uint32_t c = wl4; c < FX_FS * 4 / 1024; c += 4) {
            const uint8_t *src = (const uint8_t *)(P.s + h * FX_FS) + c * 1024 + lane * 16;
            if (P.plain) dma16(src, lds0 + FX_SRAW + c * 1024);
            else dma16_dev(src, lds0 + FX_SRAW + c * 1024);
        }
        wait_vm<0>();
    }
    lds_bar();
    ZH_TRACE_POINT(12);
    if (wa && P.late)
        for (uint32_t t = pre; t < 3; t++) issue_d(t, t);
    // the slice as XQ (48 blocks of 32): threads 0..383, 4 elements each
    const XQView xv = xq_view(lds + FX_XQ2, FX_FS / 32);
    if (tid < FX_FS / 4) {
        const uint32_t e0 = tid * 4;
        const f32x4 u = *(const f32x4 *)((const float *)(lds + FX_SRAW) + e0);
        const float a = row8_max(fmaxf(fmaxf(fabsf(u.x), fabsf(u.y)), fmaxf(fabsf(u.z), fabsf(u.w))));
        float inv, sc;
        xq_scales(a, inv, sc);
        int X[4] = {xq_quant(u.x, inv), xq_quant(u.y, inv), xq_quant(u.z, inv), xq_quant(u.w, inv)};
        int l0[4], l1[4], l2[4];
#pragma unroll
        for (int q = 0; q < 4; q++) xq_limbs(X[q], l0[q], l1[q], l2[q]);
        const uint32_t blk = e0 / 32, lo = e0 % 32;
        uint8_t *dst = (uint8_t *)xv.limb + blk * 96 + lo;
        *(uint32_t *)(dst) = pack4(l0[0], l0[1], l0[2], l0[3]);
        *(uint32_t *)(dst + 32) = pack4(l1[0], l1[1], l1[2], l1[3]);
        *(uint32_t *)(dst + 64) = pack4(l2[0], l2[1], l2[2], l2[3]);
        int sm = X[0] + X[1] + X[2] + X[3];
        sm += __builtin_amdgcn_update_dpp(0, sm, 0xB1, 0xF, 0xF, false);
        sm += __builtin_amdgcn_update_dpp(0, sm, 0x4E, 0xF, 0xF, false);
        const uint32_t sub = tid & 7;
        if (sub == 0) xv.xs[blk] = sc;
        if ((sub & 3) == 0) xv.xsum[blk * 2 + (sub >> 2)] = (float)sm * sc;
    }
    lds_bar();
    ZH_TRACE_POINT(13);
    // lane: row (team) tid / 16 of a tile, half super-block tl = tid % 16
    // (< 12) of the segment: super-block tl / 2, half tl % 2
    const uint32_t team = tid / 16, tl = tid % 16;
    const bool act = tl < FX_HB;
    const uint32_t q = act ? tl : 0u, b = q >> 1, hh = q & 1, j0 = 4 * q;
    uint32_t L[4][24];
    float xs[4], z0[4], z1[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        lds_load_limbs(L[k], (const uint8_t *)xv.limb + (j0 + k) * 96);
        xs[k] = xv.xs[j0 + k];
        z0[k] = -32.f * xv.xsum[2 * (j0 + k)];
        z1[k] = -32.f * xv.xsum[2 * (j0 + k) + 1];
    }
    ZH_TRACE_POINT(5);
    for (uint32_t t = 0; t < FX_NT; t++) {
        // copies after tile t's: tiles 1, 2 (t = 0); 2 (t = 1); 3 (t = 2)
        static_assert(FX_NT == 4, "the ring schedule below");
        if (wa) wait_vm_dyn((t == 0 ? 2u : t < 3 ? 1u : 0u) * (FX_TCH / 4));
        lds_bar();
        if (wa && t == 1) issue_d(3, 0);
        ZH_TRACE_POINT(7 + t);
        const uint8_t *slot = lds + (t % 3) * FX_SLOT;
        const uint32_t boff = team * FX_RS + oh + b * 210;  // 2-byte aligned block start
        const uint32_t sh = boff & 3;
        uint32_t rq[17], rh[9], rs[3];
        {
            const uint32_t *a = (const uint32_t *)(slot + ((boff + 64 * hh) & ~3u));
#pragma unroll
            for (int i = 0; i < 17; i++) rq[i] = a[i];
            const uint32_t *c = (const uint32_t *)(slot + ((boff + 128 + 32 * hh) & ~3u));
#pragma unroll
            for (int i = 0; i < 9; i++) rh[i] = c[i];
            const uint32_t *sp = (const uint32_t *)(slot + ((boff + 192 + 8 * hh) & ~3u));
#pragma unroll
            for (int i = 0; i < 3; i++) rs[i] = sp[i];
        }
        const uint32_t scw0 = __builtin_amdgcn_alignbyte(rs[1], rs[0], sh), scw1 = __builtin_amdgcn_alignbyte(rs[2], rs[1], sh);
        const uint32_t dw = *(const uint16_t *)(slot + boff + 208);  // d (2-byte aligned)
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            int D[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int qi = (g & 1) * 8 + i;
                const uint32_t av = __builtin_amdgcn_alignbyte(rq[qi + 1], rq[qi], sh);
                const uint32_t cv = __builtin_amdgcn_alignbyte(rh[i + 1], rh[i], sh);
                const uint32_t lo4 = (g >> 1) ? ((av >> 4) & 0x0F0F0F0Fu) : (av & 0x0F0F0F0Fu);
                const uint32_t hi2 = ((cv >> (2 * g)) << 4) & 0x30303030u;
                const uint32_t qv = lo4 | hi2;  // unsigned code; the -32 offset enters through z0 / z1
                const int grp = i >> 2;
#pragma unroll
                for (int k = 0; k < 3; k++) D[grp][k] = sdot4(qv, L[g][k * 8 + i], D[grp][k]);
            }
            const uint32_t sw = g >> 1 ? scw1 : scw0;
            const int sc0 = (int)(int8_t)((sw >> (16 * (g & 1))) & 0xFF);  // scales[8 hh + 2 g]
            const int sc1 = (int)(int8_t)((sw >> (16 * (g & 1) + 8)) & 0xFF);
            const float S0 = comb_f(D[0][0], D[0][1], D[0][2]);
            const float S1 = comb_f(D[1][0], D[1][1], D[1][2]);
            acc = fmaf((float)sc0, fmaf(xs[g], S0, z0[g]), acc);
            acc = fmaf((float)sc1, fmaf(xs[g], S1, z1[g]), acc);
        }
        float res = act ? h2f(dw) * acc : 0.f;
        res = team_sum_dpp<16>(res);
        if (!ok) res = __builtin_nanf("");  // the slices' wait gave up
        if (tl == 0)
            __hip_atomic_fetch_add(P.acc + j * FX_RB + t * FX_TR + team, res, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    ZH_TRACE_POINT(6);
}

ZH_TRACE_DUMP_FN(zh_debug_trace_ffn)

uint32_t zhk_ffn_xcd_flag_words() { return FX_FLAG_WORDS; }

bool zhk_ffn_xcd_supported(zh_ctx *c, uint32_t hidden, uint32_t ffn) {
    return hidden == FX_H && ffn == FX_F && !c->concurrent && zhk_xcd_round_robin(c);
}

int zhk_ffn_xcd(zh_ctx *c, const float *xa, const float *xb, const float *norm_w, float eps, const uint8_t *wg,
                const uint8_t *wu, const uint8_t *wd, float *s, float *xout, float *acc, float *zero,
                uint32_t *flags) {
    if (((uintptr_t)xa & 15) || ((uintptr_t)xb & 15) || ((uintptr_t)norm_w & 15) || ((uintptr_t)wg & 15) ||
        ((uintptr_t)wu & 15) || ((uintptr_t)wd & 15) || ((uintptr_t)s & 15) || ((uintptr_t)xout & 15) || !acc || !zero)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "ffn_xcd: 16-byte aligned operands");
    FfnP P = {};
    P.xa = xa; P.xb = xb; P.norm_w = norm_w; P.eps = eps; P.wg = wg; P.wu = wu; P.wd = wd;
    P.pre = (uint32_t)min(max(zh_knob_int("ZH_FFN_PRE", 3), 1), 3);
    P.late = (uint32_t)zh_knob_int("ZH_FFN_LATE", 0);
    P.plain = (uint32_t)zh_knob_int("ZH_FFN_PLAIN", 0);
    P.s = s; P.xout = xout; P.acc = acc; P.zero = zero; P.flags = flags; P.ctl = c->err_dev;
    static bool attr = false;
    if (!attr) {
        ZH_HIP(c, hipFuncSetAttribute((const void *)k_ffn_xcd, hipFuncAttributeMaxDynamicSharedMemorySize, (int)RG_LDS));
        attr = true;
    }
    hipLaunchKernelGGL(k_ffn_xcd, dim3(XCD_N * XCD_PER), dim3(RG_T), RG_LDS, c->stream, P);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
