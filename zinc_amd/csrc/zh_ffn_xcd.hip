// zh_ffn_xcd.hip — the dense FFN of one decode layer (ffn_norm, gate/up +
// SwiGLU, down + residual) in one launch (8B shape: hidden 4096, FFN 12288,
// Q4_K gate/up, Q6_K down).
//
// Replaces three dispatches of the reference's decode step: ffn_norm, the
// fused gate/up/SwiGLU DMMV and the down DMMV with its residual add
// (forward.zig:8237-8290; dmmv_q4k.comp, dmmv_q6k.comp).
//
// Workgroup w = 32 h + j (XCD h, slot j: zh_xcd.h) owns FFN rows
// [48 w, 48 w + 48), so XCD h owns FFN rows [1536 h, 1536 h + 1536):
//   1. gate/up: its 48 gate and 48 up rows against ffn_norm(x) as XQ limbs
//      (the Q4_K ring's arithmetic, zh_ring_q4k.h), SwiGLU of the 48 pairs;
//   2. the SwiGLU values (as XQ limbs) go to the XCD's other 31 workgroups
//      through its L2 (epoch-tagged words, zh_xcd.h);
//   3. down: rows [128 j, 128 j + 128) of ffn_down over the XCD's 1536
//      columns, i.e. the XCD's share of those rows' dot products, added into
//      the residual with one device atomic per XCD and row.
// Steps 1 and 3 are one stream: the 6 gate/up tiles (36 KB) and then the 8
// down tiles (22 KB) flow through one three-slot LDS ring of asynchronous
// global_load_lds copies; three down tiles are in flight while the exchange
// of step 2 completes, so HBM does not wait for it.
//
// The down matrix comes from a copy of ffn_down that the engine repacks
// (k_ffn_pack_down): per workgroup, its 128 rows x the XCD's 32 column groups
// of 48 as records of 44 bytes, [row][group], contiguous — the 48 6-bit
// codes (three 16-element groups: low nibbles in two dwords, high bit pairs
// in a third), the three groups' int8 scales and the f16 super-block scales
// of groups 0 and 2 (group 1 shares one of them). 44-byte records make the
// lanes' LDS reads conflict-free (11 dwords apart). The values are Q6_K's,
// unchanged: d * scale * (code - 32).
//
// The residual is kept as A + D (zh_engine.hip): this launch reads x = xa +
// xb, stores its 16 rows of x into xout, adds the down projection into acc
// (zeroed by the previous launch) and zeroes its 16 rows of `zero`.
#include "zh_ring_q4k.h"
#include "zh_xcd.h"

namespace {
constexpr uint32_t FX_H = 4096, FX_F = 12288;
constexpr uint32_t FX_RA = FX_F / (XCD_N * XCD_PER);   // gate/up rows per workgroup (48)
constexpr uint32_t FX_REC = 44;                         // packed down record per row and workgroup
constexpr uint32_t FX_SLICE = FX_H * FX_REC;            // a workgroup's packed columns (176 KB)
constexpr uint32_t FX_DR = 512;                         // down rows per tile (one per thread)
constexpr uint32_t FX_DT = FX_H / FX_DR;                // down tiles (8)
constexpr uint32_t FX_DTB = FX_DR * FX_REC;             // down tile bytes (22 KB)
constexpr uint32_t FX_DCH = FX_DTB / 1024;              // its 1 KB copies (22)
constexpr uint32_t FX_GT = 6;                           // gate/up tiles (48 rows / 8 per pass)
constexpr uint32_t FX_NU = FX_GT + FX_DT;               // ring units
constexpr uint32_t FX_RROWS = FX_H / XCD_PER;           // down rows of each workgroup (128)
constexpr uint32_t FX_DWV = 6;                          // waves that copy the down tiles
#ifndef ZH_FFN_DS
#define ZH_FFN_DS 4
#endif
#ifndef ZH_FFN_EARLY
#define ZH_FFN_EARLY 1
#endif
constexpr uint32_t FX_DS = ZH_FFN_DS;                   // down tile slots (22 KB apart)
constexpr uint32_t FX_XW = 48;                          // tagged words of a workgroup's SwiGLU block (42 used)
constexpr uint32_t FX_XPW = XCD_PER / 2 * FX_XW / 64;   // words per lane of each of the two polling waves (12)
constexpr uint32_t FX_XBLK = XCD_PER * FX_XW * 4;       // LDS: the XCD's blocks, then this workgroup's own
// LDS beyond the ring (the layout of zh_ring_q4k.h): the XQ image's region
// takes the 4096 partial sums, the f32 staging region the SwiGLU values'
// limbs
constexpr uint32_t FX_ACT = RG_D * RG_TILE + RG_XQ_BYTES;
static_assert(FX_DTB % 1024 == 0 && FX_DS * FX_DTB <= RG_D * RG_TILE + RG_XQ_BYTES, "down slots over the ring and the XQ image");
// the down slots the gate/up loop fills lie in ring slots it no longer reads:
// tile 0 (issued with unit 4) in unit 3's slot, tiles 1 and 2 (with unit 5)
// in units 3 and 4's
static_assert(FX_DTB <= RG_TILE && 3 * FX_DTB <= 2 * RG_TILE, "down slots 0-2 below unit 5's ring slot");
static_assert(FX_XBLK + 256 + FX_RROWS * 4 <= RG_RAW_BYTES && XCD_PER / 2 * FX_XW % 64 == 0, "exchange in the staging region");
static_assert(FX_GT * 8 == FX_RA, "gate/up: 8 rows per pass (16 super-blocks, 32 lanes per row)");
}  // namespace

// Flag words (zero when the engine is created): [0, 256) unused (the SwiGLU
// blocks carry epoch tags), [256, 264) epochs.
constexpr uint32_t FX_FLAG_WORDS = XCD_N * XCD_PER + XCD_N;

struct FfnP {
    const float *xa;             // x = xa + xb
    const zh_fix *xb;            //   (xb: fixed point, zh_xcd.h)
    const float *norm_w;         // ffn_norm weight
    float eps;
    const uint8_t *wg, *wu;      // Q4_K gate, up [12288][4096]
    const uint8_t *pk;           // packed down columns [256][4096][44 B]
    uint64_t *xact;              // [256][FX_XW] epoch-tagged SwiGLU blocks (exchanged inside each XCD)
    float *xout;                 // xa + xb (16 rows per workgroup)
    zh_fix *acc;                 // += the down projection (fixed-point atomics)
    zh_fix *zero;                // zeroed (16 rows per workgroup)
    uint32_t *flags;             // FX_FLAG_WORDS
    uint32_t *ctl;               // device control words: [0] error word, [1] wait limit
};

ZH_DEV int row16_sum_i(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
    return v + __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
}

__global__ __launch_bounds__(RG_T, 1) void k_ffn_xcd(FfnP P) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int NB = 16, MODE = LPB_GATE_UP;
    using TT = Q4Tiles<NB, MODE>;
    constexpr int TL = TT::TL, RPP = TT::RPP;
    constexpr uint32_t NBLK = NB * 8;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t h = min(xcc_id(), XCD_N - 1), j = blockIdx.x / XCD_N, w = h * XCD_PER + j;
    uint32_t *ep = P.flags + XCD_N * XCD_PER + h;
    const uint32_t E = *(const __attribute__((address_space(4))) uint32_t *)ep + 1u;
    ZH_TRACE_POINT(0);
    ZH_TRACE_VALUE(h + 1);  // (the XCD, + 1: a slot of 0 reads as unset)

    RingP p = {};
    p.norm_w = P.norm_w; p.eps = P.eps; p.M = FX_F; p.K = FX_H; p.nseg = 1; p.rpw = FX_RA;
    p.segW[0] = P.wg; p.segW[1] = P.wg; p.segW[2] = P.wg; p.W2 = P.wu;
    p.seg_end[0] = FX_F; p.seg_end[1] = FX_F; p.seg_end[2] = FX_F;
    const TT tiles(p, w, tid, lds);
    const uint32_t wave = tiles.wave, lds0 = tiles.lds0, tcw = tiles.tcw;
    // a wave's 1 KB copies per down tile (chunk c = wave + 6 i < 22: waves
    // 0-5; waves 6 and 7 poll the SwiGLU exchange)
    const uint32_t dcw = wave >= FX_DWV ? 0u : wave < FX_DCH % FX_DWV ? FX_DCH / FX_DWV + 1 : FX_DCH / FX_DWV;
    const uint8_t *pk = P.pk + (size_t)w * FX_SLICE;
    // unit u of the stream: gate/up tile u into ring slot u % 3, then down
    // tile u - 6 into down slot (u - 6) % 5 (22 KB apart, over the ring and
    // the XQ image's region: FX_DS)
    auto issue = [&](uint32_t u) __attribute__((always_inline)) {
        if (u < FX_GT) {
            tiles.issue(u, u % RG_D);
        } else {
            const uint32_t s = (u - FX_GT) % FX_DS;
#pragma unroll
            for (uint32_t i = 0; i < (FX_DCH + FX_DWV - 1) / FX_DWV; i++) {
                const uint32_t c = wave + FX_DWV * i;
                if (wave < FX_DWV && c < FX_DCH)  // uniform per wave
                    dma16(pk + (u - FX_GT) * FX_DTB + c * 1024 + lane * 16, lds0 + s * FX_DTB + c * 1024);
            }
        }
    };
    // a wave's copies of unit u (the ring waits count them)
    auto cnt = [&](uint32_t u) { return u < FX_GT ? tcw : dcw; };
    uint8_t *ring = lds, *xqa = lds + RG_D * RG_TILE, *raw = lds + FX_ACT;
    float *yl = (float *)(lds + RG_D * RG_TILE + RG_XQ_BYTES + RG_RAW_BYTES), *red = yl + 2 * RG_MAXROWS;

    // ---- the activation: xa and the norm weight into the staging region,
    // xb into the third ring slot (first filled by unit 2, issued after the
    // XQ image is built); 2 + 2 + 4 copies of 1 KB per wave
#pragma unroll
    for (int i = 0; i < NB / 8; i++) {
        const uint32_t c = wave + 8 * i;
        dma16((const uint8_t *)P.xa + c * 1024 + lane * 16, lds0 + FX_ACT + c * 1024);
        dma16((const uint8_t *)P.norm_w + c * 1024 + lane * 16, lds0 + FX_ACT + NB * 1024 + c * 1024);
    }
#pragma unroll
    for (int i = 0; i < NB / 4; i++) {  // xb: 8 bytes per element
        const uint32_t c = wave + 8 * i;
        dma16((const uint8_t *)P.xb + c * 1024 + lane * 16, lds0 + (RG_D - 1) * RG_TILE + c * 1024);
    }
    issue(0);
    issue(1);
    wait_vm_dyn(2 * tcw);
    lds_bar();
    ZH_TRACE_POINT(1);
    float *ixs = (float *)(xqa + NB * 2 * RG_SEG), *ixz = ixs + NBLK;
    {
        const float *xr = (const float *)raw, *wr = (const float *)(raw + NB * 1024);
        const zh_fix *xr2 = (const zh_fix *)(ring + (RG_D - 1) * RG_TILE);
        f32x4 v[NB / 8], wn[NB / 8];
        float sq = 0.f;
#pragma unroll
        for (int it = 0; it < NB / 8; it++) {
            const uint32_t e0 = (it * RG_T + tid) * 4;
            const f32x4 a = *(const f32x4 *)(xr + e0);
            v[it] = f32x4{a.x + fix_to_f(xr2[e0]), a.y + fix_to_f(xr2[e0 + 1]), a.z + fix_to_f(xr2[e0 + 2]),
                          a.w + fix_to_f(xr2[e0 + 3])};
            if ((it * RG_T + tid) / 4 == blockIdx.x) *(f32x4 *)(P.xout + e0) = v[it];  // this workgroup's 16 rows
            wn[it] = *(const f32x4 *)(wr + e0);
            sq = fmaf(v[it].x, v[it].x, sq); sq = fmaf(v[it].y, v[it].y, sq);
            sq = fmaf(v[it].z, v[it].z, sq); sq = fmaf(v[it].w, v[it].w, sq);
        }
        if (tid < 16) P.zero[blockIdx.x * 16 + tid] = 0;
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
            u.x = wn[it].x * (u.x * rms_inv); u.y = wn[it].y * (u.y * rms_inv);
            u.z = wn[it].z * (u.z * rms_inv); u.w = wn[it].w * (u.w * rms_inv);
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
    // ---- gate/up (units 0..5): this lane's half super-block of x (limbs,
    // block scales, sums) in registers
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
        for (uint32_t u = 0; u < FX_GT; u++) {
            wait_vm_dyn(cnt(u + 1));
            lds_bar();  // (u = 0: also every wave done with xb in the third slot)
            issue(u + 2);
            // (u = 5: down tile 2 too, into what was unit 4's slot)
            if (ZH_FFN_EARLY && u == FX_GT - 1) issue(u + 3);
            if (u == 0) ZH_TRACE_POINT(11);
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
    ZH_TRACE_POINT(3);
    // ---- SwiGLU of the 48 rows as XQ limbs in blocks of 16 (the Q6_K scale
    // groups), by wave 0 (lanes 48..63 form an unused fourth group), published
    // to the XCD as one block of FX_XW epoch-tagged words: limbs [3 groups][3
    // limbs][16 B] as 36 dwords, xs [3], z [3] = -32 (sum of the group's X) xs.
    uint8_t *act = lds + FX_ACT + FX_XBLK;
    if (wave == 0) {
        const float v = lane < FX_RA ? silu_mul(yl[lane], yl[RG_MAXROWS + lane]) : 0.f;
        const float a = row16_max(fabsf(v));
        float inv, sc;
        xq_scales(a, inv, sc);
        const int X = xq_quant(v, inv);
        int l0, l1, l2;
        xq_limbs(X, l0, l1, l2);
        const int sx = row16_sum_i(X);
        if (lane < FX_RA) {
            const uint32_t g = lane / 16, e = lane % 16;
            act[(g * 3 + 0) * 16 + e] = (uint8_t)l0;
            act[(g * 3 + 1) * 16 + e] = (uint8_t)l1;
            act[(g * 3 + 2) * 16 + e] = (uint8_t)l2;
            if (e == 0) {
                ((float *)(act + 144))[g] = sc;
                ((float *)(act + 156))[g] = -32.f * ((float)sx * sc);
            }
        }
        __builtin_amdgcn_wave_barrier();  // (one wave: its LDS accesses complete in order)
        const uint32_t word = lane < 42 ? ((const uint32_t *)act)[lane] : 0u;
        if (lane < FX_XW) tag_store(P.xact + (size_t)w * FX_XW + lane, __uint_as_float(word), E);
    }
    // ---- the XCD's 32 blocks (waves 6 and 7 poll 16 each; they issue no
    // down-tile copies, so their polls drain nothing of the ring) into LDS
    uint32_t *xact = (uint32_t *)(lds + FX_ACT);  // [32 blocks][FX_XW]
    __shared__ uint32_t s_okx[2];
    if (wave >= 6) {
        float v[FX_XPW];
        const uint32_t b0 = (wave - 6) * (XCD_PER / 2) * FX_XW;
        const bool okw = tag_wait<FX_XPW>(P.xact + (size_t)h * XCD_PER * FX_XW + b0, E, P.ctl, v);
#pragma unroll
        for (int i = 0; i < FX_XPW; i++) xact[b0 + lane + 64 * i] = __float_as_uint(v[i]);
        if (lane == 0) s_okx[wave - 6] = okw ? 1u : 0u;
    }
    lds_bar();
    // unit 5's slot and the XQ image are free: down tiles 3 and 4 go there.
    // (Issued only now: a CU returns vector-memory data in request order, so
    // a poll issued behind them would wait for their bytes.)
    for (uint32_t u = FX_GT + (ZH_FFN_EARLY ? 3 : 2); u < FX_GT + FX_DS; u++) issue(u);
    const bool ok = s_okx[0] != 0 && s_okx[1] != 0;
    ZH_TRACE_POINT(6);
    // every workgroup of the XCD published, so every one has read the epoch
    if (j == 0 && tid == 0 && ok) *(volatile uint32_t *)ep = E;
    // ---- down (units 6..13): thread (rr, cg) = (tid / 32, tid % 32) takes
    // the record of row 16 (u - 6) + rr of this workgroup's 128 and column
    // group cg (the SwiGLU rows of the XCD's workgroup cg); a team of 32
    // lanes sums a row
    const uint32_t rr = tid / 32, cg = tid % 32;
    uint32_t A[3][3][4];
    float axs[3], az[3];
    {
        const uint32_t *blk = xact + cg * FX_XW;
#pragma unroll
        for (int g = 0; g < 3; g++) {
#pragma unroll
            for (int k = 0; k < 3; k++) {
                const u32x4 q4 = *(const u32x4 *)(blk + (g * 3 + k) * 4);
                A[g][k][0] = q4.x; A[g][k][1] = q4.y; A[g][k][2] = q4.z; A[g][k][3] = q4.w;
            }
            axs[g] = __uint_as_float(blk[36 + g]);
            az[g] = __uint_as_float(blk[39 + g]);
        }
    }
    ZH_TRACE_POINT(4);
    float *rsum = (float *)(lds + FX_ACT + FX_XBLK + 256);  // [128] the rows' sums
    const uint32_t wc = 32 * h + cg;                         // the column group's workgroup
    const bool g1b = (3 * wc + 1) % 16 == 0;                 // its group 1 opens the second super-block
    for (uint32_t u = FX_GT; u < FX_NU; u++) {
        // copies still allowed in flight after unit u: u + 1 .. u + 4 (u = 6),
        // else u + 1 .. u + 3 (those issued)
        wait_vm_dyn(dcw * (u == FX_GT ? FX_DS - 1 : min(FX_DS - 2, FX_NU - 1 - u)));
        lds_bar();
        if (u > FX_GT && u + FX_DS - 1 < FX_NU) issue(u + FX_DS - 1);  // into unit u - 1's slot
        const uint32_t *rp = (const uint32_t *)(ring + ((u - FX_GT) % FX_DS) * FX_DTB + tid * FX_REC);
        uint32_t rc[11];
#pragma unroll
        for (int i = 0; i < 11; i++) rc[i] = rp[i];
        float r3[3];
#pragma unroll
        for (int g = 0; g < 3; g++) {
            const uint32_t q0 = rc[3 * g], q1 = rc[3 * g + 1], qh = rc[3 * g + 2];
            const uint32_t c[4] = {(q0 & 0x0F0F0F0Fu) | ((qh << 4) & 0x30303030u),
                                   ((q0 >> 4) & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u),
                                   (q1 & 0x0F0F0F0Fu) | (qh & 0x30303030u),
                                   ((q1 >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u)};
            int D[3] = {0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int k = 0; k < 3; k++) D[k] = sdot4(c[i], A[g][k][i], D[k]);
            const float sc = (float)(int)(int8_t)((rc[9] >> (8 * g)) & 0xFF);
            r3[g] = sc * fmaf(axs[g], comb_f(D[0], D[1], D[2]), az[g]);  // codes - 32 through az
        }
        const float da = h2f(rc[10]), db = h2f(rc[10] >> 16);
        float r = fmaf(da, r3[0], fmaf(g1b ? db : da, r3[1], db * r3[2]));
        r = team_sum_dpp<32>(r);
        if (cg == 0) rsum[(u - FX_GT) * 16 + rr] = r;
    }
    lds_bar();
    ZH_TRACE_POINT(5);
    // ---- the XCD's share of rows [128 j, +128) into the residual (one
    // device atomic per XCD and row)
    if (tid < FX_RROWS) {
        float s = rsum[tid];
        if (!ok) s = __builtin_nanf("");  // the exchange's wait gave up
        fix_add(P.acc + j * FX_RROWS + tid, s);
    }
    // the wait gave up: the fixed-point sums cannot carry a NaN, so the
    // workgroup's rows of the plain part become NaN instead (written by the
    // threads that stored them, so in program order after them)
    if (!ok) {
#pragma unroll
        for (int it = 0; it < NB / 8; it++)
            if ((it * RG_T + tid) / 4 == blockIdx.x)
                *(f32x4 *)(P.xout + (it * RG_T + tid) * 4) = f32x4{__builtin_nanf(""), __builtin_nanf(""),
                                                                   __builtin_nanf(""), __builtin_nanf("")};
    }
    ZH_TRACE_POINT(7);
}

ZH_TRACE_DUMP_FN(zh_debug_trace_ffn)

// Packs ffn_down (Q6_K [4096][12288]) into the per-workgroup column records
// k_ffn_xcd reads: one thread per (workgroup w, row r).
__global__ void k_ffn_pack_down(const uint8_t *q6, uint8_t *pk) {
    const uint32_t gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= XCD_N * XCD_PER * FX_H) return;
    // record of row r and column group w (columns [48 w, 48 w + 48)); stored
    // for workgroup (XCD w / 32, slot r / 128) at [row r % 128][group w % 32]
    const uint32_t w = gid / FX_H, r = gid % FX_H;
    const uint8_t *row = q6 + (size_t)r * (FX_F / 256) * 210;
    uint32_t rec[11] = {};
    for (uint32_t g = 0; g < 3; g++) {
        const uint32_t G = 3 * w + g, sb = G / 16, e0 = (G % 16) * 16;  // 16 elements of super-block sb
        const uint8_t *blk = row + sb * 210;
        uint32_t q0 = 0, q1 = 0, qh = 0;
        for (uint32_t e = 0; e < 16; e++) {
            // Q6_K element x of a super-block: half n = x / 128, sub-block
            // s = (x % 128) / 32, i = x % 32: low 4 bits from
            // ql[64 n + 32 (s & 1) + i] (nibble s >> 1), high 2 bits from
            // qh[32 n + i] >> 2 s
            const uint32_t x = e0 + e, n = x / 128, s = (x % 128) / 32, i = x % 32;
            const uint32_t lo = (blk[64 * n + 32 * (s & 1) + i] >> (4 * (s >> 1))) & 0xF;
            const uint32_t hi = (blk[128 + 32 * n + i] >> (2 * s)) & 3;
            // record: elements 0-3 in the low nibbles of q0's bytes, 4-7 in
            // the high nibbles; 8-15 likewise in q1; high pairs in byte e % 4
            // of qh, bits 2 (e / 4)
            if (e < 8) q0 |= lo << (8 * (e % 4) + 4 * (e / 4));
            else q1 |= lo << (8 * (e % 4) + 4 * ((e - 8) / 4));
            qh |= hi << (8 * (e % 4) + 2 * (e / 4));
        }
        rec[3 * g] = q0;
        rec[3 * g + 1] = q1;
        rec[3 * g + 2] = qh;
        rec[9] |= (uint32_t)blk[192 + G % 16] << (8 * g);  // int8 scale of the 16 elements
    }
    const uint8_t *ba = row + ((3 * w) / 16) * 210, *bb = row + ((3 * w + 2) / 16) * 210;
    rec[10] = (uint32_t)ba[208] | ((uint32_t)ba[209] << 8) | ((uint32_t)bb[208] << 16) | ((uint32_t)bb[209] << 24);
    const uint32_t owner = (w / XCD_PER) * XCD_PER + r / FX_RROWS;
    uint32_t *dst = (uint32_t *)(pk + (size_t)owner * FX_SLICE + ((size_t)(r % FX_RROWS) * XCD_PER + w % XCD_PER) * FX_REC);
    for (int i = 0; i < 11; i++) dst[i] = rec[i];
}

uint32_t zhk_ffn_xcd_flag_words() { return FX_FLAG_WORDS; }
uint64_t zhk_ffn_pack_bytes() { return (uint64_t)XCD_N * XCD_PER * FX_SLICE; }
uint64_t zhk_ffn_part_bytes() { return (uint64_t)XCD_N * XCD_PER * FX_XW * 8; }

bool zhk_ffn_xcd_supported(zh_ctx *c, uint32_t hidden, uint32_t ffn) {
    return hidden == FX_H && ffn == FX_F && !c->concurrent && zhk_xcd_round_robin(c);
}

int zhk_ffn_pack_down(zh_ctx *c, const uint8_t *q6, uint8_t *pk) {
    const uint32_t n = XCD_N * XCD_PER * FX_H;
    hipLaunchKernelGGL(k_ffn_pack_down, dim3((n + 255) / 256), dim3(256), 0, c->stream, q6, pk);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

int zhk_ffn_xcd(zh_ctx *c, const float *xa, const zh_fix *xb, const float *norm_w, float eps, const uint8_t *wg,
                const uint8_t *wu, const uint8_t *pk, float *part, float *xout, zh_fix *acc, zh_fix *zero,
                uint32_t *flags) {
    if (((uintptr_t)xa & 15) || ((uintptr_t)xb & 15) || ((uintptr_t)norm_w & 15) || ((uintptr_t)wg & 15) ||
        ((uintptr_t)wu & 15) || ((uintptr_t)pk & 15) || ((uintptr_t)part & 15) || ((uintptr_t)xout & 15) || !acc ||
        !zero)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "ffn_xcd: 16-byte aligned operands");
    FfnP P = {};
    P.xa = xa; P.xb = xb; P.norm_w = norm_w; P.eps = eps; P.wg = wg; P.wu = wu; P.pk = pk;
    P.xact = (uint64_t *)part; P.xout = xout; P.acc = acc; P.zero = zero; P.flags = flags; P.ctl = c->err_dev;
    static bool attr = false;
    if (!attr) {
        ZH_HIP(c, hipFuncSetAttribute((const void *)k_ffn_xcd, hipFuncAttributeMaxDynamicSharedMemorySize, (int)RG_LDS));
        attr = true;
    }
    hipLaunchKernelGGL(k_ffn_xcd, dim3(XCD_N * XCD_PER), dim3(RG_T), RG_LDS, c->stream, P);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
