// zh_dmmv_lpb.hip — "lane per block" DMMV for the K-quants (Q4_K, Q6_K).
//
// Each lane owns one 256-element super-block column of the weight matrix and
// walks rows; a team of pow2ceil(K/256) lanes covers a row. The activation is
// staged once per workgroup into LDS as XQ limbs (optionally RMS-normalised
// on the way in, which fuses the producer's rms_norm into the DMMV), and every
// lane reads the limbs of its block from LDS for R rows at a time. Compared
// with one lane per 64 elements, the per-block header (d, dmin, 12 scale
// bytes) is decoded once per 256 weights and the team reduction is 4x
// narrower, which takes the VALU cost down to ~1.4 instructions per weight.
#include "zh_device.h"
#include "zh_internal.h"

#include "zh_lpb_common.h"

// Q4_K, one lane per super-block. NM = 2 in gate/up mode (rows of gate and up).
#ifndef ZH_LPB_MINB
#define ZH_LPB_MINB 2
#endif
template <int TL, int R, int MODE>
__global__ __launch_bounds__(LPB_T, ZH_LPB_MINB) void k_dmmv_q4k_lpb(LpbP p) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    __shared__ float red[4];
    constexpr int NM = MODE == LPB_GATE_UP ? 2 : 1;
    constexpr int V = NM * R;
    constexpr int TPW = LPB_T / TL;
    const uint32_t nb = p.K / 256;
    XLds lx = xlds_view(lds_raw, nb);
    const int tid = threadIdx.x, tlane = tid % TL, team = tid / TL;
    const bool active = (uint32_t)tlane < nb;
    const uint32_t b = active ? tlane : 0;
    const uint8_t *xl = lx.limb + (size_t)b * XB_STRIDE;
    uint32_t raw[NM][R][LpbQ4K::RAW];
    // Loop trip counts are uniform across the workgroup (teams past M compute
    // a clamped row and skip the write) so the multi-wave team reduction's
    // barriers always match.
    const uint32_t wg_rows = TPW * R, wg_stride = gridDim.x * wg_rows;
    const uint32_t base_first = blockIdx.x * wg_rows;
    // the first batch's weights stream in while the activation is staged
    if (base_first < p.M) {
        const uint32_t r0 = min(base_first + team * R, p.M - 1);
        uint32_t seg_rows, rr0, sg;
        lpb_geom(p, r0, seg_rows, rr0, sg);
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t row = min(rr0 + r, seg_rows - 1);
                const uint8_t *Wb = m ? p.segW2 : lpb_w(p, sg);
                LpbQ4K::load(Wb + (size_t)row * p.row_bytes + (size_t)b * 144, raw[m][r]);  // inactive lanes read block 0
            }
    }
    if (p.xq) stage_xq(p.xq, p.K, lx);
    else stage_x(p.x, p.norm_w, p.eps, p.K, lx, red, p.normed_out);
    for (uint32_t base = base_first; base < p.M; base += wg_stride) {
        const bool team_ok = base + team * R < p.M;
        const uint32_t r0 = min(base + team * R, p.M - 1);
        uint32_t seg_rows, rr0, sg;
        lpb_geom(p, r0, seg_rows, rr0, sg);
        float *yb = lpb_y(p, sg);
        if (base != base_first) {
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t row = min(rr0 + r, seg_rows - 1);
                    const uint8_t *Wb = m ? p.segW2 : lpb_w(p, sg);
                    LpbQ4K::load(Wb + (size_t)row * p.row_bytes + (size_t)b * 144, raw[m][r]);  // inactive lanes read block 0
                }
        }
        // Row-mats are processed one after another; each sub-pair's LDS limb
        // offset is chained through an empty asm to the previous accumulator
        // so the compiler keeps one sub-pair of limbs (48 VGPRs) live at a
        // time instead of hoisting every load of the batch.
        float part[V];
        float dep = 0.f;
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const LpbQ4K::Hdr h = LpbQ4K::header(raw[m][r]);
                float accd = 0.f, accm = 0.f;
#pragma unroll
                for (int pp = 0; pp < 4; pp++) {
                    uint32_t xo = (uint32_t)(2 * pp) * 96u;
                    asm volatile("" : "+v"(xo) : "v"(dep));
                    uint32_t L[2][24];
                    lds_load_limbs(L[0], xl + xo);
                    lds_load_limbs(L[1], xl + xo + 96);
                    const float xs0 = lx.xs[b * 8 + 2 * pp], xs1 = lx.xs[b * 8 + 2 * pp + 1];
                    const float xz0 = lx.xz16[b * 16 + 4 * pp] + lx.xz16[b * 16 + 4 * pp + 1];
                    const float xz1 = lx.xz16[b * 16 + 4 * pp + 2] + lx.xz16[b * 16 + 4 * pp + 3];
                    int D[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const uint32_t w = raw[m][r][4 + 8 * pp + i];
                        const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                        for (int k = 0; k < 3; k++) {
                            D[0][k] = sdot4(lo, L[0][k * 8 + i], D[0][k]);
                            D[1][k] = sdot4(hi, L[1][k * 8 + i], D[1][k]);
                        }
                    }
                    const uint32_t scw = (2 * pp < 4) ? h.scA : h.scB, mw = (2 * pp < 4) ? h.mA : h.mB;
                    const float sc0 = ubyte_f(scw, (2 * pp) & 3), sc1 = ubyte_f(scw, (2 * pp + 1) & 3);
                    const float m0 = ubyte_f(mw, (2 * pp) & 3), m1 = ubyte_f(mw, (2 * pp + 1) & 3);
                    const float S0 = (float)comb_i(D[0][0], D[0][1], D[0][2]);
                    const float S1 = (float)comb_i(D[1][0], D[1][1], D[1][2]);
                    accd = fmaf(sc0 * xs0, S0, accd);
                    accd = fmaf(sc1 * xs1, S1, accd);
                    accm = fmaf(m0, xz0, accm);
                    accm = fmaf(m1, xz1, accm);
                    dep = accd;
                }
                part[m * R + r] = active ? fmaf(h.d, accd, -h.dmin * accm) : 0.f;
            }

        float res;
        int idx;
        constexpr int TLW = TL > 64 ? 64 : TL;  // lanes of the team inside one wave
        constexpr int STRIDE = TLW / V;
        res = team_reduce_multi<TLW, V>(part, tlane % TLW);
        idx = owner_index<TLW, V>(tlane % TLW);
        if (TL > 64) {  // teams spanning several waves: add the per-wave sums
            __shared__ float xred[4][V];
            const int wave = tid >> 6;
            if ((tlane % TLW) % STRIDE == 0) xred[wave][idx] = res;
            __syncthreads();
            float t = 0.f;
#pragma unroll
            for (int w = 0; w < TL / 64; w++) t += xred[(team * TL) / 64 + w][idx];
            res = t;
            __syncthreads();
        }
        const bool writer = team_ok && (tlane < TLW) && ((tlane % STRIDE) == 0);
        if (MODE == LPB_GATE_UP) {
            const float upv = __shfl(res, ((tid & 63) + R * STRIDE) & 63, 64);
            if (writer && idx < R && rr0 + idx < seg_rows) yb[rr0 + idx] = silu_mul(res, upv);
        } else if (writer && rr0 + idx < seg_rows) {
            float out = res;
            if (p.acc) out += yb[rr0 + idx];
            yb[rr0 + idx] = out;
            if (p.ycopy) p.ycopy[rr0 + idx] = out;
        }
    }
}

// ---------------------------------------------------------------------------
// Q6_K block: 210 bytes {ql[128], qh[64], int8 sc[16], f16 d}, dword-aligned
// loads of 14 dwords (+ realignment) per half-block would exceed the register
// budget, so a lane owns half a super-block (128 elements, h = half index):
// ql[64h..64h+64), qh[32h..32h+32), sc[8h..8h+8), d.
// ---------------------------------------------------------------------------
template <int TL, int R>
__global__ __launch_bounds__(LPB_T, ZH_LPB_MINB) void k_dmmv_q6k_lpb(LpbP p) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    __shared__ float red[4];
    constexpr int TPW = LPB_T / TL;
    const uint32_t nb = p.K / 256, nh = nb * 2;
    XLds lx = xlds_view(lds_raw, nb);
    if (p.xq) stage_xq(p.xq, p.K, lx);
    else stage_x(p.x, p.norm_w, p.eps, p.K, lx, red, p.normed_out);
    const int tid = threadIdx.x, tlane = tid % TL, team = tid / TL;
    const bool active = (uint32_t)tlane < nh;
    const uint32_t hb = active ? tlane : 0, b = hb >> 1, h = hb & 1;
    const uint8_t *xl = lx.limb + (size_t)b * XB_STRIDE + h * 4 * 96;  // sub-blocks 4h..4h+3
    const uint32_t wg_rows = TPW * R, wg_stride = gridDim.x * wg_rows;
    for (uint32_t base = blockIdx.x * wg_rows; base < p.M; base += wg_stride) {
        const bool team_ok = base + team * R < p.M;
        const uint32_t r0 = min(base + team * R, p.M - 1);
        uint32_t seg_rows, rr0, sg;
        lpb_geom(p, r0, seg_rows, rr0, sg);
        const uint8_t *W = lpb_w(p, sg);
        float *yb = lpb_y(p, sg);
        // per row: ql 64 B (17 dwords w/ realign), qh 32 B (9), sc 8 B + d (6 dwords cover 192+8h..210)
        uint32_t rq[R][17], rh[R][9], rs[R][6], sh[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t row = min(rr0 + r, seg_rows - 1);
            const uint8_t *blk = W + (size_t)row * p.row_bytes + (size_t)b * 210;
            sh[r] = (uint32_t)((uintptr_t)blk & 3);
            if (active) {
                const uint32_t *a = (const uint32_t *)((uintptr_t)(blk + 64 * h) & ~(uintptr_t)3);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    u32x4 v = *(const u32x4_a4 *)(a + 4 * i);
                    rq[r][4 * i] = v.x; rq[r][4 * i + 1] = v.y; rq[r][4 * i + 2] = v.z; rq[r][4 * i + 3] = v.w;
                }
                rq[r][16] = a[16];
                const uint32_t *c = (const uint32_t *)((uintptr_t)(blk + 128 + 32 * h) & ~(uintptr_t)3);
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    u32x4 v = *(const u32x4_a4 *)(c + 4 * i);
                    rh[r][4 * i] = v.x; rh[r][4 * i + 1] = v.y; rh[r][4 * i + 2] = v.z; rh[r][4 * i + 3] = v.w;
                }
                rh[r][8] = c[8];
                const uint32_t *s = (const uint32_t *)((uintptr_t)(blk + 192) & ~(uintptr_t)3);
                u32x4 v = *(const u32x4_a4 *)s;
                rs[r][0] = v.x; rs[r][1] = v.y; rs[r][2] = v.z; rs[r][3] = v.w;
                rs[r][4] = s[4];
                rs[r][5] = s[5];
            }
        }
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.f;
        // quarter g of this half: elements 32g + l, x sub-block 4h + g
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t xo = (uint32_t)g * 96u;
            asm volatile("" : "+v"(xo) : "v"(acc[R - 1]));
            uint32_t L[24];
            lds_load_limbs(L, xl + xo);
            const float xs = lx.xs[b * 8 + 4 * h + g];
            const float z0 = -32.f * lx.xz16[b * 16 + (4 * h + g) * 2];
            const float z1 = -32.f * lx.xz16[b * 16 + (4 * h + g) * 2 + 1];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t s_ = sh[r];
                int D[2][3] = {{0, 0, 0}, {0, 0, 0}};  // two 16-element scale groups
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    // ql byte index within the half: l + 32*(g&1); nibble g>>1
                    const int qi = (g & 1) * 8 + i;
                    const uint32_t a = __builtin_amdgcn_alignbyte(rq[r][qi + 1], rq[r][qi], s_);
                    const uint32_t c = __builtin_amdgcn_alignbyte(rh[r][i + 1], rh[r][i], s_);
                    const uint32_t lo4 = (g >> 1) ? ((a >> 4) & 0x0F0F0F0Fu) : (a & 0x0F0F0F0Fu);
                    const uint32_t hi2 = ((c >> (2 * g)) << 4) & 0x30303030u;
                    const uint32_t q = lo4 | hi2;  // 6-bit code, unsigned (offset 32 applied via sums)
                    const int grp = i >> 2;       // 16-element scale group within the quarter
#pragma unroll
                    for (int k = 0; k < 3; k++) D[grp][k] = sdot4(q, L[k * 8 + i], D[grp][k]);
                }
                // scales sc[8h + l/16 + 2g] for l-groups 0, 1; d at byte 16 of the realigned tail
                uint32_t s0 = __builtin_amdgcn_alignbyte(rs[r][1], rs[r][0], s_);
                uint32_t s1 = __builtin_amdgcn_alignbyte(rs[r][2], rs[r][1], s_);
                uint32_t s2 = __builtin_amdgcn_alignbyte(rs[r][3], rs[r][2], s_);
                uint32_t s3 = __builtin_amdgcn_alignbyte(rs[r][4], rs[r][3], s_);
                const uint32_t scw[4] = {s0, s1, s2, s3};
                const int i0 = 8 * h + 2 * g, i1 = i0 + 1;  // scale byte indices (h folded in at runtime)
                const int sc0 = (int)(int8_t)((scw[i0 >> 2] >> (8 * (i0 & 3))) & 0xFF);
                const int sc1 = (int)(int8_t)((scw[i1 >> 2] >> (8 * (i1 & 3))) & 0xFF);
                const float S0 = comb_f(D[0][0], D[0][1], D[0][2]);
                const float S1 = comb_f(D[1][0], D[1][1], D[1][2]);
                acc[r] = fmaf((float)sc0, fmaf(xs, S0, z0), acc[r]);
                acc[r] = fmaf((float)sc1, fmaf(xs, S1, z1), acc[r]);
            }
        }
        float part[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint32_t dw = __builtin_amdgcn_alignbyte(rs[r][5], rs[r][4], sh[r]);  // bytes 208..211
            part[r] = active ? h2f(dw) * acc[r] : 0.f;
        }
        constexpr int TLW = TL > 64 ? 64 : TL;
        constexpr int STRIDE = TLW / R;
        float res = team_reduce_multi<TLW, R>(part, tlane % TLW);
        const int idx = owner_index<TLW, R>(tlane % TLW);
        if (TL > 64) {
            __shared__ float xred[4][R];
            const int wave = tid >> 6;
            if ((tlane % TLW) % STRIDE == 0) xred[wave][idx] = res;
            __syncthreads();
            float t = 0.f;
#pragma unroll
            for (int w = 0; w < TL / 64; w++) t += xred[(team * TL) / 64 + w][idx];
            res = t;
            __syncthreads();
        }
        if (team_ok && tlane < TLW && (tlane % STRIDE) == 0 && rr0 + idx < seg_rows) {
            float out = res;
            if (p.acc) out += yb[rr0 + idx];
            yb[rr0 + idx] = out;
            if (p.ycopy) p.ycopy[rr0 + idx] = out;
        }
    }
}


// ---------------------------------------------------------------------------
// Coalesced-tile variant for Q4_K. In the lane-per-block load pattern the 64
// lanes of one 16-byte load sit 144 bytes apart, so each load instruction
// touches 64 cache lines; on MI355X that caps a pure read at ~2.2 TB/s against
// ~6.2 TB/s when consecutive lanes read consecutive 16-byte chunks. Here each
// batch of rows -- a contiguous byte range of the weight matrix -- is read
// with the contiguous pattern into registers and written to an LDS tile, and
// every lane then reads its own super-block from LDS (16-byte reads at a
// 144-byte lane stride hit all 64 banks once per 16 lanes: conflict-free).
// The next batch's loads are in flight while the current batch is computed.
// ---------------------------------------------------------------------------

#define TRACE(slot) ZH_TRACE_POINT(slot)
ZH_TRACE_DUMP_FN(zh_debug_trace_lpb)

// 64-lane teams (K > 8192) stage an XQ image of up to 56 KB: two workgroups per CU
template <int TL, int MODE>
__global__ __launch_bounds__(LPB_T, TL >= 64 ? 2 : 3) void k_dmmv_q4k_tile(LpbP p) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    __shared__ float red[4];
    __shared__ float gate_res[LPB_T / TL];
    constexpr int NM = MODE == LPB_GATE_UP ? 2 : 1;
    constexpr int TPB = LPB_T / TL;         // teams (one row each) per batch
    constexpr int RPB = TPB / NM;           // rows of each matrix per batch
    constexpr int NCH = (9 + NM - 1) / NM;  // 16-byte chunks per lane per matrix
    const uint32_t nb = p.K / 256, row_bytes = nb * 144, sub_bytes = RPB * row_bytes;
    XLds lx = xlds_view(lds_raw, nb);
    uint8_t *tile = lds_raw + (size_t)nb * (XB_STRIDE + 96);
    const int tid = threadIdx.x, tlane = tid % TL, team = tid / TL;
    const int mat = team / RPB, rt = team % RPB;
    const bool active = (uint32_t)tlane < nb;
    const uint32_t b = active ? tlane : 0;
    const uint8_t *xl = lx.limb + (size_t)b * XB_STRIDE;
    const uint32_t nbatch = (p.M + RPB - 1) / RPB;
    // Batches are dealt round-robin, except when the SwiGLU output is emitted
    // as XQ: then each workgroup takes a contiguous run of `per` batches so it
    // completes whole 32-row groups where it can and publishes once, after its
    // loop (the host sizes the grid so every run is non-empty).
    const bool contig = MODE == LPB_GATE_UP && p.xq_out;
    const uint32_t per = (nbatch + gridDim.x - 1) / gridDim.x;
    const uint32_t b0 = contig ? blockIdx.x * per : blockIdx.x;
    const uint32_t b1 = contig ? min(nbatch, b0 + per) : nbatch;
    const uint32_t bstep = contig ? 1u : gridDim.x;
    u32x4 st[NM][NCH];
    uint32_t bi = b0;
    TRACE(0);
    // grid <= nbatch (host), so the first batch always exists
    stage_and_fetch<(3 * TL + 15) / 16, (TL / 4 > 1 ? TL / 4 : 1)>(
        p, lx, red, [&] { tile_fetch<NM, NCH, RPB>(p, bi, row_bytes, st); });
    TRACE(1);
    int it = 0;
    for (; bi < b1; bi += bstep, it++) {
        uint32_t seg_rows, rr0, sg;
        lpb_geom(p, bi * RPB, seg_rows, rr0, sg);
        const uint32_t nrows = min((uint32_t)RPB, seg_rows - rr0);
        const uint32_t n16 = nrows * row_bytes / 16;
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int j = 0; j < NCH; j++) {
                const uint32_t c = j * LPB_T + tid;
                if (c < n16) *(u32x4 *)(tile + m * sub_bytes + c * 16) = st[m][j];
            }
        __syncthreads();
        TRACE(2 + min(it, 4));
        if (bi + bstep < b1) tile_fetch<NM, NCH, RPB>(p, bi + bstep, row_bytes, st);
        uint32_t raw[LpbQ4K::RAW];
        {
            const uint8_t *blk = tile + mat * sub_bytes + rt * row_bytes + b * 144;
#pragma unroll
            for (int i = 0; i < 9; i++) {
                const u32x4 v = *(const u32x4 *)(blk + 16 * i);
                raw[4 * i] = v.x; raw[4 * i + 1] = v.y; raw[4 * i + 2] = v.z; raw[4 * i + 3] = v.w;
            }
        }
        const LpbQ4K::Hdr h = LpbQ4K::header(raw);
        float accd = 0.f, accm = 0.f;
#pragma unroll
        for (int pp = 0; pp < 4; pp++) {
            uint32_t xo = (uint32_t)(2 * pp) * 96u;
            asm volatile("" : "+v"(xo) : "v"(accd));
            uint32_t L[2][24];
            lds_load_limbs(L[0], xl + xo);
            lds_load_limbs(L[1], xl + xo + 96);
            const float xs0 = lx.xs[b * 8 + 2 * pp], xs1 = lx.xs[b * 8 + 2 * pp + 1];
            const float xz0 = lx.xz16[b * 16 + 4 * pp] + lx.xz16[b * 16 + 4 * pp + 1];
            const float xz1 = lx.xz16[b * 16 + 4 * pp + 2] + lx.xz16[b * 16 + 4 * pp + 3];
            int D[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t w = raw[4 + 8 * pp + i];
                const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                for (int k = 0; k < 3; k++) {
                    D[0][k] = sdot4(lo, L[0][k * 8 + i], D[0][k]);
                    D[1][k] = sdot4(hi, L[1][k * 8 + i], D[1][k]);
                }
            }
            const uint32_t scw = (2 * pp < 4) ? h.scA : h.scB, mw = (2 * pp < 4) ? h.mA : h.mB;
            const float sc0 = ubyte_f(scw, (2 * pp) & 3), sc1 = ubyte_f(scw, (2 * pp + 1) & 3);
            const float m0 = ubyte_f(mw, (2 * pp) & 3), m1 = ubyte_f(mw, (2 * pp + 1) & 3);
            const float S0 = (float)comb_i(D[0][0], D[0][1], D[0][2]);
            const float S1 = (float)comb_i(D[1][0], D[1][1], D[1][2]);
            accd = fmaf(sc0 * xs0, S0, accd);
            accd = fmaf(sc1 * xs1, S1, accd);
            accm = fmaf(m0, xz0, accm);
            accm = fmaf(m1, xz1, accm);
        }
        float res = active ? fmaf(h.d, accd, -h.dmin * accm) : 0.f;
        res = team_sum_dpp<TL>(res);
        float *yb = lpb_y(p, sg);
        if (MODE == LPB_GATE_UP) {
            if (mat == 0 && tlane == 0) gate_res[rt] = res;
            __syncthreads();
            if (mat == 1 && tlane == 0 && (uint32_t)rt < nrows) {
                const float v = silu_mul(gate_res[rt], res);
                if (p.xq_out) st_dev(yb + rr0 + rt, v);  // device scope: read by another workgroup below
                else yb[rr0 + rt] = v;
            }
        } else if (tlane == 0 && (uint32_t)rt < nrows) {
            float out = res;
            if (p.acc) out += yb[rr0 + rt];
            yb[rr0 + rt] = out;
            if (p.ycopy) p.ycopy[rr0 + rt] = out;
        }
        __syncthreads();  // the tile is rewritten by the next batch
    }
    if (contig) {
        // The SwiGLU output as XQ, the down projection's input: each 32-row
        // group is counted up to 32 published rows; the workgroup whose rows
        // complete it quantises the group's block. Rows were stored at device
        // scope, so after this workgroup's stores drain they are visible to
        // whichever workgroup's counter increment comes last.
        __shared__ uint32_t s_last[LPB_XQ_MAX_GROUPS];
        const uint32_t r0 = b0 * RPB, r1 = min(p.M, b1 * RPB);
        const uint32_t g0 = r0 / 32, ng = (r1 - 1) / 32 - g0 + 1;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if ((uint32_t)tid < ng) {
            const uint32_t g = g0 + tid;
            const uint32_t n = min(r1, g * 32 + 32) - max(r0, g * 32);
            const uint32_t prev = __hip_atomic_fetch_add(p.grp_cnt + g, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last[tid] = prev + n == 32 ? 1u : 0u;
        }
        __syncthreads();
        const float *yb = p.segY[0];
        for (uint32_t i = tid / 64; i < ng; i += LPB_T / 64) {
            if (!s_last[i]) continue;
            const uint32_t g = g0 + i;
            // both 32-lane halves quantise the same block (identical writes)
            const float v = ld_dev(yb + g * 32 + (tid & 31));
            xq_store_block32(v, tid & 31, xq_view(p.xq_out, p.M / 32), g);
            if ((tid & 63) == 0) __hip_atomic_store(p.grp_cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    TRACE(7);
}


// Q6_K on the coalesced tile: one lane per half super-block (128 elements,
// ql[64h..), qh[32h..), sc[8h..), d) as in k_dmmv_q6k_lpb, with the block
// bytes read from the LDS tile. Q6_K blocks are 210 bytes, so a block starts
// 2-byte aligned; dword reads are realigned with alignbyte.
template <int TL, int NCH>
__global__ __launch_bounds__(LPB_T, 2) void k_dmmv_q6k_tile(LpbP p) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    __shared__ float red[4];
    constexpr int RPB = LPB_T / TL;  // rows per batch
    // NCH = ceil(RPB * row bytes / 4 KB) 16-byte chunks per lane and tile
    const uint32_t nb = p.K / 256, row_bytes = nb * 210, nh = nb * 2;
    XLds lx = xlds_view(lds_raw, nb);
    uint8_t *tile = lds_raw + (size_t)nb * (XB_STRIDE + 96);
    const int tid = threadIdx.x, tlane = tid % TL, rt = tid / TL;
    const bool active = (uint32_t)tlane < nh;
    const uint32_t hb = active ? tlane : 0, b = hb >> 1, h = hb & 1;
    const uint8_t *xl = lx.limb + (size_t)b * XB_STRIDE + h * 4 * 96;  // sub-blocks 4h..4h+3
    const uint32_t nbatch = (p.M + RPB - 1) / RPB;
    u32x4 st[1][NCH];
    uint32_t bi = blockIdx.x;
    TRACE(0);
    // grid <= nbatch (host), so the first batch always exists
    stage_and_fetch<(3 * TL / 2 + 15) / 16, (TL / 8 > 1 ? TL / 8 : 1)>(
        p, lx, red, [&] { tile_fetch<1, NCH, RPB>(p, bi, row_bytes, st); });
    TRACE(1);
    int it = 0;
    for (; bi < nbatch; bi += gridDim.x, it++) {
        uint32_t seg_rows, rr0, sg;
        lpb_geom(p, bi * RPB, seg_rows, rr0, sg);
        const uint32_t nrows = min((uint32_t)RPB, seg_rows - rr0);
        const uint32_t n16 = nrows * row_bytes / 16;
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            const uint32_t c = j * LPB_T + tid;
            if (c < n16) *(u32x4 *)(tile + c * 16) = st[0][j];
        }
        __syncthreads();
        TRACE(2 + min(it, 4));
        if (bi + gridDim.x < nbatch) tile_fetch<1, NCH, RPB>(p, bi + gridDim.x, row_bytes, st);
        const uint32_t boff = rt * row_bytes + b * 210;
        const uint32_t sh = boff & 3;
        uint32_t rq[17], rh[9], rs[6];
        {
            const uint32_t *a = (const uint32_t *)(tile + ((boff + 64 * h) & ~3u));
#pragma unroll
            for (int i = 0; i < 17; i++) rq[i] = a[i];
            const uint32_t *c = (const uint32_t *)(tile + ((boff + 128 + 32 * h) & ~3u));
#pragma unroll
            for (int i = 0; i < 9; i++) rh[i] = c[i];
            const uint32_t *sp = (const uint32_t *)(tile + ((boff + 192) & ~3u));
#pragma unroll
            for (int i = 0; i < 6; i++) rs[i] = sp[i];
        }
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint32_t xo = (uint32_t)g * 96u;
            asm volatile("" : "+v"(xo) : "v"(acc));
            uint32_t L[24];
            lds_load_limbs(L, xl + xo);
            const float xs = lx.xs[b * 8 + 4 * h + g];
            const float z0 = -32.f * lx.xz16[b * 16 + (4 * h + g) * 2];
            const float z1 = -32.f * lx.xz16[b * 16 + (4 * h + g) * 2 + 1];
            int D[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int qi = (g & 1) * 8 + i;
                const uint32_t av = __builtin_amdgcn_alignbyte(rq[qi + 1], rq[qi], sh);
                const uint32_t cv = __builtin_amdgcn_alignbyte(rh[i + 1], rh[i], sh);
                const uint32_t lo4 = (g >> 1) ? ((av >> 4) & 0x0F0F0F0Fu) : (av & 0x0F0F0F0Fu);
                const uint32_t hi2 = ((cv >> (2 * g)) << 4) & 0x30303030u;
                const uint32_t q = lo4 | hi2;  // unsigned 6-bit code; the -32 offset enters via z0/z1
                const int grp = i >> 2;
#pragma unroll
                for (int k = 0; k < 3; k++) D[grp][k] = sdot4(q, L[k * 8 + i], D[grp][k]);
            }
            const uint32_t s0 = __builtin_amdgcn_alignbyte(rs[1], rs[0], sh);
            const uint32_t s1 = __builtin_amdgcn_alignbyte(rs[2], rs[1], sh);
            const uint32_t s2 = __builtin_amdgcn_alignbyte(rs[3], rs[2], sh);
            const uint32_t s3 = __builtin_amdgcn_alignbyte(rs[4], rs[3], sh);
            // scales 8h + 2g and 8h + 2g + 1: word 2h + g / 2, bytes 2 (g % 2)
            // and 2 (g % 2) + 1 (a select on the per-lane h, g static: an
            // indexed register array would become scratch memory)
            const uint32_t sw = h ? (g < 2 ? s2 : s3) : (g < 2 ? s0 : s1);
            const int sc0 = (int)(int8_t)((sw >> (16 * (g & 1))) & 0xFF);
            const int sc1 = (int)(int8_t)((sw >> (16 * (g & 1) + 8)) & 0xFF);
            const float S0 = comb_f(D[0][0], D[0][1], D[0][2]);
            const float S1 = comb_f(D[1][0], D[1][1], D[1][2]);
            acc = fmaf((float)sc0, fmaf(xs, S0, z0), acc);
            acc = fmaf((float)sc1, fmaf(xs, S1, z1), acc);
        }
        const uint32_t dw = __builtin_amdgcn_alignbyte(rs[5], rs[4], sh);  // bytes 208..211
        float res = active ? h2f(dw) * acc : 0.f;
        constexpr int TLW = TL > 64 ? 64 : TL;
        res = team_sum_dpp<TLW>(res);
        if (TL > 64) {  // team spans TL/64 waves
            __shared__ float xred[LPB_T / 64];
            if ((tid & 63) == 0) xred[tid >> 6] = res;
            __syncthreads();
            float t = 0.f;
#pragma unroll
            for (int w = 0; w < TL / 64; w++) t += xred[(rt * TL) / 64 + w];
            res = t;
        }
        float *yb = lpb_y(p, sg);
        if (tlane == 0 && (uint32_t)rt < nrows) {
            float out = res;
            if (p.acc) out += yb[rr0 + rt];
            yb[rr0 + rt] = out;
            if (p.ycopy) p.ycopy[rr0 + rt] = out;
        }
        __syncthreads();  // the tile (and xred) are rewritten by the next batch
        }
    TRACE(7);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
static uint32_t pow2ceil(uint32_t v) {
    uint32_t t = 1;
    while (t < v) t <<= 1;
    return t;
}

template <int TL>
static int launch_q4k(zh_ctx *c, const LpbP &p, uint32_t wgs, uint32_t lds) {
    if (p.mode == LPB_GATE_UP)
        hipLaunchKernelGGL((k_dmmv_q4k_lpb<TL, 1, LPB_GATE_UP>), dim3(wgs), dim3(LPB_T), lds, c->stream, p);
    else
        hipLaunchKernelGGL((k_dmmv_q4k_lpb<TL, 1, LPB_PLAIN>), dim3(wgs), dim3(LPB_T), lds, c->stream, p);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
template <int TL>
static int launch_q6k(zh_ctx *c, const LpbP &p, uint32_t wgs, uint32_t lds) {
    hipLaunchKernelGGL((k_dmmv_q6k_lpb<TL, 1>), dim3(wgs), dim3(LPB_T), lds, c->stream, p);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}


template <int TL>
static int launch_q4k_tile(zh_ctx *c, const LpbP &p, uint32_t wgs, uint32_t lds) {
    if (p.mode == LPB_GATE_UP)
        hipLaunchKernelGGL((k_dmmv_q4k_tile<TL, LPB_GATE_UP>), dim3(wgs), dim3(LPB_T), lds, c->stream, p);
    else
        hipLaunchKernelGGL((k_dmmv_q4k_tile<TL, LPB_PLAIN>), dim3(wgs), dim3(LPB_T), lds, c->stream, p);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

// Tile path: Q4_K with K <= 8192 (team of <= 32 lanes, LDS image + tile
// within 64 KB), 16-byte aligned matrices, and every segment but the last a
// whole number of batches.
static int try_q4k_tile(zh_ctx *c, const LpbP &p, uint32_t nseg, const uint32_t *M) {
    const bool off = zh_knob("ZH_NO_TILE");
    const int capm = zh_knob_int("ZH_TILE_CAP", 3);
    const uint32_t nb = p.K / 256;
    if (off || nb > 64) return -1;
    const uint32_t TL = pow2ceil(nb < 4 ? 4 : nb);
    const uint32_t nm = p.mode == LPB_GATE_UP ? 2 : 1;
    const uint32_t rpb = LPB_T / TL / nm;
    for (uint32_t s = 0; s < nseg; s++) {
        if (((uintptr_t)p.segW[s] & 15) || (s + 1 < nseg && M[s] % rpb)) return -1;
    }
    if (nm == 2 && ((uintptr_t)p.segW2 & 15)) return -1;
    const uint32_t nbatch = (p.M + rpb - 1) / rpb;
    uint32_t wgs = nbatch, cap = (uint32_t)c->cu_count * (uint32_t)(capm > 0 ? capm : 3);
    if (wgs > cap) wgs = cap;
    if (p.xq_out) {
        // contiguous batch runs: every workgroup gets a non-empty run
        const uint32_t per = (nbatch + wgs - 1) / wgs;
        wgs = (nbatch + per - 1) / per;
        if (nseg != 1 || nm != 2 || p.M % 32 || per * rpb / 32 + 2 > LPB_XQ_MAX_GROUPS) return -1;
    }
    const uint32_t lds = nb * (XB_STRIDE + 96) + TILE_BYTES;
    switch (TL) {
    case 4: return launch_q4k_tile<4>(c, p, wgs, lds);
    case 8: return launch_q4k_tile<8>(c, p, wgs, lds);
    case 16: return launch_q4k_tile<16>(c, p, wgs, lds);
    case 32: return launch_q4k_tile<32>(c, p, wgs, lds);
    default: return launch_q4k_tile<64>(c, p, wgs, lds);
    }
}


template <int TL>
static int launch_q6k_tile(zh_ctx *c, const LpbP &p, uint32_t wgs, uint32_t lds, uint32_t nch) {
    switch (nch) {
#define Q6T(N) case N: hipLaunchKernelGGL((k_dmmv_q6k_tile<TL, N>), dim3(wgs), dim3(LPB_T), lds, c->stream, p); break;
    Q6T(4) Q6T(5) Q6T(6) Q6T(7)  // RPB * K/256 is in (64, 128], so a tile is 3.3 .. 6.6 x 4 KB
#undef Q6T
    default: return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "q6k tile: %u chunks", nch);
    }
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

// Q6_K tile path: rows a multiple of 16 bytes (K % 2048 == 0), team of <= 128
// lanes (K <= 16384) and LDS image + tile within 64 KB.
static int try_q6k_tile(zh_ctx *c, const LpbP &p, uint32_t nseg, const uint32_t *M) {
    const bool off = zh_knob("ZH_NO_TILE");
    const int capm = zh_knob_int("ZH_TILE6_CAP", 2);
    const uint32_t nb = p.K / 256, row_bytes = nb * 210;
    // Very tall matrices (the LM head) give every workgroup dozens of batches;
    // there the per-row limb re-reads from LDS and the Q6_K unpack bound the
    // tile kernel, and the lane-per-block kernel measures faster.
    if (off || row_bytes % 16 || nb > 64 || p.M >= 65536) return -1;
    const uint32_t TL = pow2ceil(2 * nb < 4 ? 4 : 2 * nb);
    const uint32_t rpb = LPB_T / TL;
    const uint32_t lds = nb * (XB_STRIDE + 96) + rpb * row_bytes;
    if (lds > 65536) return -1;
    for (uint32_t s = 0; s < nseg; s++)
        if (((uintptr_t)p.segW[s] & 15) || (s + 1 < nseg && M[s] % rpb)) return -1;
    const uint32_t nbatch = (p.M + rpb - 1) / rpb;
    uint32_t per_cu = 163840 / (lds + 1024);
    if (per_cu > (uint32_t)(capm > 0 ? capm : 2)) per_cu = (uint32_t)(capm > 0 ? capm : 2);
    uint32_t wgs = nbatch, cap = (uint32_t)c->cu_count * (per_cu ? per_cu : 1);
    if (wgs > cap) wgs = cap;
    const uint32_t nch = (rpb * row_bytes + 4095) / 4096;
    switch (TL) {
    case 4: return launch_q6k_tile<4>(c, p, wgs, lds, nch);
    case 8: return launch_q6k_tile<8>(c, p, wgs, lds, nch);
    case 16: return launch_q6k_tile<16>(c, p, wgs, lds, nch);
    case 32: return launch_q6k_tile<32>(c, p, wgs, lds, nch);
    case 64: return launch_q6k_tile<64>(c, p, wgs, lds, nch);
    default: return launch_q6k_tile<128>(c, p, wgs, lds, nch);
    }
}

bool zhk_lpb_supported(uint32_t qtype, uint32_t K) {
    if (K % 256 || K == 0) return false;
    if (qtype == ZH_Q4_K) return K / 256 <= 256;
    if (qtype == ZH_Q6_K) return K / 128 <= 256;
    return false;
}

int zhk_dmmv_lpb(zh_ctx *c, uint32_t qtype, int mode, uint32_t nseg, const uint8_t *const *W, const uint8_t *W2,
                 float *const *y, const uint32_t *M, const float *x, const float *norm_w, float eps,
                 float *normed_out, uint32_t K, uint32_t acc, const void *xq, uint8_t *xq_out, uint32_t *grp_cnt,
                 float *ycopy) {
    if (!zhk_lpb_supported(qtype, K) || (mode == LPB_GATE_UP && qtype != ZH_Q4_K) || nseg < 1 || nseg > 3 ||
        (ycopy && (qtype != ZH_Q6_K || nseg != 1 || mode != LPB_PLAIN)))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "lpb: unsupported qtype/K/mode");
    LpbP p = {};
    p.x = x; p.norm_w = norm_w; p.eps = eps; p.normed_out = normed_out;
    p.xq = (const uint8_t *)xq;
    p.K = K; p.acc = acc; p.nseg = nseg; p.mode = (uint32_t)mode;
    p.row_bytes = zh_tensor_bytes(qtype, 1, K);
    uint32_t end = 0;
    const uint32_t R = 1;
    for (uint32_t s = 0; s < nseg; s++) {
        if (M[s] % R) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "lpb: segment rows %% %u", R);
        p.segW[s] = W[s]; p.segY[s] = y[s];
        end += M[s];
        p.seg_end[s] = end;
    }
    p.segW2 = W2;
    p.M = end;
    p.xq_out = xq_out;
    p.grp_cnt = grp_cnt;
    p.ycopy = ycopy;
    if (xq_out && (mode != LPB_GATE_UP || nseg != 1 || p.M % 32 || !grp_cnt))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "lpb: XQ output needs gate/up mode, one segment, M %% 32 == 0");
    {
        const int rc = zhk_dmmv_ring(c, qtype, mode, nseg, W, W2, y, M, x, norm_w, eps, normed_out, K, acc, xq,
                                     xq_out, grp_cnt);
        if (rc >= 0) return rc;
    }
    {
        const int rc = qtype == ZH_Q4_K ? try_q4k_tile(c, p, nseg, M) : try_q6k_tile(c, p, nseg, M);
        if (rc >= 0) return rc;
    }
    if (xq_out) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "lpb: XQ output needs the tile kernel (K <= 8192)");
    const uint32_t lanes = qtype == ZH_Q4_K ? K / 256 : K / 128;
    const uint32_t TL = pow2ceil(lanes < 4 ? 4 : lanes);
    const uint32_t teams = (p.M + R - 1) / R;
    const uint32_t tpw = LPB_T / TL;
    uint32_t wgs = (teams + tpw - 1) / tpw;
    const int capm = zh_knob_int("ZH_LPB_CAP", 0);
    const uint32_t cap = (uint32_t)c->cu_count * (capm > 0 ? (uint32_t)capm : 4u);
    if (wgs > cap) wgs = cap;
    const uint32_t lds = xlds_bytes(K);
    if (qtype == ZH_Q4_K) {
        switch (TL) {
        case 4: return launch_q4k<4>(c, p, wgs, lds);
        case 8: return launch_q4k<8>(c, p, wgs, lds);
        case 16: return launch_q4k<16>(c, p, wgs, lds);
        case 32: return launch_q4k<32>(c, p, wgs, lds);
        case 64: return launch_q4k<64>(c, p, wgs, lds);
        case 128: return launch_q4k<128>(c, p, wgs, lds);
        default: return launch_q4k<256>(c, p, wgs, lds);
        }
    }
    switch (TL) {
    case 4: return launch_q6k<4>(c, p, wgs, lds);
    case 8: return launch_q6k<8>(c, p, wgs, lds);
    case 16: return launch_q6k<16>(c, p, wgs, lds);
    case 32: return launch_q6k<32>(c, p, wgs, lds);
    case 64: return launch_q6k<64>(c, p, wgs, lds);
    case 128: return launch_q6k<128>(c, p, wgs, lds);
    default: return launch_q6k<256>(c, p, wgs, lds);
    }
}
