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

namespace {

constexpr int LPB_T = 256;       // threads per workgroup
constexpr int XB_STRIDE = 784;   // LDS bytes per 256-element x block (768 limbs + pad)

// LDS image of the activation: limbs[b][j][k][32] (j = 32-element sub-block,
// k = limb) at b*XB_STRIDE, then per-sub-block scale xs and 16-element sums.
struct XLds {
    uint8_t *limb;   // nb * XB_STRIDE bytes
    float *xs;       // nb * 8
    float *xz16;     // nb * 16
};

ZH_DEV XLds xlds_view(uint8_t *base, uint32_t nb) {
    XLds v;
    v.limb = base;
    v.xs = (float *)(base + (size_t)nb * XB_STRIDE);
    v.xz16 = v.xs + nb * 8;
    return v;
}
static inline uint32_t xlds_bytes(uint32_t K) { return (K / 256) * (XB_STRIDE + 8 * 4 + 16 * 4); }

// Workgroup-cooperative: x[0..K) (f32, global) -> XQ limbs in LDS.
// With norm_w != nullptr, x is replaced by norm_w * x * rsqrt(mean(x^2)+eps)
// (cpuRmsNormMul, forward.zig:618-626) first; the normalised vector is also
// written to `normed_out` by workgroup 0 when that pointer is non-null.
ZH_DEV void stage_x(const float *__restrict__ x, const float *__restrict__ norm_w, float eps, uint32_t K,
                    XLds lx, float *red, float *normed_out) {
    const uint32_t tid = threadIdx.x;
    float rms_inv = 1.f;
    if (norm_w) {
        float sq = 0.f;
        for (uint32_t i = tid * 4; i < K; i += LPB_T * 4) {
            f32x4 v = *(const f32x4 *)(x + i);
            sq = fmaf(v.x, v.x, sq); sq = fmaf(v.y, v.y, sq); sq = fmaf(v.z, v.z, sq); sq = fmaf(v.w, v.w, sq);
        }
        sq = wave_sum(sq);
        if ((tid & 63) == 0) red[tid >> 6] = sq;
        __syncthreads();
        const float tot = red[0] + red[1] + red[2] + red[3];
        rms_inv = 1.0f / sqrtf(tot / (float)K + eps);
    }
    // 8 lanes per 32-element block, 4 consecutive elements per lane
    for (uint32_t e0 = tid * 4; e0 < K; e0 += LPB_T * 4) {
        f32x4 v = *(const f32x4 *)(x + e0);
        if (norm_w) {
            f32x4 w = *(const f32x4 *)(norm_w + e0);
            v.x = w.x * (v.x * rms_inv); v.y = w.y * (v.y * rms_inv);
            v.z = w.z * (v.z * rms_inv); v.w = w.w * (v.w * rms_inv);
            if (normed_out && blockIdx.x == 0 && blockIdx.y == 0) *(f32x4 *)(normed_out + e0) = v;
        }
        // block max over the 8 lanes of this 32-element block (DPP)
        const float a = row8_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        float inv, sc;
        xq_scales(a, inv, sc);
        int X[4] = {xq_quant(v.x, inv), xq_quant(v.y, inv), xq_quant(v.z, inv), xq_quant(v.w, inv)};
        int l0[4], l1[4], l2[4];
#pragma unroll
        for (int i = 0; i < 4; i++) xq_limbs(X[i], l0[i], l1[i], l2[i]);
        const uint32_t blk32 = e0 / 32, b = blk32 / 8, j = blk32 % 8, lo = e0 % 32;
        uint8_t *dst = lx.limb + (size_t)b * XB_STRIDE + j * 96 + lo;
        *(uint32_t *)(dst) = pack4(l0[0], l0[1], l0[2], l0[3]);
        *(uint32_t *)(dst + 32) = pack4(l1[0], l1[1], l1[2], l1[3]);
        *(uint32_t *)(dst + 64) = pack4(l2[0], l2[1], l2[2], l2[3]);
        int s = X[0] + X[1] + X[2] + X[3];
        s += __builtin_amdgcn_update_dpp(0, s, 0xB1, 0xF, 0xF, false);  // 16 elements = 4 lanes
        s += __builtin_amdgcn_update_dpp(0, s, 0x4E, 0xF, 0xF, false);
        const uint32_t sub = (tid & 7);
        if (sub == 0) lx.xs[b * 8 + j] = sc;
        if ((sub & 3) == 0) lx.xz16[b * 16 + j * 2 + (sub >> 2)] = (float)s * sc;
    }
    __syncthreads();
}

// Workgroup-cooperative copy of a pre-quantised XQ vector (zh_device.h
// layout) into the LDS image: no arithmetic, 108 bytes per 32 elements.
ZH_DEV void stage_xq(const uint8_t *__restrict__ xq, uint32_t K, XLds lx) {
    const uint32_t tid = threadIdx.x, nblk = K / 32, nb = K / 256;
    const XQView v = xq_view((void *)xq, nblk);
    // limbs: 96 bytes per 32-element block = 6 x 16 B chunks
    for (uint32_t c = tid; c < nblk * 6; c += LPB_T) {
        const uint32_t blk32 = c / 6, part = c % 6;
        const u32x4 d = *(const u32x4 *)(v.limb + (size_t)blk32 * 96 + part * 16);
        *(u32x4 *)(lx.limb + (size_t)(blk32 / 8) * XB_STRIDE + (blk32 % 8) * 96 + part * 16) = d;
    }
    for (uint32_t j = tid; j < nblk; j += LPB_T) lx.xs[j] = v.xs[j];
    for (uint32_t j = tid; j < nblk * 2; j += LPB_T) lx.xz16[j] = v.xsum[j];
    (void)nb;
    __syncthreads();
}

ZH_DEV void lds_load_limbs(uint32_t *dst, const uint8_t *src) {  // 96 bytes -> 24 dwords
#pragma unroll
    for (int i = 0; i < 6; i++) {
        u32x4 v = *(const u32x4 *)(src + 16 * i);
        dst[4 * i] = v.x; dst[4 * i + 1] = v.y; dst[4 * i + 2] = v.z; dst[4 * i + 3] = v.w;
    }
}

ZH_DEV int comb_i(int d0, int d1, int d2) { return (d2 * 256 + d1) * 256 + d0; }
ZH_DEV float comb_f(int d0, int d1, int d2) { return fmaf((float)d2, 65536.f, (float)(d1 * 256 + d0)); }

// ---------------------------------------------------------------------------
// Q4_K block: 144 bytes = 9 dwordx4 {d,dmin,sc[0..3]... , qs[128]}.
// ---------------------------------------------------------------------------
struct LpbQ4K {
    static constexpr int RAW = 36, BPB = 144;
    ZH_DEVM static void load(const uint8_t *blk, uint32_t *raw) {
#pragma unroll
        for (int i = 0; i < 9; i++) {
            u32x4 v = *(const u32x4 *)(blk + 16 * i);
            raw[4 * i] = v.x; raw[4 * i + 1] = v.y; raw[4 * i + 2] = v.z; raw[4 * i + 3] = v.w;
        }
    }
    // Accumulates row partial for one lane-block over sub-pair p (sub-blocks
    // 2p, 2p+1) into accd (d-scaled part) and accm (dmin-scaled part).
    struct Hdr {
        uint32_t scA, scB, mA, mB;  // packed 6-bit scales / mins, one per byte
        float d, dmin;
    };
    ZH_DEVM static Hdr header(const uint32_t *raw) {
        // getScaleMinK4 (forward.zig:229-238) for all j at once:
        // j<4: sc = s[j]&63, m = s[j+4]&63; j>=4: sc = (s[j+4]&15)|((s[j-4]>>6)<<4),
        // m = (s[j+4]>>4)|((s[j]>>6)<<4).
        Hdr h;
        const uint32_t w1 = raw[1], w2 = raw[2], w3 = raw[3];
        h.scA = w1 & 0x3F3F3F3Fu;
        h.mA = w2 & 0x3F3F3F3Fu;
        h.scB = (w3 & 0x0F0F0F0Fu) | ((w1 >> 2) & 0x30303030u);
        h.mB = ((w3 >> 4) & 0x0F0F0F0Fu) | ((w2 >> 2) & 0x30303030u);
        h.d = h2f(raw[0]);
        h.dmin = h2f(raw[0] >> 16);
        return h;
    }
};

// byte -> f32; the compiler selects v_cvt_f32_ubyte{0..3} for constant `byte`
ZH_DEV float ubyte_f(uint32_t w, int byte) { return (float)((w >> (8 * byte)) & 0xFFu); }

template <int TL, int V>
ZH_DEV float team_reduce_multi(float (&a)[V], int tlane) {
    int o = TL / 2;
#pragma unroll
    for (int step = V; step > 1; step >>= 1) {
        const bool up = (tlane & o) != 0;
#pragma unroll
        for (int i = 0; i < step / 2; i++) {
            float lo = a[i], hi = a[i + step / 2];
            float send = up ? lo : hi, keep = up ? hi : lo;
            a[i] = keep + __shfl_xor(send, o, 64);
        }
        o >>= 1;
    }
    float v = a[0];
#pragma unroll
    for (; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
template <int TL, int V>
ZH_DEV int owner_index(int tlane) {
    int idx = 0, o = TL / 2;
#pragma unroll
    for (int step = V; step > 1; step >>= 1) {
        idx = idx * 2 + ((tlane & o) ? 1 : 0);
        o >>= 1;
    }
    return idx;
}

ZH_DEV float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

}  // namespace

struct LpbP {
    const uint8_t *xq;     // pre-quantised activation (XQ); when set, x/norm_w are unused
    const float *x;        // f32 activation (K)
    const float *norm_w;   // optional RMSNorm weight (K) fused on the way in
    float eps;
    float *normed_out;     // optional: normalised x written by workgroup 0
    uint32_t M, K, acc, nseg, mode;
    uint64_t row_bytes;
    const uint8_t *segW[3];
    const uint8_t *segW2;  // up matrix (gate/up mode)
    float *segY[3];
    uint32_t seg_end[3];
    uint8_t *xq_out;       // gate/up mode, optional: the SwiGLU output also as XQ (M % 32 == 0)
    uint32_t *grp_cnt;     // with xq_out: one zeroed counter per 32-row group
};

enum { LPB_PLAIN = 0, LPB_GATE_UP = 1 };
constexpr uint32_t LPB_XQ_MAX_GROUPS = 16;  // 32-row groups one gate/up workgroup may publish

// Segment lookup for the batch starting at stacked row r0 (batches never
// straddle segments).
ZH_DEV void lpb_geom(const LpbP &p, uint32_t r0, uint32_t &seg_rows, uint32_t &rr0, uint32_t &sg) {
    uint32_t seg_start = 0;
    sg = 0;
    seg_rows = p.M;
    if (p.nseg > 1) {
        sg = (r0 >= p.seg_end[0] ? 1u : 0u) + (p.nseg > 2 && r0 >= p.seg_end[1] ? 1u : 0u);
        seg_start = sg ? p.seg_end[sg - 1] : 0u;
        seg_rows = p.seg_end[sg] - seg_start;
    }
    rr0 = r0 - seg_start;
}

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
                const uint8_t *Wb = m ? p.segW2 : p.segW[sg];
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
        float *yb = p.segY[sg];
        if (base != base_first) {
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t row = min(rr0 + r, seg_rows - 1);
                    const uint8_t *Wb = m ? p.segW2 : p.segW[sg];
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
        const uint8_t *W = p.segW[sg];
        float *yb = p.segY[sg];
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
constexpr uint32_t TILE_BYTES = LPB_T * 144;  // 256 Q4_K super-blocks

#ifdef ZH_EXP_TRACE
__device__ uint64_t g_exp_trace[8192 * 8];
#define TRACE(slot) do { if (threadIdx.x == 0 && blockIdx.x < 8192 && (slot) < 8) \
    g_exp_trace[blockIdx.x * 8 + (slot)] = __builtin_amdgcn_s_memrealtime(); } while (0)
extern "C" int zh_exp_trace_dump(uint64_t *host, uint32_t n) {
    int rc = (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_exp_trace), (size_t)n * 8, 0, hipMemcpyDeviceToHost);
    static uint64_t zeros[8192 * 8];
    return rc | (int)hipMemcpyToSymbol(HIP_SYMBOL(g_exp_trace), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice);
}
#else
#define TRACE(slot) do { } while (0)
#endif


// Split staging for the tile kernel: the activation loads are issued before
// the first weight tile's loads (vector memory returns in order, so loads
// issued after 36 KB of tile data would wait for all of it), held in
// registers, and turned into the LDS image in one pass once they land.
// XCH = f32x4 chunks per lane = ceil(K / 1024); with the team width
// TL = pow2ceil(K / 256) that is max(1, TL / 4).
template <int XCH>
struct XRegsF {
    f32x4 x[XCH], w[XCH];
};
template <int XCH, bool NORM>
ZH_DEV void stage_x_issue(const float *__restrict__ x, const float *__restrict__ norm_w, uint32_t K,
                          XRegsF<XCH> &r) {
#pragma unroll
    for (int i = 0; i < XCH; i++) {
        const uint32_t e0 = min((i * LPB_T + threadIdx.x) * 4, K - 4);  // clamped: static load count
        r.x[i] = *(const f32x4 *)(x + e0);
        if (NORM) r.w[i] = *(const f32x4 *)(norm_w + e0);
    }
}
template <int XCH>
ZH_DEV void stage_x_finish(const XRegsF<XCH> &r, bool has_norm, float eps, uint32_t K, XLds lx, float *red,
                           float *normed_out) {
    const uint32_t tid = threadIdx.x;
    float rms_inv = 1.f;
    if (has_norm) {
        float sq = 0.f;
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            if ((i * LPB_T + tid) * 4 < K) {
                const f32x4 v = r.x[i];
                sq = fmaf(v.x, v.x, sq); sq = fmaf(v.y, v.y, sq); sq = fmaf(v.z, v.z, sq); sq = fmaf(v.w, v.w, sq);
            }
        }
        sq = wave_sum(sq);
        if ((tid & 63) == 0) red[tid >> 6] = sq;
        __syncthreads();
        const float tot = red[0] + red[1] + red[2] + red[3];
        rms_inv = 1.0f / sqrtf(tot / (float)K + eps);
    }
#pragma unroll
    for (int i = 0; i < XCH; i++) {
        const uint32_t e0 = (i * LPB_T + tid) * 4;
        if (e0 >= K) break;  // uniform per 8-lane group (K % 32 == 0)
        f32x4 v = r.x[i];
        if (has_norm) {
            const f32x4 w = r.w[i];
            v.x = w.x * (v.x * rms_inv); v.y = w.y * (v.y * rms_inv);
            v.z = w.z * (v.z * rms_inv); v.w = w.w * (v.w * rms_inv);
            if (normed_out && blockIdx.x == 0) *(f32x4 *)(normed_out + e0) = v;
        }
        // block max over the 8 lanes of this 32-element block (DPP)
        const float a = row8_max(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        float inv, sc;
        xq_scales(a, inv, sc);
        int X[4] = {xq_quant(v.x, inv), xq_quant(v.y, inv), xq_quant(v.z, inv), xq_quant(v.w, inv)};
        int l0[4], l1[4], l2[4];
#pragma unroll
        for (int q = 0; q < 4; q++) xq_limbs(X[q], l0[q], l1[q], l2[q]);
        const uint32_t blk32 = e0 / 32, b = blk32 / 8, j = blk32 % 8, lo = e0 % 32;
        uint8_t *dst = lx.limb + (size_t)b * XB_STRIDE + j * 96 + lo;
        *(uint32_t *)(dst) = pack4(l0[0], l0[1], l0[2], l0[3]);
        *(uint32_t *)(dst + 32) = pack4(l1[0], l1[1], l1[2], l1[3]);
        *(uint32_t *)(dst + 64) = pack4(l2[0], l2[1], l2[2], l2[3]);
        int sm = X[0] + X[1] + X[2] + X[3];
        sm += __builtin_amdgcn_update_dpp(0, sm, 0xB1, 0xF, 0xF, false);  // 16 elements = 4 lanes
        sm += __builtin_amdgcn_update_dpp(0, sm, 0x4E, 0xF, 0xF, false);
        const uint32_t sub = (tid & 7);
        if (sub == 0) lx.xs[b * 8 + j] = sc;
        if ((sub & 3) == 0) lx.xz16[b * 16 + j * 2 + (sub >> 2)] = (float)sm * sc;
    }
    __syncthreads();
}

// Pre-quantised XQ: limbs (96 B per 32 elements), xs, xsum16 held in registers.
// XQCH = 16-byte limb chunks per lane = ceil(6 * K/32 / 256) <= ceil(3 TL / 16);
// the K/32 block scales and 2 K/32 sums take ceil(XQCH / 6) and ceil(XQCH / 3)
// values per lane.
template <int XQCH>
struct XRegsQ {
    static constexpr int NXS = (XQCH + 5) / 6, NXZ = (XQCH + 2) / 3;
    u32x4 limb[XQCH];
    float xs[NXS];
    float xz[NXZ];
};
template <int XQCH>
ZH_DEV void stage_xq_issue(const uint8_t *__restrict__ xq, uint32_t K, XRegsQ<XQCH> &r) {
    const uint32_t tid = threadIdx.x, nblk = K / 32;
    const XQView v = xq_view((void *)xq, nblk);
#pragma unroll
    for (int i = 0; i < XQCH; i++) {
        const uint32_t c = min(i * LPB_T + tid, nblk * 6 - 1);  // clamped: static load count
        r.limb[i] = *(const u32x4 *)(v.limb + (size_t)c * 16);
    }
#pragma unroll
    for (int i = 0; i < XRegsQ<XQCH>::NXS; i++) r.xs[i] = v.xs[min(i * LPB_T + tid, nblk - 1)];
#pragma unroll
    for (int i = 0; i < XRegsQ<XQCH>::NXZ; i++) r.xz[i] = v.xsum[min(i * LPB_T + tid, nblk * 2 - 1)];
}
template <int XQCH>
ZH_DEV void stage_xq_finish(const XRegsQ<XQCH> &r, uint32_t K, XLds lx) {
    const uint32_t tid = threadIdx.x, nblk = K / 32;
#pragma unroll
    for (int i = 0; i < XQCH; i++) {
        const uint32_t c = i * LPB_T + tid;
        if (c < nblk * 6) {
            const uint32_t blk32 = c / 6, part = c % 6;
            *(u32x4 *)(lx.limb + (size_t)(blk32 / 8) * XB_STRIDE + (blk32 % 8) * 96 + part * 16) = r.limb[i];
        }
    }
#pragma unroll
    for (int i = 0; i < XRegsQ<XQCH>::NXS; i++)
        if (i * LPB_T + tid < nblk) lx.xs[i * LPB_T + tid] = r.xs[i];
#pragma unroll
    for (int i = 0; i < XRegsQ<XQCH>::NXZ; i++)
        if (i * LPB_T + tid < nblk * 2) lx.xz16[i * LPB_T + tid] = r.xz[i];
    __syncthreads();
}

// Stages the activation into the LDS image (XQ copy, f32, or f32 with a
// fused RMSNorm), calling fetch() -- the first weight tile's loads -- after
// the activation loads are issued and before they are waited on. Each of the
// three paths is straight-line so the wait counts stay exact.
template <int XQCH, int XCH, class Fetch>
ZH_DEV void stage_and_fetch(const LpbP &p, XLds lx, float *red, const Fetch &fetch) {
    if (p.xq) {
        XRegsQ<XQCH> xr;
        stage_xq_issue(p.xq, p.K, xr);
        fetch();
        stage_xq_finish(xr, p.K, lx);
    } else if (p.norm_w) {
        XRegsF<XCH> xr;
        stage_x_issue<XCH, true>(p.x, p.norm_w, p.K, xr);
        fetch();
        stage_x_finish(xr, true, p.eps, p.K, lx, red, p.normed_out);
    } else {
        XRegsF<XCH> xr;
        stage_x_issue<XCH, false>(p.x, nullptr, p.K, xr);
        fetch();
        stage_x_finish(xr, false, p.eps, p.K, lx, red, nullptr);
    }
}

template <int NM, int NCH, int RPB>
ZH_DEV void tile_fetch(const LpbP &p, uint32_t bi, uint32_t row_bytes, u32x4 (&st)[NM][NCH]) {
    uint32_t seg_rows, rr0, sg;
    lpb_geom(p, bi * RPB, seg_rows, rr0, sg);
    const uint32_t n16 = min((uint32_t)RPB, seg_rows - rr0) * row_bytes / 16;
#pragma unroll
    for (int m = 0; m < NM; m++) {
        const u32x4 *src = (const u32x4 *)((m ? p.segW2 : p.segW[sg]) + (size_t)rr0 * row_bytes);
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            // unconditional (clamped) loads keep the outstanding-load count
            // static, so waits on earlier loads need not drain the tile
            const uint32_t c = min(j * LPB_T + threadIdx.x, n16 - 1);
            st[m][j] = __builtin_nontemporal_load(src + c);
        }
    }
}

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
#ifdef ZH_EXP_TILE
        uint32_t xx = 0;
        for (int i = 0; i < 36; i++) xx ^= raw[i];
        accd = (float)(xx & 1);
#else
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
#endif
        float res = active ? fmaf(h.d, accd, -h.dmin * accm) : 0.f;
        res = team_sum_dpp<TL>(res);
        float *yb = p.segY[sg];
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
            const uint32_t scw[4] = {s0, s1, s2, s3};
            const int i0 = 8 * h + 2 * g, i1 = i0 + 1;
            const int sc0 = (int)(int8_t)((scw[i0 >> 2] >> (8 * (i0 & 3))) & 0xFF);
            const int sc1 = (int)(int8_t)((scw[i1 >> 2] >> (8 * (i1 & 3))) & 0xFF);
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
        float *yb = p.segY[sg];
        if (tlane == 0 && (uint32_t)rt < nrows) {
            float out = res;
            if (p.acc) out += yb[rr0 + rt];
            yb[rr0 + rt] = out;
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
    static int off = -1, capm = -1;
    if (off < 0) {
        off = getenv("ZH_NO_TILE") ? 1 : 0;
        const char *e = getenv("ZH_TILE_CAP");
        capm = e ? atoi(e) : 3;
    }
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
    static int off = -1, capm = -1;
    if (off < 0) {
        off = getenv("ZH_NO_TILE") ? 1 : 0;
        const char *e = getenv("ZH_TILE6_CAP");
        capm = e ? atoi(e) : 2;
    }
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
                 float *normed_out, uint32_t K, uint32_t acc, const void *xq, uint8_t *xq_out, uint32_t *grp_cnt) {
    if (!zhk_lpb_supported(qtype, K) || (mode == LPB_GATE_UP && qtype != ZH_Q4_K) || nseg < 1 || nseg > 3)
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
    if (xq_out && (mode != LPB_GATE_UP || nseg != 1 || p.M % 32 || !grp_cnt))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "lpb: XQ output needs gate/up mode, one segment, M %% 32 == 0");
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
    static int capm = -1;
    if (capm < 0) {
        const char *e = getenv("ZH_LPB_CAP");
        capm = e ? atoi(e) : 0;
    }
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
