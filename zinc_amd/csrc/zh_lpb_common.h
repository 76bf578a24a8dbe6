// zh_lpb_common.h -- device helpers shared by the lane-per-block and tile
// DMMV kernels (zh_dmmv_lpb.hip) and their several-vector forms
// (zh_dmmv_batched.hip): the LDS activation image, the staging of f32 / XQ
// activations into it, the Q4_K block header, team reductions and the
// tile fetch.
#pragma once
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
    float *ycopy;          // optional (one segment, Q6_K): every output row also stored here
};

enum { LPB_PLAIN = 0, LPB_GATE_UP = 1 };

// Segment sg's matrix and output by selects: an index into the kernel
// argument's arrays with a per-batch value makes the compiler copy the
// arrays to scratch memory.
ZH_DEV const uint8_t *lpb_w(const LpbP &p, uint32_t sg) { return sg == 0 ? p.segW[0] : sg == 1 ? p.segW[1] : p.segW[2]; }
ZH_DEV float *lpb_y(const LpbP &p, uint32_t sg) { return sg == 0 ? p.segY[0] : sg == 1 ? p.segY[1] : p.segY[2]; }
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

constexpr uint32_t TILE_BYTES = LPB_T * 144;  // 256 Q4_K super-blocks

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
        const u32x4 *src = (const u32x4 *)((m ? p.segW2 : lpb_w(p, sg)) + (size_t)rr0 * row_bytes);
#pragma unroll
        for (int j = 0; j < NCH; j++) {
            // unconditional (clamped) loads keep the outstanding-load count
            // static, so waits on earlier loads need not drain the tile
            const uint32_t c = min(j * LPB_T + threadIdx.x, n16 - 1);
            st[m][j] = __builtin_nontemporal_load(src + c);
        }
    }
}
