// zh_dmmv.hip — dequantise-fused mat-vec (DMMV) for Q4_K, Q6_K, Q8_0 and
// MXFP4 on gfx950, plus the activation quantiser and bit-exact dequant.
//
// Design (MI355X-first, not a translation of dmmv_*.comp):
//  * A "unit" is a fixed 64-element column slice of a row (32 for MXFP4).
//    Lane t of a team always owns unit t of every row it visits, so its slice
//    of the activation vector is loaded ONCE into registers (as XQ int8 limbs)
//    and reused for every row: no LDS or L1 traffic for x in the row loop.
//  * A team is K/64 lanes (power-of-two padded when it fits in a wave, or
//    whole waves when K > 4096). Teams walk R rows at a time, issuing all R
//    rows' 128-bit weight loads before any arithmetic (memory-level
//    parallelism for HBM3E), then reduce across the team with wave shuffles.
//  * Inner products run on v_dot4_i32_i8 against the 4/6/8-bit codes with
//    exact int32 accumulation; per-sub-block scales and mins are applied in
//    f32 afterwards: y = sum_j d*sc_j*(xs_j*S_j) - dmin*m_j*sum(x_j).
//  * Weights are read in GGUF layout straight from HBM (dword-aligned loads
//    plus v_alignbyte for the 210/34/17-byte block formats).
#include "zh_device.h"
#include "zh_internal.h"

#include <stdlib.h>

#include <vector>

// ---------------------------------------------------------------------------
// Activation quantiser: x (f32) -> XQ. One 32-lane half-wave per block.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_quantize_xq(const float *__restrict__ x, uint8_t *__restrict__ xq,
                                                     uint32_t K, uint32_t x_stride, uint64_t xq_stride) {
    const uint32_t nblk = K / 32;
    const uint32_t vec = blockIdx.y;
    const uint32_t blk = blockIdx.x * 8 + (threadIdx.x >> 5);
    const uint32_t l = threadIdx.x & 31;
    if (blk >= nblk) return;
    const float *xv = x + (size_t)vec * x_stride;
    XQView v = xq_view(xq + vec * xq_stride, nblk);
    float xi = xv[blk * 32 + l];
    float a = fabsf(xi);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 32));
    float inv, sc;
    xq_scales(a, inv, sc);
    int X = xq_quant(xi, inv);
    int l0, l1, l2;
    xq_limbs(X, l0, l1, l2);
    v.limb[blk * 96 + l] = (int8_t)l0;
    v.limb[blk * 96 + 32 + l] = (int8_t)l1;
    v.limb[blk * 96 + 64 + l] = (int8_t)l2;
    int s = X;
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 32);  // sum within 16-lane halves
    if (l == 0) v.xs[blk] = sc;
    if ((l & 15) == 0) v.xsum[blk * 2 + (l >> 4)] = (float)s * sc;
}

int zhk_quantize_xq(zh_ctx *c, const float *x, void *xq, uint32_t K, uint32_t n_vec, uint32_t x_stride) {
    uint32_t nblk = K / 32;
    hipLaunchKernelGGL(k_quantize_xq, dim3((nblk + 7) / 8, n_vec), dim3(256), 0, c->stream, x,
                       (uint8_t *)xq, K, x_stride, (uint64_t)zh_xq_bytes_int(K));
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

// ---------------------------------------------------------------------------
// Per-lane activation registers: 48 limb dwords + 4 scale/sum pairs.
// ---------------------------------------------------------------------------
struct XReg {
    uint32_t L[48];
    float xs[4];
    float xz[4];
};

ZH_DEV void load_limbs(uint32_t *dst, const int8_t *src, int ndw) {
    const u32x4 *p = (const u32x4 *)src;
#pragma unroll
    for (int i = 0; i < ndw / 4; i++) {
        u32x4 v = p[i];
        dst[4 * i + 0] = v.x; dst[4 * i + 1] = v.y; dst[4 * i + 2] = v.z; dst[4 * i + 3] = v.w;
    }
}

ZH_DEV u32x4 ld4(const uint8_t *p) { return *(const u32x4_a4 *)p; }

ZH_DEV int comb_int(int d0, int d1, int d2) { return (d2 * 256 + d1) * 256 + d0; }
ZH_DEV float comb_f32(int d0, int d1, int d2) { return fmaf((float)d2, 65536.f, (float)(d1 * 256 + d0)); }

// Q4_K / Q5_K sub-pair epilogue: raw[0..3] hold {d, dmin, scales[12]}, S0/S1
// the code . limb sums of sub-blocks 2p and 2p+1.
// getScaleMinK4 (forward.zig:229-238) for j = 2p, 2p+1, branch-free:
// p < 2: sc = s[j] & 63, m = s[j+4] & 63 (6-bit fields of w1, w2);
// p >= 2: sc = low nibble of s[j+4] | (s[j-4] >> 6) << 4,
//          m = high nibble of s[j+4] | (s[j] >> 6) << 4.
ZH_DEV float k4_epilogue(const uint32_t *raw, const XReg &xr, int p, float S0, float S1) {
    const bool lo4 = p < 2;
    const uint32_t w1 = raw[1], w2 = raw[2], w3 = raw[3];
    const uint32_t srcS = lo4 ? w1 : w3, srcM = lo4 ? w2 : w3;
    const uint32_t wa = lo4 ? 6u : 4u, wb = lo4 ? 0u : 2u, mo = lo4 ? 0u : 4u;
    uint32_t sc[2], mn[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; s2++) {
        const uint32_t off = 16u * (uint32_t)(p & 1) + 8u * (uint32_t)s2;
        sc[s2] = __builtin_amdgcn_ubfe(srcS, off, wa) | (__builtin_amdgcn_ubfe(w1, off + 6u, wb) << 4);
        mn[s2] = __builtin_amdgcn_ubfe(srcM, off + mo, wa) | (__builtin_amdgcn_ubfe(w2, off + 6u, wb) << 4);
    }
    float d = h2f(raw[0]), dmin = h2f(raw[0] >> 16);
    float A = fmaf((float)sc[1] * xr.xs[1], S1, (float)sc[0] * xr.xs[0] * S0);
    float B = fmaf((float)mn[1], xr.xz[1], (float)mn[0] * xr.xz[0]);
    return fmaf(d, A, -dmin * B);
}

// ---------------------------------------------------------------------------
// Q4_K: 144-byte blocks {f16 d, f16 dmin, 12 B packed 6-bit scales/mins,
// 128 B nibbles} (forward.zig:370-409). Unit u = (block u>>2, sub-pair p=u&3):
// qs[32p..32p+31] low nibbles -> sub-block 2p, high -> 2p+1.
// ---------------------------------------------------------------------------
struct FmtQ4K {
    static constexpr int EPU = 64, RAW = 12, QK = 256, BPB = 144;
    ZH_DEVM static void load_x(XReg &xr, XQView v, int u) {
        int xb = 2 * u;  // (256*(u>>2) + 64*(u&3)) / 32
#pragma unroll
        for (int s = 0; s < 2; s++) {
            load_limbs(&xr.L[s * 24], v.limb + (size_t)(xb + s) * 96, 24);
            xr.xs[s] = v.xs[xb + s];
            xr.xz[s] = v.xsum[(xb + s) * 2] + v.xsum[(xb + s) * 2 + 1];
        }
    }
    ZH_DEVM static void load_raw(const uint8_t *row, int u, uint32_t *raw) {
        const uint8_t *b = row + (size_t)(u >> 2) * 144;
        int p = u & 3;
        u32x4 h = ld4(b), q0 = ld4(b + 16 + 32 * p), q1 = ld4(b + 32 + 32 * p);
        raw[0] = h.x; raw[1] = h.y; raw[2] = h.z; raw[3] = h.w;
        raw[4] = q0.x; raw[5] = q0.y; raw[6] = q0.z; raw[7] = q0.w;
        raw[8] = q1.x; raw[9] = q1.y; raw[10] = q1.z; raw[11] = q1.w;
    }
    ZH_DEVM static float compute(const uint32_t *raw, const XReg &xr, int u) {
        int D[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t w = raw[4 + i];
            uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int k = 0; k < 3; k++) {
                D[0][k] = sdot4(lo, xr.L[k * 8 + i], D[0][k]);
                D[1][k] = sdot4(hi, xr.L[24 + k * 8 + i], D[1][k]);
            }
        }
        return k4_epilogue(raw, xr, u & 3, (float)comb_int(D[0][0], D[0][1], D[0][2]),
                           (float)comb_int(D[1][0], D[1][1], D[1][2]));
    }
};

// ---------------------------------------------------------------------------
// Q5_K: 176-byte blocks {f16 d, f16 dmin, 12 B packed scales/mins, qh[32],
// qs[128]} (forward.zig:326-368). Units as Q4_K; the fifth bit of element l
// of 64-group p is bit 2p (low half) / 2p+1 (high half) of qh[l]. Codes reach
// 31, so 31 * 32 * 2^22 overflows int32: the limb sums combine in f32.
// ---------------------------------------------------------------------------
struct FmtQ5K {
    static constexpr int EPU = 64, RAW = 20, QK = 256, BPB = 176;
    ZH_DEVM static void load_x(XReg &xr, XQView v, int u) { FmtQ4K::load_x(xr, v, u); }
    ZH_DEVM static void load_raw(const uint8_t *row, int u, uint32_t *raw) {
        const uint8_t *b = row + (size_t)(u >> 2) * 176;
        int p = u & 3;
        u32x4 h = ld4(b), q0 = ld4(b + 48 + 32 * p), q1 = ld4(b + 64 + 32 * p), e0 = ld4(b + 16), e1 = ld4(b + 32);
        raw[0] = h.x; raw[1] = h.y; raw[2] = h.z; raw[3] = h.w;
        raw[4] = q0.x; raw[5] = q0.y; raw[6] = q0.z; raw[7] = q0.w;
        raw[8] = q1.x; raw[9] = q1.y; raw[10] = q1.z; raw[11] = q1.w;
        raw[12] = e0.x; raw[13] = e0.y; raw[14] = e0.z; raw[15] = e0.w;
        raw[16] = e1.x; raw[17] = e1.y; raw[18] = e1.z; raw[19] = e1.w;
    }
    ZH_DEVM static float compute(const uint32_t *raw, const XReg &xr, int u) {
        const uint32_t p2 = 2u * (uint32_t)(u & 3);
        int D[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t w = raw[4 + i], h = raw[12 + i];
            const uint32_t lo = (w & 0x0F0F0F0Fu) | (((h >> p2) & 0x01010101u) << 4);
            const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | (((h >> (p2 + 1u)) & 0x01010101u) << 4);
#pragma unroll
            for (int k = 0; k < 3; k++) {
                D[0][k] = sdot4(lo, xr.L[k * 8 + i], D[0][k]);
                D[1][k] = sdot4(hi, xr.L[24 + k * 8 + i], D[1][k]);
            }
        }
        return k4_epilogue(raw, xr, u & 3, comb_f32(D[0][0], D[0][1], D[0][2]), comb_f32(D[1][0], D[1][1], D[1][2]));
    }
};

// ---------------------------------------------------------------------------
// Q6_K: 210-byte blocks {ql[128], qh[64], int8 sc[16], f16 d}
// (forward.zig:276-325). Unit u = (block u>>2, half h=(u>>1)&1, l0=16*(u&1)):
// l in [l0, l0+16) of all four quarters g (element 128h + 32g + l).
// ---------------------------------------------------------------------------
struct FmtQ6K {
    static constexpr int EPU = 64, RAW = 22, QK = 256, BPB = 210;
    ZH_DEVM static void load_x(XReg &xr, XQView v, int u) {
        int b = u >> 2, h = (u >> 1) & 1, half = u & 1;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            int xb = 8 * b + 4 * h + g;
#pragma unroll
            for (int k = 0; k < 3; k++) {
                u32x4 t = *(const u32x4 *)(v.limb + (size_t)xb * 96 + k * 32 + half * 16);
                xr.L[(g * 3 + k) * 4 + 0] = t.x; xr.L[(g * 3 + k) * 4 + 1] = t.y;
                xr.L[(g * 3 + k) * 4 + 2] = t.z; xr.L[(g * 3 + k) * 4 + 3] = t.w;
            }
            xr.xs[g] = v.xs[xb];
            xr.xz[g] = -32.f * v.xsum[xb * 2 + half];
        }
    }
    ZH_DEVM static void load_raw(const uint8_t *row, int u, uint32_t *raw) {
        const uint8_t *b = row + (size_t)(u >> 2) * 210;
        int h = (u >> 1) & 1, l0 = 16 * (u & 1);
        const uint8_t *pA = b + 64 * h + l0, *pB = pA + 32, *pC = b + 128 + 32 * h + l0;
        const uint8_t *srcs[3] = {pA, pB, pC};
#pragma unroll
        for (int s = 0; s < 3; s++) {
            uintptr_t a = (uintptr_t)srcs[s] & ~(uintptr_t)3;
            u32x4 t = *(const u32x4 *)a;
            raw[s * 5 + 0] = t.x; raw[s * 5 + 1] = t.y; raw[s * 5 + 2] = t.z; raw[s * 5 + 3] = t.w;
            raw[s * 5 + 4] = *(const uint32_t *)(a + 16);
        }
        {   // scales sc[0..16) and d: bytes 192..211 of the block
            uintptr_t a = (uintptr_t)(b + 192) & ~(uintptr_t)3;
            u32x4 t = *(const u32x4 *)a;
            raw[15] = t.x; raw[16] = t.y; raw[17] = t.z; raw[18] = t.w;
            raw[19] = *(const uint32_t *)(a + 16);
            raw[20] = *(const uint32_t *)(a + 20);
        }
        raw[21] = (uint32_t)((uintptr_t)b & 3);
    }
    ZH_DEVM static float compute(const uint32_t *raw, const XReg &xr, int u) {
        uint32_t sh = raw[21];
        uint32_t A[4], B[4], C[4], S[5];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            A[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], sh);
            B[i] = __builtin_amdgcn_alignbyte(raw[5 + i + 1], raw[5 + i], sh);
            C[i] = __builtin_amdgcn_alignbyte(raw[10 + i + 1], raw[10 + i], sh);
        }
#pragma unroll
        for (int i = 0; i < 5; i++) S[i] = __builtin_amdgcn_alignbyte(raw[15 + i + 1], raw[15 + i], sh);
        int D[4][3];
#pragma unroll
        for (int g = 0; g < 4; g++) D[g][0] = D[g][1] = D[g][2] = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t a = A[i], bq = B[i], c = C[i];
            uint32_t q[4];
            q[0] = (a & 0x0F0F0F0Fu) | ((c << 4) & 0x30303030u);
            q[1] = (bq & 0x0F0F0F0Fu) | ((c << 2) & 0x30303030u);
            q[2] = ((a >> 4) & 0x0F0F0F0Fu) | (c & 0x30303030u);
            q[3] = ((bq >> 4) & 0x0F0F0F0Fu) | ((c >> 2) & 0x30303030u);
#pragma unroll
            for (int g = 0; g < 4; g++)
#pragma unroll
                for (int k = 0; k < 3; k++) D[g][k] = sdot4(q[g], xr.L[(g * 3 + k) * 4 + i], D[g][k]);
        }
        int h = (u >> 1) & 1, half = u & 1;
        float d = h2f(S[4]);  // bytes 208..209
        float acc = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            int idx = 8 * h + half + 2 * g;  // sc[is + 2g], is = 8h + l/16
            int scv = (int)(int8_t)((S[idx >> 2] >> (8 * (idx & 3))) & 0xFF);
            float Sg = comb_f32(D[g][0], D[g][1], D[g][2]);
            // sum_l d*sc*(q-32)*x = d*sc*(xs*S - 32*sum x)
            acc = fmaf((float)scv, fmaf(xr.xs[g], Sg, xr.xz[g]), acc);
        }
        return d * acc;
    }
};

// ---------------------------------------------------------------------------
// Q8_0: 34-byte blocks {f16 d, int8 q[32]} (forward.zig:258-275). Unit u = two
// consecutive blocks (68 bytes, dword aligned when K % 64 == 0).
// ---------------------------------------------------------------------------
struct FmtQ80 {
    static constexpr int EPU = 64, RAW = 17, QK = 64, BPB = 68;
    ZH_DEVM static void load_x(XReg &xr, XQView v, int u) {
        int xb = 2 * u;
#pragma unroll
        for (int s = 0; s < 2; s++) {
            load_limbs(&xr.L[s * 24], v.limb + (size_t)(xb + s) * 96, 24);
            xr.xs[s] = v.xs[xb + s];
        }
    }
    ZH_DEVM static void load_raw(const uint8_t *row, int u, uint32_t *raw) {
        const uint8_t *b = row + (size_t)u * 68;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            u32x4 t = ld4(b + 16 * i);
            raw[4 * i] = t.x; raw[4 * i + 1] = t.y; raw[4 * i + 2] = t.z; raw[4 * i + 3] = t.w;
        }
        raw[16] = *(const uint32_t *)(b + 64);
    }
    ZH_DEVM static float compute(const uint32_t *raw, const XReg &xr, int u) {
        int D[2][3] = {{0, 0, 0}, {0, 0, 0}};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t q0 = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], 2);
            uint32_t q1 = raw[9 + i];
#pragma unroll
            for (int k = 0; k < 3; k++) {
                D[0][k] = sdot4(q0, xr.L[k * 8 + i], D[0][k]);
                D[1][k] = sdot4(q1, xr.L[24 + k * 8 + i], D[1][k]);
            }
        }
        float d0 = h2f(raw[0]), d1 = h2f(raw[8] >> 16);
        float S0 = comb_f32(D[0][0], D[0][1], D[0][2]);
        float S1 = comb_f32(D[1][0], D[1][1], D[1][2]);
        return fmaf(d1 * xr.xs[1], S1, d0 * xr.xs[0] * S0);
    }
};

// Q8_0 with K % 64 == 32 (GGUF's Q8_0 rows are any whole number of blocks):
// one 34-byte block per unit. A row of an odd block count is 2 bytes off a
// dword boundary every other row, so the block is read with dword-aligned
// loads and realigned (byte shift sh = 0 or 2).
struct FmtQ80s {
    static constexpr int EPU = 32, RAW = 10, QK = 32, BPB = 34;
    ZH_DEVM static void load_x(XReg &xr, XQView v, int u) {
        load_limbs(xr.L, v.limb + (size_t)u * 96, 24);
        xr.xs[0] = v.xs[u];
    }
    ZH_DEVM static void load_raw(const uint8_t *row, int u, uint32_t *raw) {
        const uint8_t *b = row + (size_t)u * 34;
        const uint32_t sh = (uint32_t)((uintptr_t)b & 3);
        const uint8_t *a = b - sh;
        const u32x4 t0 = *(const u32x4_a4 *)a, t1 = *(const u32x4_a4 *)(a + 16);
        raw[0] = t0.x; raw[1] = t0.y; raw[2] = t0.z; raw[3] = t0.w;
        raw[4] = t1.x; raw[5] = t1.y; raw[6] = t1.z; raw[7] = t1.w;
        raw[8] = *(const uint32_t *)(a + 32);
        raw[9] = sh;
    }
    ZH_DEVM static float compute(const uint32_t *raw, const XReg &xr, int u) {
        const uint32_t sh = raw[9];
        int D[3] = {0, 0, 0};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // quant dword i = block bytes 2 + 4i .. : stream offset sh + 2 + 4i
            const uint32_t q = sh ? raw[i + 1] : __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], 2);
#pragma unroll
            for (int k = 0; k < 3; k++) D[k] = sdot4(q, xr.L[k * 8 + i], D[k]);
        }
        const float d = h2f(sh ? raw[0] >> 16 : raw[0]);
        return d * xr.xs[0] * comb_f32(D[0], D[1], D[2]);
    }
};

// ---------------------------------------------------------------------------
// MXFP4: 17-byte blocks {e8m0 e, 16 B of E2M1 codes}; low nibble -> element j,
// high -> j+16 (forward.zig:441-459). Unit = one block (32 elements).
// 2*value is an int8 in {0,+-1,2,3,4,6,8,12}: looked up 4 at a time with
// v_perm_b32 and dotted against the limbs; the scale is 2^(e-127)/2.
// ---------------------------------------------------------------------------
struct FmtMXFP4 {
    static constexpr int EPU = 32, RAW = 6, QK = 32, BPB = 17;
    ZH_DEVM static void load_x(XReg &xr, XQView v, int u) {
        load_limbs(xr.L, v.limb + (size_t)u * 96, 24);
        xr.xs[0] = v.xs[u];
    }
    ZH_DEVM static void load_raw(const uint8_t *row, int u, uint32_t *raw) {
        const uint8_t *b = row + (size_t)u * 17;
        const uint32_t sh = (uint32_t)((uintptr_t)b & 3);
        const uint8_t *a = b - sh;  // (pointer arithmetic keeps an LDS pointer an LDS pointer)
        u32x4 t = *(const u32x4_a4 *)a;  // dword-aligned (also read from LDS tiles)
        raw[0] = t.x; raw[1] = t.y; raw[2] = t.z; raw[3] = t.w;
        raw[4] = *(const uint32_t *)(a + 16);
        raw[5] = sh;
    }
    ZH_DEVM static uint32_t e2m1x2(uint32_t nib) {
        uint32_t sel = nib & 0x07070707u;
        uint32_t pos = __builtin_amdgcn_perm(0x0C080604u, 0x03020100u, sel);
        uint32_t neg = __builtin_amdgcn_perm(0xF4F8FAFCu, 0xFDFEFF00u, sel);
        uint32_t sm = (nib >> 3) & 0x01010101u;
        uint32_t mask = (sm << 8) - sm;
        return (neg & mask) | (pos & ~mask);
    }
    ZH_DEVM static float compute(const uint32_t *raw, const XReg &xr, int u) {
        uint32_t sh = raw[5];
        uint32_t w[5];
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], sh);
        w[4] = __builtin_amdgcn_alignbyte(0u, raw[4], sh);  // byte 16 of the block in bits 0..7
        uint32_t e = w[0] & 0xFF;
        int D[3] = {0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t c = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 1);  // code bytes 1+4i..4+4i
            uint32_t lo = e2m1x2(c & 0x0F0F0F0Fu), hi = e2m1x2((c >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int k = 0; k < 3; k++) {
                D[k] = sdot4(lo, xr.L[k * 8 + i], D[k]);
                D[k] = sdot4(hi, xr.L[k * 8 + 4 + i], D[k]);
            }
        }
        float d = __uint_as_float(e == 0 ? 0x00400000u : (e << 23));
        return d * (0.5f * xr.xs[0]) * (float)comb_int(D[0], D[1], D[2]);
    }
};

#include "zh_fring.inc"

// ---------------------------------------------------------------------------
// Team kernel.
// ---------------------------------------------------------------------------
struct DmmvP {
    const uint8_t *W, *W2;  // W2: up matrix for the fused gate/up/SwiGLU mode
    const uint8_t *xq;
    float *y;
    uint32_t M, K;
    uint64_t row_bytes;
    uint32_t acc;
    const uint32_t *routing;  // MoE: expert id per grid.y slot
    uint32_t n_experts;       // MoE: ids are clamped below this (a NaN router yields id ~0)
    uint32_t *err;            // MoE, optional: ZH_DEVERR_EXPERT_ID when an id was clamped
    uint64_t expert_stride, xq_slot_stride;
    uint32_t y_slot_stride;
    // Plain mode may stack up to three matrices that share K and x (Q/K/V):
    // rows [seg_end[s-1], seg_end[s]) come from segW[s] and go to segY[s].
    // Segment sizes are multiples of the row batch R.
    uint32_t nseg;
    const uint8_t *segW[3];
    float *segY[3];
    uint32_t seg_end[3];
    float *ycopy;  // plain mode, one matrix: the outputs also stored here
};

enum { MODE_PLAIN = 0, MODE_GATE_UP = 1 };
static int dmmv_rows_per_batch(int mode);

ZH_DEV float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

// Joint reduction of V per-lane partials (V a power of two) across a team of
// TL lanes: log2(V) halving-exchange steps, then plain xor steps. Returns
// the team sum of partial `owner_index(lane)`; every lane of the team gets a
// valid result for its index.
template <int TL, int V>
ZH_DEV float team_reduce_multi(float (&a)[V], int tlane) {
    int n = V;
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
        n >>= 1;
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

template <class F, int TL, int NW, int R, int MODE, bool MOE>
__global__ __launch_bounds__(NW == 1 ? 256 : NW * 64) void k_dmmv(DmmvP p) {
    constexpr int TPW = (NW == 1) ? 256 / TL : 1;  // teams per workgroup
    constexpr int NM = (MODE == MODE_GATE_UP) ? 2 : 1;
    constexpr int V = NM * R;
    constexpr bool UNIFORM = (NW > 1) || (TL == 64);  // one team per wave or wider
    const int tid = threadIdx.x;
    const int tlane = (NW == 1) ? (tid % TL) : tid;
    const int team_in_wg = (NW == 1) ? (tid / TL) : 0;
    const uint32_t U = p.K / F::EPU;
    const bool active = (uint32_t)tlane < U;

    const uint8_t *Wm[2] = {p.W, p.W2};
    const uint8_t *xqb = p.xq;
    float *y = p.y;
    if (MOE) {
        const uint32_t slot = blockIdx.y;
        const uint32_t id = p.routing[slot];
        if (p.err && id >= p.n_experts && blockIdx.x == 0 && threadIdx.x == 0) atomicOr(p.err, ZH_DEVERR_EXPERT_ID);
        const uint64_t e = min(id, p.n_experts - 1);
        Wm[0] += e * p.expert_stride;
        if (NM == 2) Wm[1] += e * p.expert_stride;
        xqb += slot * p.xq_slot_stride;
        y += (size_t)slot * p.y_slot_stride;
    }
    XQView v = xq_view((void *)xqb, p.K / 32);
    XReg xr;
    if (active) F::load_x(xr, v, tlane);

    __shared__ float red[NW > 1 ? NW * V : 1];
    const uint32_t nteams = gridDim.x * TPW;
    uint32_t r0 = (blockIdx.x * TPW + team_in_wg) * R;
    if (UNIFORM) r0 = __builtin_amdgcn_readfirstlane(r0);
    for (; r0 < p.M; r0 += nteams * R) {
        uint32_t raw[NM][R][F::RAW];
        // segment of this batch (batches never straddle segments)
        uint32_t seg_start = 0, seg_rows = p.M;
        const uint8_t *Wb[2] = {Wm[0], Wm[1]};
        float *yb = y;
        if (!MOE && MODE == MODE_PLAIN && p.nseg > 1) {
            const uint32_t sg = (r0 >= p.seg_end[0] ? 1u : 0u) + (p.nseg > 2 && r0 >= p.seg_end[1] ? 1u : 0u);
            seg_start = sg ? p.seg_end[sg - 1] : 0u;
            seg_rows = p.seg_end[sg] - seg_start;
            Wb[0] = p.segW[sg];
            yb = p.segY[sg];
        }
        const uint32_t rr0 = r0 - seg_start;
        // rows past the segment end are clamped to its last row (loaded, computed, not written)
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t row = min(rr0 + r, seg_rows - 1);
                if (active) F::load_raw(Wb[m] + (size_t)row * p.row_bytes, tlane, raw[m][r]);
            }
        float part[V];
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < R; r++) {
            part[m * R + r] = active ? F::compute(raw[m][r], xr, tlane) : 0.f;
        }
        float res;
        int idx;
        if (NW == 1) {
            res = team_reduce_multi<TL, V>(part, tlane);
            idx = owner_index<TL, V>(tlane);
        } else {
            const int wave = tid >> 6, lane = tid & 63;
            float s = team_reduce_multi<64, V>(part, lane);
            int wi = owner_index<64, V>(lane);
            if ((lane & (64 / V - 1)) == 0) red[wi * NW + wave] = s;
            __syncthreads();
            idx = tid;
            res = 0.f;
            if (tid < V) {
#pragma unroll
                for (int w = 0; w < NW; w++) res += red[tid * NW + w];
            }
            __syncthreads();
        }
        // idx = m*R + r. The team sum of index i sits on team lane i*(TL/V)
        // (NW > 1: on thread i). In gate/up mode the up value of row r is
        // index R + r.
        constexpr int STRIDE = (NW == 1) ? (TL / V) : 1;
        const bool writer = (NW == 1) ? ((tlane % STRIDE) == 0) : (tid < V);
        if (MODE == MODE_GATE_UP) {
            const int lane = tid & 63;
            const float upv = __shfl(res, (lane + R * STRIDE) & 63, 64);
            if (writer && idx < R && rr0 + idx < seg_rows) yb[rr0 + idx] = silu_mul(res, upv);
        } else {
            if (writer && rr0 + idx < seg_rows) {
                float out = res;
                if (p.acc) out += yb[rr0 + idx];
                yb[rr0 + idx] = out;
                if (p.ycopy) p.ycopy[rr0 + idx] = out;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Host dispatch.
// ---------------------------------------------------------------------------
template <class F, int TL, int NW, int R, int MODE, bool MOE>
static int launch_one(zh_ctx *c, const DmmvP &p, uint32_t n_slots) {
    constexpr int TPW = (NW == 1) ? 256 / TL : 1;
    constexpr int BS = (NW == 1) ? 256 : NW * 64;
    uint32_t teams = (p.M + R - 1) / R;
    uint32_t wgs = (teams + TPW - 1) / TPW;
    const int capm = zh_knob_int("ZH_DMMV_CAP", 0);
    uint32_t cap = capm > 0 ? (uint32_t)c->cu_count * (uint32_t)capm
                            : (uint32_t)c->cu_count * (NW == 1 ? 8u : 16u / NW + 1u);
    if (MOE) cap = (cap + n_slots - 1) / n_slots;
    if (wgs > cap) wgs = cap;
    if (wgs == 0) wgs = 1;
    hipLaunchKernelGGL((k_dmmv<F, TL, NW, R, MODE, MOE>), dim3(wgs, MOE ? n_slots : 1), dim3(BS), 0,
                       c->stream, p);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

template <class F, int R, int MODE, bool MOE>
static int launch_fmt_r(zh_ctx *c, const DmmvP &p, uint32_t n_slots) {
    uint32_t U = p.K / F::EPU;
    if (U <= 8) return launch_one<F, 8, 1, R, MODE, MOE>(c, p, n_slots);
    if (U <= 16) return launch_one<F, 16, 1, R, MODE, MOE>(c, p, n_slots);
    if (U <= 32) return launch_one<F, 32, 1, R, MODE, MOE>(c, p, n_slots);
    if (U <= 64) return launch_one<F, 64, 1, R, MODE, MOE>(c, p, n_slots);
    if (U <= 128) return launch_one<F, 64, 2, R, MODE, MOE>(c, p, n_slots);
    if (U <= 192) return launch_one<F, 64, 3, R, MODE, MOE>(c, p, n_slots);
    if (U <= 256) return launch_one<F, 64, 4, R, MODE, MOE>(c, p, n_slots);
    if (U <= 512) return launch_one<F, 64, 8, R, MODE, MOE>(c, p, n_slots);
    return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "K=%u too large", p.K);
}

static int dmmv_rows_per_batch(int mode) {
    const int env = zh_knob_int("ZH_DMMV_R", 0);
    if (env == 2 || env == 4) return env;
    return mode == MODE_GATE_UP ? 2 : 4;
}

template <class F, int MODE, bool MOE>
static int launch_fmt(zh_ctx *c, const DmmvP &p, uint32_t n_slots) {
    if (dmmv_rows_per_batch(MODE) == 2) return launch_fmt_r<F, 2, MODE, MOE>(c, p, n_slots);
    return launch_fmt_r<F, 4, MODE, MOE>(c, p, n_slots);
}

template <int MODE, bool MOE>
static int launch_dmmv(zh_ctx *c, uint32_t qtype, const DmmvP &p, uint32_t n_slots) {
    switch (qtype) {
    case ZH_Q4_K: return launch_fmt<FmtQ4K, MODE, MOE>(c, p, n_slots);
    case ZH_Q5_K: return launch_fmt<FmtQ5K, MODE, MOE>(c, p, n_slots);
    case ZH_Q6_K: return launch_fmt<FmtQ6K, MODE, MOE>(c, p, n_slots);
    case ZH_Q8_0:
        return p.K % 64 ? launch_fmt<FmtQ80s, MODE, MOE>(c, p, n_slots) : launch_fmt<FmtQ80, MODE, MOE>(c, p, n_slots);
    case ZH_MXFP4: return launch_fmt<FmtMXFP4, MODE, MOE>(c, p, n_slots);
    default: return zh_set_err(c, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "qtype %u has no DMMV kernel", qtype);
    }
}

static int check_k(zh_ctx *c, uint32_t qtype, uint32_t K) {
    switch (qtype) {
    case ZH_Q4_K: case ZH_Q5_K: case ZH_Q6_K:
        if (K % 256) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "K=%u not a multiple of 256", K);
        return ZH_OK;
    case ZH_Q8_0:
        if (K % 32) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "K=%u not a multiple of 32", K);
        return ZH_OK;
    case ZH_MXFP4:
        if (K % 32) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "K=%u not a multiple of 32", K);
        return ZH_OK;
    default: return zh_set_err(c, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "qtype %u has no DMMV kernel", qtype);
    }
}

static int try_ftile(zh_ctx *c, uint32_t qtype, const uint8_t *W, const void *xq, const float *xf, float *y,
                     uint32_t M, uint32_t K, uint32_t acc);

int zhk_dmmv(zh_ctx *c, uint32_t qtype, const uint8_t *W, const void *xq, float *y, uint32_t M,
             uint32_t K, uint32_t acc, float *ycopy) {
    if (ycopy) {  // the team kernel writes the copy
        DmmvP p = {};
        p.W = W; p.W2 = W; p.xq = (const uint8_t *)xq; p.y = y; p.M = M; p.K = K;
        p.row_bytes = zh_tensor_bytes(qtype, 1, K); p.acc = acc; p.ycopy = ycopy;
        p.nseg = 1; p.segW[0] = W; p.segY[0] = y; p.seg_end[0] = M;
        return launch_dmmv<MODE_PLAIN, false>(c, qtype, p, 1);
    }
    if (qtype == ZH_MXFP4) {  // (Q8_0 on an XQ activation: the team kernel measured faster, 7.0 vs 8.5 us at 4096^2)
        const int rc = zhk_dmmv_fring(c, qtype, 1, &W, &y, &M, nullptr, nullptr, 0.f, xq, K, acc);
        if (rc >= 0) return rc;
    }
    const int rc = try_ftile(c, qtype, W, xq, nullptr, y, M, K, acc);
    if (rc >= 0) return rc;
    DmmvP p = {};
    p.W = W; p.W2 = W; p.xq = (const uint8_t *)xq; p.y = y; p.M = M; p.K = K;
    p.row_bytes = zh_tensor_bytes(qtype, 1, K); p.acc = acc;
    p.nseg = 1; p.segW[0] = W; p.segY[0] = y; p.seg_end[0] = M;
    return launch_dmmv<MODE_PLAIN, false>(c, qtype, p, 1);
}

int zhk_dmmv_multi(zh_ctx *c, uint32_t qtype, uint32_t nseg, const uint8_t *const *W, float *const *y,
                   const uint32_t *M, const void *xq, uint32_t K) {
    int R = dmmv_rows_per_batch(MODE_PLAIN);
    bool ok = nseg >= 1 && nseg <= 3;
    for (uint32_t s2 = 0; ok && s2 < nseg; s2++) ok = (M[s2] % (uint32_t)R) == 0 && M[s2] > 0;
    if (!ok) {  // fall back to one launch per matrix
        for (uint32_t s2 = 0; s2 < nseg; s2++) {
            int rc = zhk_dmmv(c, qtype, W[s2], xq, y[s2], M[s2], K, 0);
            if (rc) return rc;
        }
        return ZH_OK;
    }
    DmmvP p = {};
    p.W = W[0]; p.W2 = W[0]; p.xq = (const uint8_t *)xq; p.y = y[0]; p.K = K;
    p.row_bytes = zh_tensor_bytes(qtype, 1, K);
    p.nseg = nseg;
    uint32_t end = 0;
    for (uint32_t s2 = 0; s2 < nseg; s2++) {
        p.segW[s2] = W[s2]; p.segY[s2] = y[s2];
        end += M[s2];
        p.seg_end[s2] = end;
    }
    p.M = end;
    return launch_dmmv<MODE_PLAIN, false>(c, qtype, p, 1);
}

int zhk_dmmv_gate_up(zh_ctx *c, uint32_t qtype, const uint8_t *Wg, const uint8_t *Wu, const void *xq,
                     float *y, uint32_t M, uint32_t K) {
    DmmvP p = {};
    p.W = Wg; p.W2 = Wu; p.xq = (const uint8_t *)xq; p.y = y; p.M = M; p.K = K;
    p.row_bytes = zh_tensor_bytes(qtype, 1, K);
    return launch_dmmv<MODE_GATE_UP, false>(c, qtype, p, 1);
}

int zhk_dmmv_moe(zh_ctx *c, uint32_t qtype, const uint8_t *W, uint64_t expert_stride,
                 const uint32_t *routing, const void *xq, uint64_t xq_slot_stride, float *y, uint32_t M,
                 uint32_t K, uint32_t n_used, int gate_up, const uint8_t *W2, uint32_t n_experts, uint32_t *err) {
    if (n_experts == 0) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "n_experts");
    DmmvP p = {};
    p.n_experts = n_experts;
    p.err = err;
    p.W = W; p.W2 = W2 ? W2 : W; p.xq = (const uint8_t *)xq; p.y = y; p.M = M; p.K = K;
    p.row_bytes = zh_tensor_bytes(qtype, 1, K);
    p.routing = routing; p.expert_stride = expert_stride; p.xq_slot_stride = xq_slot_stride;
    p.y_slot_stride = M;
    if (gate_up) return launch_dmmv<MODE_GATE_UP, true>(c, qtype, p, n_used);
    return launch_dmmv<MODE_PLAIN, true>(c, qtype, p, n_used);
}

// ---------------------------------------------------------------------------
// LDS-staged team kernel (MoE decode path). The activation is staged once per
// workgroup into an LDS XQ image from f32 -- with the RMSNorm fused when a
// norm weight is given -- so the standalone rms_norm / quantise launches
// disappear; every lane then reads its unit's limbs from LDS.
//  * DL_PLAIN: y = W x (or y += W x) over up to three stacked matrices
//    (attn_norm fused into Q/K/V; ffn_norm fused into the router). Optional:
//    workgroup 0 stores the staged image as XQ for later kernels, and the
//    last workgroup to finish selects the router top-k (softmax_topk_v2.comp)
//    from the M outputs, published with device-scope stores and a counter.
//  * DL_DOWN_ACC: the expert down projections of all selected slots and the
//    routing-weighted sum, y[r] += sum_j w_j (W_{e_j} x_j)[r] in slot order
//    (dmmv down :6361-6408 + moe_weighted_acc.comp:23-33 in one launch), on
//    XQ inputs that every lane reads for its own unit (staging them per
//    workgroup re-quantised every slot in every workgroup and measured slower).
// ---------------------------------------------------------------------------
constexpr int DL_T = 256;
constexpr int DL_MAXS = 8;   // expert slots held in flight by DL_DOWN_ACC
enum { DL_PLAIN = 0, DL_DOWN_ACC = 1 };

struct DlP {
    uint32_t M, K;
    uint64_t row_bytes;
    const float *xf;       // DL_PLAIN: f32 activation
    const uint8_t *xq;     // DL_DOWN_ACC: XQ inputs, slot j at xq + j * 108 K/32
    const float *norm_w;   // DL_PLAIN: fused RMSNorm weight (nullptr: none)
    float eps;
    uint8_t *xq_out;       // DL_PLAIN: workgroup 0 stores the staged XQ image here
    uint32_t acc;          // DL_PLAIN: y += W x
    uint32_t nseg;         // DL_PLAIN: stacked matrices, rows [seg_end[s-1], seg_end[s]) -> segY[s]
    const uint8_t *segW[3];
    float *segY[3];
    uint32_t seg_end[3];
    const uint8_t *W;      // DL_DOWN_ACC: expert-stacked weights
    uint64_t expert_stride;
    const uint32_t *routing;  // [ids u32 x n_slots][weights f32 x n_slots]
    uint32_t n_slots;
    uint32_t n_experts;    // ids are clamped below this (a NaN router yields id ~0)
    float *y;
    uint32_t topk;         // DL_PLAIN router: k > 0 selects the top-k of the M outputs
    uint32_t *routing_out;
    uint32_t *cnt;         // zero between launches
};

// Stages the f32 activation of K (a multiple of 32, at most DL_XE * DL_T)
// elements, RMSNorm'ed with w when w != nullptr (w[i] * (x[i] * rms_inv),
// cpuRmsNormMul forward.zig:618-626), into an XQ image in LDS. Every element
// a thread owns is loaded before any arithmetic, so staging costs one memory
// latency; each 32-element block is quantised by the 32 lanes that own it (a
// 32-lane group covers 32 consecutive elements, so each half-wave is wholly
// active or inactive).
constexpr int DL_XE = 16;
ZH_DEV void dl_stage(const float *__restrict__ x, const float *__restrict__ w, float eps, uint32_t K, uint8_t *lds,
                     float *red) {
    const uint32_t t = threadIdx.x, nblk = K / 32;
    float xr[DL_XE], wr[DL_XE];
#pragma unroll
    for (int j = 0; j < DL_XE; j++) {
        const uint32_t i = t + DL_T * j;
        xr[j] = i < K ? x[i] : 0.f;
        wr[j] = i < K && w ? w[i] : 1.f;
    }
    float rms_inv = 1.f;
    if (w) {
        float sq = 0.f;
#pragma unroll
        for (int j = 0; j < DL_XE; j++) sq = fmaf(xr[j], xr[j], sq);
        sq = wave_sum(sq);
        if ((t & 63) == 0) red[t >> 6] = sq;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int k = 0; k < DL_T / 64; k++) tot += red[k];
        rms_inv = 1.0f / sqrtf(tot / (float)K + eps);
    }
    const XQView q = xq_view(lds, nblk);
#pragma unroll
    for (int j = 0; j < DL_XE; j++) {
        const uint32_t i = t + DL_T * j;
        if (DL_T * j >= K) break;  // uniform
        if (i < K) xq_store_block32(w ? wr[j] * (xr[j] * rms_inv) : xr[j], t & 31, q, i / 32);
    }
    __syncthreads();
}

template <class F, int TL, int R, int MODE>
__global__ __launch_bounds__(DL_T) void k_dmmv_lds(DlP p) {
    extern __shared__ __align__(16) uint8_t dl_lds[];
    __shared__ float red[DL_T / 64];
    constexpr int TPW = DL_T / TL;
    const int tid = threadIdx.x, tlane = tid % TL, team = tid / TL;
    const uint32_t U = p.K / F::EPU, nblk = p.K / 32;
    const bool active = (uint32_t)tlane < U;
    const uint32_t nteams = gridDim.x * TPW;
    if (MODE == DL_PLAIN) {
        // segment of a batch (batches never straddle segments); rows past a
        // segment are clamped to its last row (loaded, computed, not written)
        auto geom = [&](uint32_t r0, uint32_t &sg, uint32_t &rr0, uint32_t &seg_rows) {
            uint32_t seg_start = 0;
            sg = 0;
            seg_rows = p.M;
            if (p.nseg > 1) {
                sg = (r0 >= p.seg_end[0] ? 1u : 0u) + (p.nseg > 2 && r0 >= p.seg_end[1] ? 1u : 0u);
                seg_start = sg ? p.seg_end[sg - 1] : 0u;
                seg_rows = p.seg_end[sg] - seg_start;
            }
            rr0 = r0 - seg_start;
        };
        auto fetch = [&](uint32_t r0, uint32_t (&raw)[R][F::RAW]) {
            uint32_t sg, rr0, seg_rows;
            geom(min(r0, p.M - 1), sg, rr0, seg_rows);
#pragma unroll
            for (int r = 0; r < R; r++)
                if (active) F::load_raw(p.segW[sg] + (size_t)min(rr0 + r, seg_rows - 1) * p.row_bytes, tlane, raw[r]);
        };
        uint32_t r0 = (blockIdx.x * TPW + team) * R;
        uint32_t raw[R][F::RAW];
        fetch(r0, raw);  // the first batch's weights are in flight while x is staged
        dl_stage(p.xf, p.norm_w, p.eps, p.K, dl_lds, red);
        if (p.xq_out && blockIdx.x == 0)
            for (uint32_t i = tid; i < nblk * 27; i += DL_T)  // 108 B per block = 27 dwords
                ((uint32_t *)p.xq_out)[i] = ((const uint32_t *)dl_lds)[i];
        XReg xr;
        if (active) F::load_x(xr, xq_view(dl_lds, nblk), tlane);
        for (; r0 < p.M; r0 += nteams * R) {
            uint32_t sg, rr0, seg_rows;
            geom(r0, sg, rr0, seg_rows);
            if (r0 != (blockIdx.x * TPW + team) * R) fetch(r0, raw);
            float part[R];
#pragma unroll
            for (int r = 0; r < R; r++) part[r] = active ? F::compute(raw[r], xr, tlane) : 0.f;
            const float res = team_reduce_multi<TL, R>(part, tlane);
            const int idx = owner_index<TL, R>(tlane);
            if (tlane % (TL / R) == 0 && rr0 + idx < seg_rows) {
                float *yo = p.segY[sg] + rr0 + idx;
                const float out = p.acc ? res + *yo : res;
                if (p.topk) st_dev(yo, out);  // read by another workgroup below
                else *yo = out;
            }
        }
        if (p.topk) {
            __shared__ uint32_t s_last;
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (tid == 0)
                s_last = __hip_atomic_fetch_add(p.cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                         gridDim.x - 1;
            __syncthreads();
            if (s_last && tid < 64) {
                float vals[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t e = tid + 64 * i;
                    vals[i] = e < p.M ? ld_dev(p.segY[0] + e) : -INFINITY;
                }
                topk_softmax_wave(vals, p.M, p.topk, p.routing_out);
                if (tid == 0) __hip_atomic_store(p.cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    } else {
        // one row per team; every slot's weight unit is requested before any
        // arithmetic, then the slots are reduced and weighted in order
        uint32_t ex[DL_MAXS];
        float wgt[DL_MAXS];
#pragma unroll
        for (int j = 0; j < DL_MAXS; j++) {
            ex[j] = (uint32_t)j < p.n_slots ? min(p.routing[j], p.n_experts - 1) : 0u;
            wgt[j] = (uint32_t)j < p.n_slots ? __uint_as_float(p.routing[p.n_slots + j]) : 0.f;
        }
        uint32_t raw[DL_MAXS][F::RAW];
        auto fetch = [&](uint32_t r) {
#pragma unroll
            for (int j = 0; j < DL_MAXS; j++)
                if (active && (uint32_t)j < p.n_slots)
                    F::load_raw(p.W + ex[j] * p.expert_stride + (size_t)min(r, p.M - 1) * p.row_bytes, tlane, raw[j]);
        };
        const uint32_t r_first = blockIdx.x * TPW + team;
        fetch(r_first);
        for (uint32_t r = r_first; r < p.M; r += nteams) {
            if (r != r_first) fetch(r);
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < DL_MAXS; j++) {
                if ((uint32_t)j >= p.n_slots) break;  // uniform
                XReg xr;
                if (active) F::load_x(xr, xq_view((uint8_t *)p.xq + (size_t)j * nblk * 108, nblk), tlane);
                const float dot = team_sum_dpp<TL>(active ? F::compute(raw[j], xr, tlane) : 0.f);
                s += wgt[j] * dot;
            }
            if (tlane == 0) p.y[r] += s;
        }
    }
}

template <class F, int MODE>
static int launch_dl(zh_ctx *c, const DlP &p) {
    const uint32_t U = p.K / F::EPU;
    const uint32_t lds = MODE == DL_DOWN_ACC ? 0u : (p.K / 32) * 108;
    constexpr int R = MODE == DL_PLAIN ? 2 : 1;
    const uint32_t tl = U <= 16 ? 16 : U <= 32 ? 32 : 64;
    if (U > 64 || p.K > (uint32_t)(DL_XE * DL_T))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "LDS-staged DMMV: K=%u too large", p.K);
    const uint32_t teams = (p.M + R - 1) / R, tpw = DL_T / tl;
    uint32_t wgs = (teams + tpw - 1) / tpw, cap = (uint32_t)c->cu_count * 4u;
    if (wgs > cap) wgs = cap;
#define DL_L(TT) hipLaunchKernelGGL((k_dmmv_lds<F, TT, R, MODE>), dim3(wgs), dim3(DL_T), lds, c->stream, p)
    if (tl == 16) DL_L(16);
    else if (tl == 32) DL_L(32);
    else DL_L(64);
#undef DL_L
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

template <int MODE>
static int launch_dl_q(zh_ctx *c, uint32_t qtype, const DlP &p) {
    switch (qtype) {
    case ZH_Q4_K: return launch_dl<FmtQ4K, MODE>(c, p);
    case ZH_Q5_K: return launch_dl<FmtQ5K, MODE>(c, p);
    case ZH_Q6_K: return launch_dl<FmtQ6K, MODE>(c, p);
    case ZH_Q8_0: return launch_dl<FmtQ80, MODE>(c, p);
    case ZH_MXFP4: return launch_dl<FmtMXFP4, MODE>(c, p);
    default: return zh_set_err(c, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "qtype %u has no DMMV kernel", qtype);
    }
}

bool zhk_dmmv_lds_supported(uint32_t qtype, uint32_t K) {
    const uint32_t epu = qtype == ZH_MXFP4 ? 32 : 64;
    const uint32_t q = (qtype == ZH_Q4_K || qtype == ZH_Q5_K || qtype == ZH_Q6_K) ? 256 : epu;
    return K > 0 && K % q == 0 && K % 32 == 0 && K / epu <= 64;
}

int zhk_dmmv_lds_plain(zh_ctx *c, uint32_t qtype, uint32_t nseg, const uint8_t *const *W, float *const *y,
                       const uint32_t *M, const float *x, const float *norm_w, float eps, uint32_t K,
                       uint32_t acc, void *xq_out, uint32_t topk, uint32_t *routing_out, uint32_t *cnt) {
    if (nseg < 1 || nseg > 3 || !zhk_dmmv_lds_supported(qtype, K) || (topk && (nseg != 1 || M[0] > 256)))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "LDS-staged DMMV shape");
    if (!xq_out && !topk) {
        const int rc = zhk_dmmv_fring(c, qtype, nseg, W, y, M, x, norm_w, eps, nullptr, K, acc);
        if (rc >= 0) return rc;
    }
    DlP p = {};
    p.K = K; p.row_bytes = zh_tensor_bytes(qtype, 1, K); p.xf = x; p.norm_w = norm_w; p.eps = eps;
    p.xq_out = (uint8_t *)xq_out; p.acc = acc; p.nseg = nseg;
    uint32_t end = 0;
    for (uint32_t s = 0; s < nseg; s++) {
        if (s + 1 < nseg && M[s] % 2) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "segment rows must be even");
        p.segW[s] = W[s]; p.segY[s] = y[s];
        end += M[s];
        p.seg_end[s] = end;
    }
    p.M = end; p.topk = topk; p.routing_out = routing_out; p.cnt = cnt;
    return launch_dl_q<DL_PLAIN>(c, qtype, p);
}

int zhk_dmmv_lds_down_acc(zh_ctx *c, uint32_t qtype, const uint8_t *W, uint64_t expert_stride,
                          const uint32_t *routing, uint32_t n_slots, uint32_t n_experts, const void *xq, float *y,
                          uint32_t M, uint32_t K) {
    if (n_slots == 0 || n_slots > DL_MAXS || n_experts == 0 || !zhk_dmmv_lds_supported(qtype, K))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "expert down shape");
    DlP p = {};
    p.M = M; p.K = K; p.row_bytes = zh_tensor_bytes(qtype, 1, K);
    p.W = W; p.expert_stride = expert_stride; p.routing = routing; p.n_slots = n_slots; p.y = y;
    p.n_experts = n_experts; p.xq = (const uint8_t *)xq;
    return launch_dl_q<DL_DOWN_ACC>(c, qtype, p);
}

// ---------------------------------------------------------------------------
// Coalesced-tile kernel for a format of the team kernel (used for MXFP4):
// the activation is staged once per workgroup as an XQ image in LDS (copied,
// or quantised from f32), each batch of rows -- a contiguous byte range -- is
// fetched with consecutive lanes on consecutive 16-byte chunks (one batch
// ahead) into an LDS tile, and each row is reduced by one wave whose lanes
// walk the row's units, reading limbs and weight bytes from LDS. Batches hold
// RPB = 4, 8 or 16 rows so that a batch is a whole number of 16-byte chunks.
// ---------------------------------------------------------------------------
constexpr int FT_NCH = 8;  // 16-byte chunks per lane per batch (tile <= 32 KB)
struct FtP {
    const uint8_t *W;
    uint32_t M, K, rpb;
    uint64_t row_bytes;
    const uint8_t *xq;  // XQ activation, or
    const float *xf;    // f32 activation (quantised while staging)
    float *y;
    uint32_t acc;
};

template <class F>
__global__ __launch_bounds__(256, 2) void k_dmmv_ftile(FtP p) {
    extern __shared__ __align__(16) uint8_t ft_lds[];
    __shared__ float red[4];
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t nblk = p.K / 32, U = p.K / F::EPU;
    uint8_t *tile = ft_lds + ((size_t)nblk * 108 + 15) / 16 * 16;
    const uint32_t nbatch = (p.M + p.rpb - 1) / p.rpb;
    const uint32_t batch_bytes = p.rpb * (uint32_t)p.row_bytes;
    u32x4 st[FT_NCH];
    auto fetch = [&](uint32_t bi) {
        const uint32_t nr = min(p.rpb, p.M - bi * p.rpb), n16 = (nr * (uint32_t)p.row_bytes + 15) / 16;
        const u32x4 *src = (const u32x4 *)(p.W + (size_t)bi * batch_bytes);
#pragma unroll
        for (int j = 0; j < FT_NCH; j++) st[j] = src[min(j * 256 + tid, n16 - 1)];  // clamped: static count
    };
    uint32_t bi = blockIdx.x;  // grid <= nbatch (host)
    fetch(bi);
    // activation -> LDS XQ image
    if (p.xq) {
        for (uint32_t i = tid; i < nblk * 27; i += 256) ((uint32_t *)ft_lds)[i] = ((const uint32_t *)p.xq)[i];
        __syncthreads();
    } else {
        dl_stage(p.xf, nullptr, 0.f, p.K, ft_lds, red);
    }
    const XQView xv = xq_view(ft_lds, nblk);
    for (; bi < nbatch; bi += gridDim.x) {
        const uint32_t nr = min(p.rpb, p.M - bi * p.rpb), n16 = (nr * (uint32_t)p.row_bytes + 15) / 16;
#pragma unroll
        for (int j = 0; j < FT_NCH; j++) {
            const uint32_t c = j * 256 + tid;
            if (c < n16) *(u32x4 *)(tile + c * 16) = st[j];
        }
        __syncthreads();
        if (bi + gridDim.x < nbatch) fetch(bi + gridDim.x);
        for (uint32_t r = wave; r < p.rpb; r += 4) {  // uniform per wave
            const uint8_t *row = tile + (size_t)r * p.row_bytes;
            float part = 0.f;
            for (uint32_t u = lane; u < U; u += 64) {
                XReg xr;
                uint32_t raw[F::RAW];
                F::load_x(xr, xv, u);
                F::load_raw(row, u, raw);
                part += F::compute(raw, xr, u);
            }
            part = wave_sum(part);
            if (lane == 0 && r < nr) {
                float *yo = p.y + (size_t)bi * p.rpb + r;
                *yo = p.acc ? *yo + part : part;
            }
        }
        __syncthreads();  // the tile is rewritten by the next batch
    }
}

// Launches the tile kernel when it applies; returns -1 to use the team kernel.
static int try_ftile(zh_ctx *c, uint32_t qtype, const uint8_t *W, const void *xq, const float *xf, float *y,
                     uint32_t M, uint32_t K, uint32_t acc) {
    static int off = -1;
    if (off < 0) off = zh_knob("ZH_NO_FTILE")? 1 : 0;
    // MXFP4 only: for Q8_0 the team kernel (x in registers, four rows per
    // team in flight) measured faster than 4-row tiles
    if (off || qtype != ZH_MXFP4 || ((uintptr_t)W & 15)) return -1;
    if (!xq && K > (uint32_t)(DL_XE * DL_T)) return -1;  // f32 staging holds K <= 4096
    const uint64_t rb = zh_tensor_bytes(qtype, 1, K);
    uint32_t rpb = 4;
    while ((rpb * rb) % 16) rpb *= 2;  // 4, 8 or 16 rows
    // whole batches only: every 16-byte chunk lies inside the matrix
    if (M % rpb) return -1;
    if (rpb * rb > (uint64_t)FT_NCH * 256 * 16) return -1;
    const uint32_t lds = ((K / 32) * 108 + 15) / 16 * 16 + (uint32_t)(rpb * rb);
    if (lds > 65536) return -1;
    FtP p = {};
    p.W = W; p.M = M; p.K = K; p.rpb = rpb; p.row_bytes = rb; p.xq = (const uint8_t *)xq; p.xf = xf; p.y = y;
    p.acc = acc;
    const uint32_t nbatch = (M + rpb - 1) / rpb;
    uint32_t wgs = nbatch, cap = (uint32_t)c->cu_count * 2;
    if (wgs > cap) wgs = cap;
    hipLaunchKernelGGL(k_dmmv_ftile<FmtMXFP4>, dim3(wgs), dim3(256), lds, c->stream, p);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

// ---------------------------------------------------------------------------
// C ABI wrappers with argument validation (shapes are checked on the host
// before any launch so a kernel never sees a shape it does not assume).
// ---------------------------------------------------------------------------
static bool in_range(const zh_buf *b, uint64_t off, uint64_t n) { return b && off <= b->size && n <= b->size - off; }

extern "C" int zh_dmmv_supported(uint32_t qtype, uint32_t K) {
    // the team kernel covers up to 512 units of a row (64 elements per unit
    // for the K-quants and K % 64 == 0 Q8_0, 32 for MXFP4 and odd-block Q8_0)
    switch (qtype) {
    case ZH_Q4_K: case ZH_Q5_K: case ZH_Q6_K: return K > 0 && K % 256 == 0 && K / 64 <= 512 ? 1 : 0;
    case ZH_Q8_0: return K > 0 && K % 32 == 0 && K / (K % 64 ? 32 : 64) <= 512 ? 1 : 0;
    case ZH_MXFP4: return K > 0 && K % 32 == 0 && K / 32 <= 512 ? 1 : 0;
    default: return 0;
    }
}

extern "C" int zh_dmmv(zh_ctx *c, uint32_t qtype, const zh_buf *W, uint64_t a_off, const zh_buf *x,
                       uint64_t x_off, zh_buf *y, uint64_t y_off, uint32_t M, uint32_t K, uint32_t acc_mode) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    int rc = check_k(c, qtype, K);
    if (rc) return rc;
    if (M == 0 || K == 0) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "empty shape");
    if (acc_mode > 1) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "acc_mode %u", acc_mode);
    if (!in_range(W, a_off, zh_tensor_bytes(qtype, M, K)) || !in_range(x, x_off, (uint64_t)K * 4) ||
        !in_range(y, y_off, (uint64_t)M * 4))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "buffer too small for M=%u K=%u", M, K);
    if ((a_off & 3) || (x_off & 3) || (y_off & 3))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "offsets must be 4-byte aligned");
    if (qtype == ZH_Q4_K && (a_off & 15)) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "Q4_K a_off must be 16-byte aligned");
    if (zhk_lpb_supported(qtype, K) && (x_off & 15) == 0 && !zh_knob("ZH_NO_LPB")) {
        const uint8_t *w = (const uint8_t *)W->ptr + a_off;
        float *yy = (float *)((char *)y->ptr + y_off);
        int R = 2;
        if (M % R == 0)
            return zhk_dmmv_lpb(c, qtype, 0, 1, &w, nullptr, &yy, &M, (const float *)((const char *)x->ptr + x_off),
                                nullptr, 0.f, nullptr, K, acc_mode);
    }
    if ((x_off & 15) == 0) {  // f32 staged and quantised per workgroup
        const uint8_t *w = (const uint8_t *)W->ptr + a_off;
        float *yy = (float *)((char *)y->ptr + y_off);
        rc = zhk_dmmv_fring(c, qtype, 1, &w, &yy, &M, (const float *)((const char *)x->ptr + x_off), nullptr, 0.f,
                            nullptr, K, acc_mode);
        if (rc >= 0) return rc;
        rc = try_ftile(c, qtype, (const uint8_t *)W->ptr + a_off, nullptr, (const float *)((const char *)x->ptr + x_off),
                       (float *)((char *)y->ptr + y_off), M, K, acc_mode);
        if (rc >= 0) return rc;
    }
    void *xq;
    if ((rc = zh_scratch(c, zh_xq_bytes_int(K), &xq))) return rc;
    if ((rc = zhk_quantize_xq(c, (const float *)((const char *)x->ptr + x_off), xq, K, 1, 0))) return rc;
    return zhk_dmmv(c, qtype, (const uint8_t *)W->ptr + a_off, xq, (float *)((char *)y->ptr + y_off), M, K, acc_mode);
}

extern "C" uint64_t zh_xq_bytes(uint32_t K) { return zh_xq_bytes_int(K); }

extern "C" int zh_quantize_activation(zh_ctx *c, const zh_buf *x, uint64_t x_off, uint32_t K, uint32_t n_vec,
                                      uint32_t x_stride, zh_buf *xq, uint64_t xq_off) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (K == 0 || K % 32 || n_vec == 0 || (n_vec > 1 && x_stride < K) || (x_off & 3) || (xq_off & 15))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "quantize_activation shape");
    if (!in_range(x, x_off, 4ull * ((uint64_t)(n_vec - 1) * x_stride + K)) ||
        !in_range(xq, xq_off, zh_xq_bytes_int(K) * n_vec))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "quantize_activation range");
    return zhk_quantize_xq(c, (const float *)((const char *)x->ptr + x_off), (char *)xq->ptr + xq_off, K, n_vec,
                           x_stride);
}

extern "C" int zh_dmmv_xq(zh_ctx *c, uint32_t qtype, const zh_buf *W, uint64_t a_off, const zh_buf *xq,
                          uint64_t xq_off, zh_buf *y, uint64_t y_off, uint32_t M, uint32_t K, uint32_t acc_mode) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    int rc = check_k(c, qtype, K);
    if (rc) return rc;
    if (M == 0 || acc_mode > 1) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "shape");
    if (!in_range(W, a_off, zh_tensor_bytes(qtype, M, K)) || !in_range(xq, xq_off, zh_xq_bytes_int(K)) ||
        !in_range(y, y_off, 4ull * M) || (a_off & (qtype == ZH_Q4_K ? 15 : 3)) || (xq_off & 15) || (y_off & 3))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "range/alignment");
    if (zhk_lpb_supported(qtype, K) && !zh_knob("ZH_NO_LPB")) {
        const uint8_t *w = (const uint8_t *)W->ptr + a_off;
        float *yy = (float *)((char *)y->ptr + y_off);
        return zhk_dmmv_lpb(c, qtype, 0, 1, &w, nullptr, &yy, &M, nullptr, nullptr, 0.f, nullptr, K, acc_mode,
                            (const char *)xq->ptr + xq_off);
    }
    return zhk_dmmv(c, qtype, (const uint8_t *)W->ptr + a_off, (const char *)xq->ptr + xq_off,
                    (float *)((char *)y->ptr + y_off), M, K, acc_mode);
}

extern "C" int zh_dmmv_fused_gate_up_swiglu_xq(zh_ctx *c, uint32_t qtype, const zh_buf *Wg, uint64_t g_off,
                                               const zh_buf *Wu, uint64_t u_off, const zh_buf *xq, uint64_t xq_off,
                                               zh_buf *y, uint64_t y_off, uint32_t M, uint32_t K) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    int rc = check_k(c, qtype, K);
    if (rc) return rc;
    uint64_t wb = zh_tensor_bytes(qtype, M, K);
    if (M == 0 || !in_range(Wg, g_off, wb) || !in_range(Wu, u_off, wb) || !in_range(xq, xq_off, zh_xq_bytes_int(K)) ||
        !in_range(y, y_off, 4ull * M) || (g_off & 15) || (u_off & 15) || (xq_off & 15) || (y_off & 3))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "range/alignment");
    if (qtype == ZH_Q4_K && zhk_lpb_supported(qtype, K) && !zh_knob("ZH_NO_LPB")) {
        const uint8_t *wg = (const uint8_t *)Wg->ptr + g_off;
        float *yy = (float *)((char *)y->ptr + y_off);
        return zhk_dmmv_lpb(c, qtype, 1, 1, &wg, (const uint8_t *)Wu->ptr + u_off, &yy, &M, nullptr, nullptr, 0.f,
                            nullptr, K, 0, (const char *)xq->ptr + xq_off);
    }
    return zhk_dmmv_gate_up(c, qtype, (const uint8_t *)Wg->ptr + g_off, (const uint8_t *)Wu->ptr + u_off,
                            (const char *)xq->ptr + xq_off, (float *)((char *)y->ptr + y_off), M, K);
}

extern "C" int zh_dmmv_fused_gate_up_swiglu(zh_ctx *c, uint32_t qtype, const zh_buf *Wg, uint64_t g_off,
                                            const zh_buf *Wu, uint64_t u_off, const zh_buf *x, uint64_t x_off,
                                            zh_buf *y, uint64_t y_off, uint32_t M, uint32_t K) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    int rc = check_k(c, qtype, K);
    if (rc) return rc;
    uint64_t wb = zh_tensor_bytes(qtype, M, K);
    if (M == 0 || !in_range(Wg, g_off, wb) || !in_range(Wu, u_off, wb) || !in_range(x, x_off, (uint64_t)K * 4) ||
        !in_range(y, y_off, (uint64_t)M * 4))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "buffer too small for M=%u K=%u", M, K);
    if ((g_off & 15) || (u_off & 15) || (x_off & 3) || (y_off & 3))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "misaligned offsets");
    if (qtype == ZH_Q4_K && zhk_lpb_supported(qtype, K) && (x_off & 15) == 0 && !zh_knob("ZH_NO_LPB")) {
        const uint8_t *wg = (const uint8_t *)Wg->ptr + g_off;
        float *yy = (float *)((char *)y->ptr + y_off);
        return zhk_dmmv_lpb(c, qtype, 1, 1, &wg, (const uint8_t *)Wu->ptr + u_off, &yy, &M,
                            (const float *)((const char *)x->ptr + x_off), nullptr, 0.f, nullptr, K, 0);
    }
    void *xq;
    if ((rc = zh_scratch(c, zh_xq_bytes_int(K), &xq))) return rc;
    if ((rc = zhk_quantize_xq(c, (const float *)((const char *)x->ptr + x_off), xq, K, 1, 0))) return rc;
    return zhk_dmmv_gate_up(c, qtype, (const uint8_t *)Wg->ptr + g_off, (const uint8_t *)Wu->ptr + u_off, xq,
                            (float *)((char *)y->ptr + y_off), M, K);
}

extern "C" int zh_dmmv_moe(zh_ctx *c, uint32_t qtype, const zh_buf *W, uint64_t expert_stride,
                           const zh_buf *routing, const zh_buf *x, uint32_t x_expert_stride, uint64_t x_off,
                           zh_buf *y, uint64_t y_off, uint32_t M, uint32_t K, uint32_t n_used) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    int rc = check_k(c, qtype, K);
    if (rc) return rc;
    if (n_used == 0 || n_used > 64 || M == 0) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "n_used/M");
    if (!routing || routing->size < (uint64_t)n_used * 4) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "routing");
    if (expert_stride < zh_tensor_bytes(qtype, M, K) || (expert_stride & 15))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "expert_stride");
    if (!in_range(x, x_off, ((uint64_t)(n_used - 1) * x_expert_stride + K) * 4) ||
        !in_range(y, y_off, (uint64_t)n_used * M * 4) || (x_off & 3) || (y_off & 3))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "x/y range");
    if (!in_range(W, 0, zh_tensor_bytes(qtype, M, K))) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "W range");
    // Expert ids stay on the device: the kernel clamps each to the experts
    // the weight buffer holds and flags a clamped id in the context's error
    // word, which zh_sync reports (the call itself only enqueues).
    void *xq;
    uint64_t xqs = zh_xq_bytes_int(K);
    if ((rc = zh_scratch(c, xqs * n_used, &xq))) return rc;
    if ((rc = zhk_quantize_xq(c, (const float *)((const char *)x->ptr + x_off), xq, K, n_used, x_expert_stride)))
        return rc;
    return zhk_dmmv_moe(c, qtype, (const uint8_t *)W->ptr, expert_stride, (const uint32_t *)routing->ptr, xq, xqs,
                        (float *)((char *)y->ptr + y_off), M, K, n_used, 0, nullptr,
                        (uint32_t)((W->size - zh_tensor_bytes(qtype, M, K)) / expert_stride + 1), c->err_dev);
}

// ---------------------------------------------------------------------------
// Bit-exact dequantisation (dequantRow, forward.zig:242-465): one thread per
// output element, every product and difference rounded separately (_rn
// intrinsics), matching Zig's unfused f32 arithmetic.
// ---------------------------------------------------------------------------
ZH_DEV uint32_t blk_elems(uint32_t t) { return (t == ZH_Q4_K || t == ZH_Q5_K || t == ZH_Q6_K) ? 256 : (t == ZH_Q8_0 || t == ZH_MXFP4) ? 32 : 1; }
ZH_DEV uint32_t blk_bytes(uint32_t t) {
    return t == ZH_Q4_K ? 144 : t == ZH_Q5_K ? 176 : t == ZH_Q6_K ? 210 : t == ZH_Q8_0 ? 34 : t == ZH_MXFP4 ? 17 : t == ZH_F16 ? 2 : 4;
}

__global__ void k_dequant(uint32_t qtype, const uint8_t *__restrict__ W, uint32_t row0, uint32_t n_rows,
                          uint32_t K, float *__restrict__ out, const uint32_t *row_from_dev, uint32_t clamp_rows,
                          uint32_t gather) {
    uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t rr = blockIdx.y;
    if (e >= K || rr >= n_rows) return;
    uint32_t row = row0 + rr;
    if (row_from_dev) {
        // one id and consecutive rows, or (gather) one id per output row
        row = gather ? row_from_dev[rr] : row_from_dev[0] + rr;
        if (row >= clamp_rows) row = clamp_rows - 1;  // embedToken safe_id clamp (forward.zig:4271)
    }
    uint64_t rb = (uint64_t)(K / blk_elems(qtype)) * blk_bytes(qtype);
    const uint8_t *r = W + (uint64_t)row * rb;
    float v = 0.f;
    switch (qtype) {
    case ZH_Q4_K: {
        const uint8_t *b = r + (e / 256) * 144;
        uint32_t w = e % 256, p = w / 64, hi = (w / 32) & 1, l = w % 32, j = 2 * p + hi;
        const uint8_t *s = b + 4;
        uint32_t sc, m;
        if (j < 4) { sc = s[j] & 63; m = s[j + 4] & 63; }
        else { sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4); m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4); }
        uint32_t q = (b[16 + 32 * p + l] >> (4 * hi)) & 0xF;
        float d = h2f(b[0] | (b[1] << 8)), dmin = h2f(b[2] | (b[3] << 8));
        v = __fsub_rn(__fmul_rn(__fmul_rn(d, (float)sc), (float)q), __fmul_rn(dmin, (float)m));
        break;
    }
    case ZH_Q5_K: {
        const uint8_t *b = r + (e / 256) * 176;
        uint32_t w = e % 256, p = w / 64, hi = (w / 32) & 1, l = w % 32, j = 2 * p + hi;
        const uint8_t *s = b + 4;
        uint32_t sc, m;
        if (j < 4) { sc = s[j] & 63; m = s[j + 4] & 63; }
        else { sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4); m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4); }
        uint32_t q = ((b[48 + 32 * p + l] >> (4 * hi)) & 0xF) | (((b[16 + l] >> j) & 1) << 4);
        float d = h2f(b[0] | (b[1] << 8)), dmin = h2f(b[2] | (b[3] << 8));
        v = __fsub_rn(__fmul_rn(__fmul_rn(d, (float)sc), (float)q), __fmul_rn(dmin, (float)m));
        break;
    }
    case ZH_Q6_K: {
        const uint8_t *b = r + (e / 256) * 210;
        uint32_t w = e % 256, h = w / 128, g = (w % 128) / 32, l = w % 32;
        uint32_t qlb = b[64 * h + l + 32 * (g & 1)];
        uint32_t lo = (g >> 1) ? (qlb >> 4) : (qlb & 0xF);
        uint32_t hb = (b[128 + 32 * h + l] >> (2 * g)) & 3;
        int q = (int)(lo | (hb << 4)) - 32;
        float sc = (float)(int8_t)b[192 + 8 * h + l / 16 + 2 * g];
        float d = h2f(b[208] | (b[209] << 8));
        v = __fmul_rn(__fmul_rn(d, sc), (float)q);
        break;
    }
    case ZH_Q8_0: {
        const uint8_t *b = r + (e / 32) * 34;
        v = __fmul_rn((float)(int8_t)b[2 + e % 32], h2f(b[0] | (b[1] << 8)));
        break;
    }
    case ZH_MXFP4: {
        const uint8_t *b = r + (e / 32) * 17;
        uint32_t j = e % 32, code = j < 16 ? (b[1 + j] & 0xF) : (b[1 + j - 16] >> 4);
        const float lut[16] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f, -0.f, -.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f};
        uint32_t ex = b[0];
        float d = __uint_as_float(ex == 0 ? 0x00400000u : (ex << 23));
        v = __fmul_rn(d, lut[code]);
        break;
    }
    case ZH_F16: v = h2f(((const uint16_t *)r)[e]); break;
    case ZH_F32: v = ((const float *)r)[e]; break;
    }
    out[(size_t)rr * K + e] = v;
}

int zhk_dequant_rows(zh_ctx *c, uint32_t qtype, const uint8_t *W, uint32_t row0, uint32_t n_rows, uint32_t K,
                     float *out, const uint32_t *row_from_dev, uint32_t clamp_rows, uint32_t gather) {
    hipLaunchKernelGGL(k_dequant, dim3((K + 255) / 256, n_rows), dim3(256), 0, c->stream, qtype, W, row0, n_rows,
                       K, out, row_from_dev, clamp_rows, gather);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

extern "C" int zh_dequant_rows(zh_ctx *c, uint32_t qtype, const zh_buf *W, uint64_t a_off, uint32_t row0,
                               uint32_t n_rows, uint32_t K, zh_buf *out, uint64_t out_off) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (zh_bytes_per_block(qtype) == 0) return zh_set_err(c, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "qtype %u", qtype);
    if (K % zh_block_size(qtype) || n_rows == 0) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "shape");
    if (!in_range(W, a_off, zh_tensor_bytes(qtype, (uint64_t)row0 + n_rows, K)) ||
        !in_range(out, out_off, (uint64_t)n_rows * K * 4) || (out_off & 3))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "range");
    return zhk_dequant_rows(c, qtype, (const uint8_t *)W->ptr + a_off, row0, n_rows, K,
                            (float *)((char *)out->ptr + out_off), nullptr, 0);
}
