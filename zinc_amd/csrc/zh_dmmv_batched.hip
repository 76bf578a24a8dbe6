// zh_dmmv_batched.hip -- batched decode DMMV: the Q4_K and Q6_K tile kernels
// over several activation vectors (a skinny GEMM, recordBatchDispatchPush
// dmmv.zig:880-925 / dmmv_q4k_batch.comp, dmmv_q6k_batch.comp). Each weight
// tile is read from HBM once and staged in LDS; the lane that owns a
// super-block meets every vector's LDS image, so the weight stream is shared
// and only the LDS reads and dot products grow with the vector count. Per
// vector the arithmetic is that of the one-vector tile kernels in
// zh_dmmv_lpb.hip (kept in their own translation unit, whose code these
// kernels leave untouched).
#include "zh_device.h"
#include "zh_internal.h"

#include "zh_lpb_common.h"

#define TRACE(slot) do { } while (0)

// Batched tile kernels (NV > 1 activation vectors): vector v reads x[v] (f32)
// or xq[v] (XQ) and writes y[s][v] for segment s (LpbP's x / xq / segY are
// unused). A second kernel argument, so the one-vector kernels' argument
// block and code stay as they are.
constexpr int BT_MAXV = 4;
struct LpbB {
    const float *x[BT_MAXV];
    const uint8_t *xq[BT_MAXV];
    float *y[3][BT_MAXV];
    uint32_t nv;  // activation vectors of the launch (2 or 4)
};

// Batched staging: NV activation vectors into NV LDS images. Every vector's
// loads are issued, then fetch() (the first weight tile), then each image is
// built in turn, with the arithmetic of stage_and_fetch for one vector.
template <int NV, int XQCH, int XCH, class Fetch>
ZH_DEV void stage_and_fetch_nv(const LpbP &p, const LpbB &bt, const XLds (&lx)[NV], float *red, const Fetch &fetch) {
    if (bt.xq[0]) {
        XRegsQ<XQCH> xr[NV];
#pragma unroll
        for (int v = 0; v < NV; v++) stage_xq_issue(bt.xq[v], p.K, xr[v]);
        fetch();
#pragma unroll
        for (int v = 0; v < NV; v++) stage_xq_finish(xr[v], p.K, lx[v]);
    } else if (p.norm_w) {
        XRegsF<XCH> xr[NV];
#pragma unroll
        for (int v = 0; v < NV; v++) stage_x_issue<XCH, true>(bt.x[v], p.norm_w, p.K, xr[v]);
        fetch();
#pragma unroll
        for (int v = 0; v < NV; v++) stage_x_finish(xr[v], true, p.eps, p.K, lx[v], red, nullptr);
    } else {
        XRegsF<XCH> xr[NV];
#pragma unroll
        for (int v = 0; v < NV; v++) stage_x_issue<XCH, false>(bt.x[v], nullptr, p.K, xr[v]);
        fetch();
#pragma unroll
        for (int v = 0; v < NV; v++) stage_x_finish(xr[v], false, p.eps, p.K, lx[v], red, nullptr);
    }
}

// k_dmmv_q4k_tile over NV > 1 activation vectors (batched decode,
// recordBatchDispatchPush dmmv.zig:880-925 with num_cols = NV): the weight
// tile is read once and each lane's super-block meets every vector's LDS
// image; per vector the arithmetic is that of k_dmmv_q4k_tile. (A separate
// kernel: folding the vector loop into the one-vector kernel changed its
// instruction schedule and cost it time.)
template <int TL, int MODE, int NV>
__global__ __launch_bounds__(LPB_T, NV == 2 ? 2 : 1) void k_dmmv_q4k_tile_nv(LpbP p, LpbB bt) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    __shared__ float red[4];
    __shared__ float gate_res[NV][LPB_T / TL];
    constexpr int NM = MODE == LPB_GATE_UP ? 2 : 1;
    constexpr int TPB = LPB_T / TL;         // teams (one row each) per batch
    constexpr int RPB = TPB / NM;           // rows of each matrix per batch
    constexpr int NCH = (9 + NM - 1) / NM;  // 16-byte chunks per lane per matrix
    const uint32_t nb = p.K / 256, row_bytes = nb * 144, sub_bytes = RPB * row_bytes;
    XLds lx[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) lx[v] = xlds_view(lds_raw + (size_t)v * nb * (XB_STRIDE + 96), nb);
    uint8_t *tile = lds_raw + (size_t)NV * nb * (XB_STRIDE + 96);
    const int tid = threadIdx.x, tlane = tid % TL, team = tid / TL;
    const int mat = team / RPB, rt = team % RPB;
    const bool active = (uint32_t)tlane < nb;
    const uint32_t b = active ? tlane : 0;
    const uint32_t nbatch = (p.M + RPB - 1) / RPB;
    // Batches are dealt round-robin, except when the SwiGLU output is emitted
    // as XQ: then each workgroup takes a contiguous run of `per` batches so it
    // completes whole 32-row groups where it can and publishes once, after its
    // loop (the host sizes the grid so every run is non-empty).
    const uint32_t b0 = blockIdx.x, b1 = nbatch, bstep = gridDim.x;
    u32x4 st[NM][NCH];
    uint32_t bi = b0;
    TRACE(0);
    // grid <= nbatch (host), so the first batch always exists
    stage_and_fetch_nv<NV, (3 * TL + 15) / 16, (TL / 4 > 1 ? TL / 4 : 1)>(
            p, bt, lx, red, [&] { tile_fetch<NM, NCH, RPB>(p, bi, row_bytes, st); });
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
        float accd[NV], accm[NV];
#pragma unroll
        for (int v = 0; v < NV; v++) accd[v] = accm[v] = 0.f;
#pragma unroll
        for (int pp = 0; pp < 4; pp++) {
#pragma unroll
            for (int v = 0; v < NV; v++) {
                uint32_t xo = (uint32_t)(2 * pp) * 96u;
                asm volatile("" : "+v"(xo) : "v"(accd[v]));
                const uint8_t *xl = lx[v].limb + (size_t)b * XB_STRIDE;
                uint32_t L[2][24];
                lds_load_limbs(L[0], xl + xo);
                lds_load_limbs(L[1], xl + xo + 96);
                const float xs0 = lx[v].xs[b * 8 + 2 * pp], xs1 = lx[v].xs[b * 8 + 2 * pp + 1];
                const float xz0 = lx[v].xz16[b * 16 + 4 * pp] + lx[v].xz16[b * 16 + 4 * pp + 1];
                const float xz1 = lx[v].xz16[b * 16 + 4 * pp + 2] + lx[v].xz16[b * 16 + 4 * pp + 3];
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
                accd[v] = fmaf(sc0 * xs0, S0, accd[v]);
                accd[v] = fmaf(sc1 * xs1, S1, accd[v]);
                accm[v] = fmaf(m0, xz0, accm[v]);
                accm[v] = fmaf(m1, xz1, accm[v]);
            }
        }
        float res[NV];
#pragma unroll
        for (int v = 0; v < NV; v++) {
            res[v] = active ? fmaf(h.d, accd[v], -h.dmin * accm[v]) : 0.f;
            res[v] = team_sum_dpp<TL>(res[v]);
        }
        if (MODE == LPB_GATE_UP) {
            if (mat == 0 && tlane == 0)
#pragma unroll
                for (int v = 0; v < NV; v++) gate_res[v][rt] = res[v];
            __syncthreads();
            if (mat == 1 && tlane == 0 && (uint32_t)rt < nrows) {
#pragma unroll
                for (int v = 0; v < NV; v++) {
                    float *yb = bt.y[sg][v];
                    yb[rr0 + rt] = silu_mul(gate_res[v][rt], res[v]);
                }
            }
        } else if (tlane == 0 && (uint32_t)rt < nrows) {
#pragma unroll
            for (int v = 0; v < NV; v++) {
                float *yb = bt.y[sg][v];
                float out = res[v];
                if (p.acc) out += yb[rr0 + rt];
                yb[rr0 + rt] = out;
            }
        }
        __syncthreads();  // the tile is rewritten by the next batch
    }
    TRACE(7);
}

// k_dmmv_q6k_tile over NV > 1 activation vectors, as k_dmmv_q4k_tile_nv.
template <int TL, int NCH, int NV>
__global__ __launch_bounds__(LPB_T, 1) void k_dmmv_q6k_tile_nv(LpbP p, LpbB bt) {
    extern __shared__ __align__(16) uint8_t lds_raw[];
    __shared__ float red[4];
    constexpr int RPB = LPB_T / TL;  // rows per batch
    // NCH = ceil(RPB * row bytes / 4 KB) 16-byte chunks per lane and tile
    const uint32_t nb = p.K / 256, row_bytes = nb * 210, nh = nb * 2;
    XLds lx[NV];
#pragma unroll
    for (int v = 0; v < NV; v++) lx[v] = xlds_view(lds_raw + (size_t)v * nb * (XB_STRIDE + 96), nb);
    uint8_t *tile = lds_raw + (size_t)NV * nb * (XB_STRIDE + 96);
    const int tid = threadIdx.x, tlane = tid % TL, rt = tid / TL;
    const bool active = (uint32_t)tlane < nh;
    const uint32_t hb = active ? tlane : 0, b = hb >> 1, h = hb & 1;
    const uint32_t nbatch = (p.M + RPB - 1) / RPB;
    u32x4 st[1][NCH];
    uint32_t bi = blockIdx.x;
    TRACE(0);
    // grid <= nbatch (host), so the first batch always exists
    stage_and_fetch_nv<NV, (3 * TL / 2 + 15) / 16, (TL / 8 > 1 ? TL / 8 : 1)>(
            p, bt, lx, red, [&] { tile_fetch<1, NCH, RPB>(p, bi, row_bytes, st); });
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
        float acc[NV];
#pragma unroll
        for (int v = 0; v < NV; v++) acc[v] = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
#pragma unroll
            for (int v = 0; v < NV; v++) {
                uint32_t xo = (uint32_t)g * 96u;
                asm volatile("" : "+v"(xo) : "v"(acc[v]));
                const uint8_t *xl = lx[v].limb + (size_t)b * XB_STRIDE + h * 4 * 96;  // sub-blocks 4h..4h+3
                uint32_t L[24];
                lds_load_limbs(L, xl + xo);
                const float xs = lx[v].xs[b * 8 + 4 * h + g];
                const float z0 = -32.f * lx[v].xz16[b * 16 + (4 * h + g) * 2];
                const float z1 = -32.f * lx[v].xz16[b * 16 + (4 * h + g) * 2 + 1];
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
                acc[v] = fmaf((float)sc0, fmaf(xs, S0, z0), acc[v]);
                acc[v] = fmaf((float)sc1, fmaf(xs, S1, z1), acc[v]);
            }
        }
        const uint32_t dw = __builtin_amdgcn_alignbyte(rs[5], rs[4], sh);  // bytes 208..211
        constexpr int TLW = TL > 64 ? 64 : TL;
        float res[NV];
#pragma unroll
        for (int v = 0; v < NV; v++) {
            res[v] = active ? h2f(dw) * acc[v] : 0.f;
            res[v] = team_sum_dpp<TLW>(res[v]);
        }
        if (TL > 64) {  // team spans TL/64 waves
            __shared__ float xred[NV][LPB_T / 64];
            if ((tid & 63) == 0)
#pragma unroll
                for (int v = 0; v < NV; v++) xred[v][tid >> 6] = res[v];
            __syncthreads();
#pragma unroll
            for (int v = 0; v < NV; v++) {
                float t = 0.f;
#pragma unroll
                for (int w = 0; w < TL / 64; w++) t += xred[v][(rt * TL) / 64 + w];
                res[v] = t;
            }
        }
        if (tlane == 0 && (uint32_t)rt < nrows) {
#pragma unroll
            for (int v = 0; v < NV; v++) {
                float *yb = bt.y[sg][v];
                float out = res[v];
                if (p.acc) out += yb[rr0 + rt];
                yb[rr0 + rt] = out;
            }
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

// LDS a workgroup may hold beyond the static arrays of the tile kernels
constexpr uint32_t TILE_LDS_MAX = 163840 - 2048;

template <int TL>
static int launch_q4k_nv(zh_ctx *c, const LpbP &p, const LpbB &bt, uint32_t wgs, uint32_t lds) {
#define Q4T(MM, NN) hipLaunchKernelGGL((k_dmmv_q4k_tile_nv<TL, MM, NN>), dim3(wgs), dim3(LPB_T), lds, c->stream, p, bt)
    if (p.mode == LPB_GATE_UP) {
        if (bt.nv == 4) Q4T(LPB_GATE_UP, 4);
        else Q4T(LPB_GATE_UP, 2);
    } else {
        if (bt.nv == 4) Q4T(LPB_PLAIN, 4);
        else Q4T(LPB_PLAIN, 2);
    }
#undef Q4T
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

// Q4_K: team of <= 64 lanes (K <= 16384), 16-byte aligned matrices, every
// segment but the last a whole number of batches, NV images + tile in LDS.
// -1: this vector count does not fit (the caller tries fewer).
static int try_q4k_nv(zh_ctx *c, const LpbP &p, uint32_t nseg, const uint32_t *M, const LpbB &bt) {
    const uint32_t nb = p.K / 256;
    if (nb > 64 || (bt.nv != 2 && bt.nv != 4)) return -1;
    const uint32_t TL = pow2ceil(nb < 4 ? 4 : nb);
    const uint32_t nm = p.mode == LPB_GATE_UP ? 2 : 1;
    const uint32_t rpb = LPB_T / TL / nm;
    for (uint32_t s = 0; s < nseg; s++)
        if (((uintptr_t)p.segW[s] & 15) || (s + 1 < nseg && M[s] % rpb)) return -1;
    if (nm == 2 && ((uintptr_t)p.segW2 & 15)) return -1;
    const uint32_t lds = bt.nv * nb * (XB_STRIDE + 96) + TILE_BYTES;
    if (lds > TILE_LDS_MAX) return -1;
    const uint32_t nbatch = (p.M + rpb - 1) / rpb;
    // the NV = 2 kernel is compiled for two workgroups per CU, NV = 4 for one
    uint32_t per_cu = bt.nv == 2 ? 2u : 1u;
    if (per_cu * (lds + 2048) > 163840) per_cu = 1;
    uint32_t wgs = nbatch, cap = (uint32_t)c->cu_count * per_cu;
    if (wgs > cap) wgs = cap;
    switch (TL) {
    case 4: return launch_q4k_nv<4>(c, p, bt, wgs, lds);
    case 8: return launch_q4k_nv<8>(c, p, bt, wgs, lds);
    case 16: return launch_q4k_nv<16>(c, p, bt, wgs, lds);
    case 32: return launch_q4k_nv<32>(c, p, bt, wgs, lds);
    default: return launch_q4k_nv<64>(c, p, bt, wgs, lds);
    }
}

template <int TL>
static int launch_q6k_nv(zh_ctx *c, const LpbP &p, const LpbB &bt, uint32_t wgs, uint32_t lds, uint32_t nch) {
    switch (nch) {
#define Q6T(N)                                                                                                  \
    case N:                                                                                                     \
        if (bt.nv == 4) hipLaunchKernelGGL((k_dmmv_q6k_tile_nv<TL, N, 4>), dim3(wgs), dim3(LPB_T), lds, c->stream, p, bt); \
        else hipLaunchKernelGGL((k_dmmv_q6k_tile_nv<TL, N, 2>), dim3(wgs), dim3(LPB_T), lds, c->stream, p, bt);           \
        break;
    Q6T(4) Q6T(5) Q6T(6) Q6T(7)  // RPB * K/256 is in (64, 128], so a tile is 3.3 .. 6.6 x 4 KB
#undef Q6T
    default: return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "q6k tile: %u chunks", nch);
    }
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

// Q6_K: rows a multiple of 16 bytes (K % 2048 == 0), team of <= 128 lanes
// (K <= 16384), NV images + tile in LDS; tall matrices (the LM head) too.
static int try_q6k_nv(zh_ctx *c, const LpbP &p, uint32_t nseg, const uint32_t *M, const LpbB &bt) {
    const uint32_t nb = p.K / 256, row_bytes = nb * 210;
    if (row_bytes % 16 || nb > 64 || (bt.nv != 2 && bt.nv != 4)) return -1;
    const uint32_t TL = pow2ceil(2 * nb < 4 ? 4 : 2 * nb);
    const uint32_t rpb = LPB_T / TL;
    const uint32_t lds = bt.nv * nb * (XB_STRIDE + 96) + rpb * row_bytes;
    if (lds > TILE_LDS_MAX) return -1;
    for (uint32_t s = 0; s < nseg; s++)
        if (((uintptr_t)p.segW[s] & 15) || (s + 1 < nseg && M[s] % rpb)) return -1;
    const uint32_t nbatch = (p.M + rpb - 1) / rpb;
    uint32_t wgs = nbatch, cap = (uint32_t)c->cu_count;  // compiled for one workgroup per CU
    if (wgs > cap) wgs = cap;
    const uint32_t nch = (rpb * row_bytes + 4095) / 4096;
    switch (TL) {
    case 4: return launch_q6k_nv<4>(c, p, bt, wgs, lds, nch);
    case 8: return launch_q6k_nv<8>(c, p, bt, wgs, lds, nch);
    case 16: return launch_q6k_nv<16>(c, p, bt, wgs, lds, nch);
    case 32: return launch_q6k_nv<32>(c, p, bt, wgs, lds, nch);
    case 64: return launch_q6k_nv<64>(c, p, bt, wgs, lds, nch);
    default: return launch_q6k_nv<128>(c, p, bt, wgs, lds, nch);
    }
}

// Batched DMMV on the tile kernels: y[s * n_vec + v] (= or +=) W[s] x_v for
// v < n_vec, x_v = x[v] (f32, with the optional fused RMSNorm) or xq[v] (XQ;
// x == nullptr). Vectors go in launches of 4 or 2 (the widest whose LDS
// images fit beside the weight tile); a single vector left over takes the
// one-vector path. Per vector the arithmetic is that of the one-vector tile
// kernel, so every output equals its single-vector DMMV bit for bit.
int zhk_dmmv_batched(zh_ctx *c, uint32_t qtype, int mode, uint32_t nseg, const uint8_t *const *W, const uint8_t *W2,
                     const uint32_t *M, uint32_t K, uint32_t n_vec, const float *const *x, const void *const *xq,
                     float *const *y, const float *norm_w, float eps, uint32_t acc) {
    if (!zhk_lpb_supported(qtype, K) || (mode == LPB_GATE_UP && qtype != ZH_Q4_K) || nseg < 1 || nseg > 3 ||
        n_vec == 0 || (!x && !xq))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "batched dmmv: unsupported qtype/K/mode/vectors");
    uint32_t v0 = 0;
    while (v0 < n_vec) {
        const uint32_t left = n_vec - v0;
        uint32_t done = 0;
        for (uint32_t nv = left >= 4 ? 4u : left >= 2 ? 2u : 0u; nv >= 2 && !done; nv /= 2) {
            LpbP p = {};
            p.norm_w = norm_w; p.eps = eps;
            p.K = K; p.acc = acc; p.nseg = nseg; p.mode = (uint32_t)mode;
            p.row_bytes = zh_tensor_bytes(qtype, 1, K);
            uint32_t end = 0;
            for (uint32_t s = 0; s < nseg; s++) {
                p.segW[s] = W[s];
                end += M[s];
                p.seg_end[s] = end;
            }
            p.segW2 = W2;
            p.M = end;
            LpbB bt = {};
            bt.nv = nv;
            for (uint32_t v = 0; v < nv; v++) {
                bt.x[v] = x ? x[v0 + v] : nullptr;
                bt.xq[v] = x ? nullptr : (const uint8_t *)xq[v0 + v];
                for (uint32_t s = 0; s < nseg; s++) bt.y[s][v] = y[s * n_vec + v0 + v];
            }
            const int rc = qtype == ZH_Q4_K ? try_q4k_nv(c, p, nseg, M, bt) : try_q6k_nv(c, p, nseg, M, bt);
            if (rc > 0) return rc;
            if (rc == 0) done = nv;
        }
        if (!done) {  // one vector
            float *yv[3];
            for (uint32_t s = 0; s < nseg; s++) yv[s] = y[s * n_vec + v0];
            const int rc = zhk_dmmv_lpb(c, qtype, mode, nseg, W, W2, yv, M, x ? x[v0] : nullptr, norm_w, eps, nullptr,
                                        K, acc, x ? nullptr : xq[v0]);
            if (rc) return rc;
            done = 1;
        }
        v0 += done;
    }
    return ZH_OK;
}

static bool buf_range(const zh_buf *b, uint64_t off, uint64_t n) { return b && off <= b->size && n <= b->size - off; }

extern "C" int zh_dmmv_batched(zh_ctx *c, uint32_t qtype, const zh_buf *W, uint64_t a_off, const zh_buf *X,
                               uint64_t x_off, zh_buf *Y, uint64_t y_off, uint32_t M, uint32_t K, uint32_t num_cols,
                               uint32_t acc_mode) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (qtype != ZH_Q4_K && qtype != ZH_Q6_K)
        return zh_set_err(c, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "batched dmmv: qtype %u (Q4_K, Q6_K)", qtype);
    if (M == 0 || K == 0 || !zhk_lpb_supported(qtype, K) || num_cols == 0 || num_cols > ZH_DMMV_MAX_COLS ||
        acc_mode > 1)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "batched dmmv: M=%u K=%u cols=%u", M, K, num_cols);
    if (!buf_range(W, a_off, zh_tensor_bytes(qtype, M, K)) || !buf_range(X, x_off, 4ull * K * num_cols) ||
        !buf_range(Y, y_off, 4ull * M * num_cols) || (a_off & 15) || (x_off & 15) || (y_off & 3) || (K % 4))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "batched dmmv: range/alignment");
    const uint8_t *w = (const uint8_t *)W->ptr + a_off;
    const float *xs[ZH_DMMV_MAX_COLS];
    float *ys[ZH_DMMV_MAX_COLS];
    for (uint32_t v = 0; v < num_cols; v++) {
        xs[v] = (const float *)((const char *)X->ptr + x_off) + (size_t)v * K;
        ys[v] = (float *)((char *)Y->ptr + y_off) + (size_t)v * M;
    }
    return zhk_dmmv_batched(c, qtype, LPB_PLAIN, 1, &w, nullptr, &M, K, num_cols, xs, nullptr, ys, nullptr, 0.f,
                            acc_mode);
}

extern "C" int zh_dmmv_fused_gate_up_swiglu_batched(zh_ctx *c, uint32_t qtype, const zh_buf *Wg, uint64_t g_off,
                                                    const zh_buf *Wu, uint64_t u_off, const zh_buf *X, uint64_t x_off,
                                                    zh_buf *Y, uint64_t y_off, uint32_t M, uint32_t K,
                                                    uint32_t num_cols) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (qtype != ZH_Q4_K) return zh_set_err(c, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "batched gate/up: qtype %u (Q4_K)", qtype);
    if (M == 0 || !zhk_lpb_supported(qtype, K) || num_cols == 0 || num_cols > ZH_DMMV_MAX_COLS)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "batched gate/up: M=%u K=%u cols=%u", M, K, num_cols);
    const uint64_t wb = zh_tensor_bytes(qtype, M, K);
    if (!buf_range(Wg, g_off, wb) || !buf_range(Wu, u_off, wb) || !buf_range(X, x_off, 4ull * K * num_cols) ||
        !buf_range(Y, y_off, 4ull * M * num_cols) || (g_off & 15) || (u_off & 15) || (x_off & 15) || (y_off & 3))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "batched gate/up: range/alignment");
    const uint8_t *wg = (const uint8_t *)Wg->ptr + g_off;
    const float *xs[ZH_DMMV_MAX_COLS];
    float *ys[ZH_DMMV_MAX_COLS];
    for (uint32_t v = 0; v < num_cols; v++) {
        xs[v] = (const float *)((const char *)X->ptr + x_off) + (size_t)v * K;
        ys[v] = (float *)((char *)Y->ptr + y_off) + (size_t)v * M;
    }
    return zhk_dmmv_batched(c, qtype, LPB_GATE_UP, 1, &wg, (const uint8_t *)Wu->ptr + u_off, &M, K, num_cols, xs,
                            nullptr, ys, nullptr, 0.f, 0);
}
