// zh_dmmv_ring.hip — the one-launch form of the streaming Q4_K DMMV
// (zh_ring_q4k.h) for the decode projections with K = 2048 or 4096 (Q/K/V,
// O, gate/up of the 8B and MoE shapes).
//
// Replaces the same dispatches as zh_dmmv_lpb.hip's tile kernels
// (DmmvDispatch.recordDispatch, src/compute/dmmv.zig:806-874, and the fused
// gate/up/SwiGLU of forward.zig:8237-8273).
#include "zh_ring_q4k.h"

template <int NB, int MODE, int XIN>
__global__ __launch_bounds__(RG_T, 1) void k_q4k_ring(RingP p) {
    extern __shared__ __align__(16) uint8_t lds[];
    q4k_ring_body<NB, MODE, XIN, false>(p, blockIdx.x, lds);
}

ZH_TRACE_DUMP_FN(zh_debug_trace_ring)

template <int NB, int MODE, int XIN>
static int launch_ring(zh_ctx *c, const RingP &p, uint32_t grid) {
    static bool attr = false;  // per instantiation: raise the dynamic-LDS limit once
    if (!attr) {
        ZH_HIP(c, hipFuncSetAttribute((const void *)k_q4k_ring<NB, MODE, XIN>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)RG_LDS));
        attr = true;
    }
    hipLaunchKernelGGL((k_q4k_ring<NB, MODE, XIN>), dim3(grid), dim3(RG_T), RG_LDS, c->stream, p);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

template <int NB>
static int launch_ring_nb(zh_ctx *c, const RingP &p, uint32_t grid, int mode, int xin) {
    if (mode == LPB_GATE_UP) {
        if (xin == 0) return launch_ring<NB, LPB_GATE_UP, 0>(c, p, grid);
        if (xin == 1) return launch_ring<NB, LPB_GATE_UP, 1>(c, p, grid);
        return launch_ring<NB, LPB_GATE_UP, 2>(c, p, grid);
    }
    if (xin == 0) return launch_ring<NB, LPB_PLAIN, 0>(c, p, grid);
    if (xin == 1) return launch_ring<NB, LPB_PLAIN, 1>(c, p, grid);
    return launch_ring<NB, LPB_PLAIN, 2>(c, p, grid);
}

// Returns -1 when the shape is not one the ring kernel takes (the caller
// then uses the tile kernels): Q4_K, K = 2048 or 4096, 16-byte aligned
// matrices and activations, at most RG_MAXROWS output rows per workgroup,
// no normalised-activation copy.
int zhk_dmmv_ring(zh_ctx *c, uint32_t qtype, int mode, uint32_t nseg, const uint8_t *const *W, const uint8_t *W2,
                  float *const *y, const uint32_t *M, const float *x, const float *norm_w, float eps,
                  float *normed_out, uint32_t K, uint32_t acc, const void *xq, uint8_t *xq_out, uint32_t *grp_cnt) {
    if (zh_knob("ZH_NO_RING") || qtype != ZH_Q4_K || (K != 4096 && K != 2048) || normed_out || nseg < 1 || nseg > 3)
        return -1;
    if (mode == LPB_GATE_UP && (nseg != 1 || !W2 || ((uintptr_t)W2 & 15))) return -1;
    const void *xin = xq ? xq : (const void *)x;
    if (!xin || ((uintptr_t)xin & 15) || (norm_w && ((uintptr_t)norm_w & 15))) return -1;
    RingP p = {};
    p.x = x; p.norm_w = norm_w; p.eps = eps; p.xq = (const uint8_t *)xq;
    p.K = K; p.acc = acc; p.nseg = nseg;
    uint32_t end = 0;
    for (uint32_t s = 0; s < nseg; s++) {
        if ((uintptr_t)W[s] & 15) return -1;
        p.segW[s] = W[s]; p.segY[s] = y[s];
        end += M[s];
        p.seg_end[s] = end;
    }
    p.W2 = W2;
    p.M = end;
    p.xq_out = xq_out;
    p.grp_cnt = grp_cnt;
    const uint32_t cus = (uint32_t)c->cu_count;
    uint32_t rpw = (p.M + cus - 1) / cus;
    if (rpw < 8) rpw = 8;
    if (rpw > RG_MAXROWS) return -1;
    const uint32_t grid = (p.M + rpw - 1) / rpw;
    p.rpw = rpw;
    if (xq_out) {
        // every workgroup publishes at most LPB_XQ_MAX_GROUPS 32-row groups
        if (mode != LPB_GATE_UP || p.M % 32 || !grp_cnt || rpw / 32 + 2 > LPB_XQ_MAX_GROUPS) return -1;
    }
    const int xin_kind = xq ? 2 : (norm_w ? 1 : 0);
    return K == 4096 ? launch_ring_nb<16>(c, p, grid, mode, xin_kind) : launch_ring_nb<8>(c, p, grid, mode, xin_kind);
}
