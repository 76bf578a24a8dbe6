// zh_step.hip — the layers of one decode step in one persistent launch.
//
// The per-layer kernels each pay a fixed cost (workgroups start, the first
// weight bytes arrive, the last workgroups finish) of about 5 us against 1.6
// .. 10 us of streaming at the HBM rate: at batch 1 that fixed cost is most
// of the step. Here one 512-thread workgroup per CU runs every layer's five
// phases in turn and a grid barrier separates the phases:
//
//   Q/K/V    attn_norm + XQ + Q4_K DMMV of the stacked Q|K|V rows  (zh_ring_q4k.h)
//   attn     q/k norm + RoPE, new K/V row, split-K attention over
//            (kv head, chunk) = one workgroup, last-arriver merge  (attn_ring_body)
//   O        Q4_K DMMV of the attention output's XQ, += residual  (zh_ring_q4k.h)
//   gate/up  ffn_norm + XQ + Q4_K gate and up rows + SwiGLU, the
//            output also as XQ (per 32-row group, last publisher) (zh_ring_q4k.h)
//   down     Q6_K DMMV of the SwiGLU XQ, += residual              (zh_ring_q6k.h)
//
// These are the bodies the one-launch kernels run, compiled with COH: what a
// phase reads was written by other workgroups of this launch, possibly on
// another XCD, whose L2 is not this one's. Such data is stored at device
// scope (write-through past the writer's L2) and read at system scope (past
// the reader's L2); the weights and the KV cache rows read here were written
// before the launch and take the normal cached path. A barrier arrival is
// s_waitcnt 0 in every wave (this workgroup's device-scope stores have
// completed) and then a relaxed device-scope counter increment, so a
// workgroup that sees the barrier complete sees every store made before it.
//
// The barrier: 16 group counters (workgroup w in group w % 16), a root
// counter the last arrival of each group bumps, and one flag per group that
// the last root arrival sets to the barrier's number; workgroups spin on
// their group's flag. The wait is bounded (100 ms); a workgroup that gives
// up sets ZH_DEVERR_STEP_BARRIER (zh_sync reports it) and every later
// barrier of the launch stops waiting, so the launch always completes.
// Every workgroup must be resident at once: one per CU (the LDS use allows
// one), launched only when no other work shares the device.
//
// Replaces the dispatch sequence of one decode step's layers
// (decodeStep, src/compute/forward.zig:4299-5600 for the dense path).
#include "zh_device.h"
#include "zh_internal.h"

// Debug build only: per-workgroup timestamps of one layer's phases (slot
// 2 ph at the phase's start, 2 ph + 1 at its end; slot 10: the next layer's
// start), read back with zh_debug_trace_step.
#ifdef ZH_DEBUG_TRACE
static __device__ uint64_t g_step_trace[1024 * 32];
#define STEP_TRACE(l, slot)                                                                              \
    do {                                                                                                 \
        if ((l) == 10 && threadIdx.x == 0 && blockIdx.x < 1024)                                          \
            g_step_trace[blockIdx.x * 32 + (slot)] = __builtin_amdgcn_s_memrealtime();                   \
    } while (0)
// the attention body's own points (every layer; the last one stays), slots 16..31
#define TRACE_OPS(slot)                                                                                  \
    do {                                                                                                 \
        if (threadIdx.x == 0 && blockIdx.x < 1024)                                                       \
            g_step_trace[blockIdx.x * 32 + 16 + (slot)] = __builtin_amdgcn_s_memrealtime();              \
    } while (0)
extern "C" int zh_debug_trace_step(uint64_t *host, uint32_t n) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_step_trace), (size_t)n * 8, 0, hipMemcpyDeviceToHost);
}
#else
#define STEP_TRACE(l, slot) do { } while (0)
#endif

#include "zh_attn_common.h"
#include "zh_ring_q4k.h"
#include "zh_ring_q6k.h"


namespace {

constexpr int ST_T = 512;
constexpr uint32_t ST_GROUPS = 16;
constexpr uint64_t ST_WAIT_TICKS = 10000000ull;  // 100 ms of the 100 MHz clock
// ctl words (u32 index): group counters and flags 64 words (256 B) apart
constexpr uint32_t ST_GC = 0, ST_ROOT = 16 * 64, ST_FLAG = 17 * 64, ST_DONE = 33 * 64, ST_ATTN = 34 * 64;
constexpr uint32_t ST_CTL_WORDS = ST_ATTN + 128;  // + two merge words per kv head (<= 64 kv heads)

struct StepP {
    zh_step_args a;
    uint32_t *err;  // device error word
    uint32_t nd;    // attention chunks per kv head
    uint32_t rpw_qkv, rpw_o, rpw_ffn, rpw_down;
};

// Grid barrier number k (1, 2, ...) of this launch, in two halves: the
// arrival (every store of the workgroup has completed), then the wait. The
// caller issues the next phase's first copies in between.
ZH_DEV void grid_arrive(uint32_t *ctl, uint32_t k, uint32_t wg, uint32_t nwg) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t ng = nwg < ST_GROUPS ? nwg : ST_GROUPS, g = wg % ng;
        const uint32_t gsz = nwg / ng + (g < nwg % ng ? 1u : 0u);
        const uint32_t prev = __hip_atomic_fetch_add(ctl + ST_GC + g * 64, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == k * gsz - 1) {
            const uint32_t r = __hip_atomic_fetch_add(ctl + ST_ROOT, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (r == k * ng - 1)
                for (uint32_t f = 0; f < ng; f++)
                    __hip_atomic_store(ctl + ST_FLAG + f * 64, k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}
ZH_DEV void grid_wait(uint32_t *ctl, uint32_t *err, uint32_t k, uint32_t wg, uint32_t nwg) {
    if (threadIdx.x == 0) {
        const uint32_t ng = nwg < ST_GROUPS ? nwg : ST_GROUPS, g = wg % ng;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (__hip_atomic_load(ctl + ST_FLAG + g * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < k) {
            if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & ZH_DEVERR_STEP_BARRIER) break;
            if (__builtin_amdgcn_s_memrealtime() - t0 > ST_WAIT_TICKS) {
                __hip_atomic_fetch_or(err, ZH_DEVERR_STEP_BARRIER, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}

// NBH = hidden / 256, NBF = ffn / 256, G = q heads per kv head.
template <int NBH, int NBF, int G>
__global__ __launch_bounds__(ST_T, 1) void k_step_layers(StepP p) {
    extern __shared__ __align__(16) uint8_t lds[];
    const zh_step_args &a = p.a;
    const uint32_t wg = blockIdx.x, nwg = gridDim.x;
    const uint32_t H = a.hidden, qd = a.n_heads * FD_HD, kvd = a.n_kv_heads * FD_HD;
    // the position, read once (written before the launch)
    const uint32_t posv = __builtin_amdgcn_readfirstlane(a.pos.dev ? *a.pos.dev + a.pos.value : a.pos.value);
    const uint32_t kvh = wg % a.n_kv_heads, chunk = wg / a.n_kv_heads;  // attention: kv head h on XCD h % 8
    // each phase's parameters for layer l
    auto qkv_p = [&](const zh_step_layer &L) {
        RingP r = {};
        r.x = a.x; r.norm_w = L.attn_norm; r.eps = a.eps;
        r.K = H; r.nseg = 3; r.acc = 0; r.rpw = p.rpw_qkv;
        r.segW[0] = L.wq; r.segW[1] = L.wk; r.segW[2] = L.wv;
        r.segY[0] = a.q; r.segY[1] = a.k; r.segY[2] = a.v;
        r.seg_end[0] = qd; r.seg_end[1] = qd + kvd; r.seg_end[2] = qd + 2 * kvd;
        r.M = qd + 2 * kvd;
        return r;
    };
    auto attn_p = [&](const zh_step_layer &L) {
        AttnP t = {};
        t.q = a.q; t.k_new = a.k; t.v_new = a.v; t.q_norm = L.q_norm; t.k_norm = L.k_norm;
        t.rope_cs = a.rope_cs; t.kc = L.kc; t.vc = L.vc; t.pages = a.pages; t.n_pages = a.n_pages;
        t.cache_tokens = a.max_ctx; t.pos = zh_pos_src{posv, nullptr}; t.scale = a.scale; t.eps = a.eps;
        t.part = a.part; t.nd = p.nd; t.n_chunks = p.nd; t.counters = a.ctl + ST_ATTN;
        t.out = a.attn; t.xq = a.xq_attn; t.nq = a.n_heads; t.ident = a.ident; t.ctl = p.err;
        return t;
    };
    auto o_p = [&](const zh_step_layer &L) {
        RingP r = {};
        r.xq = a.xq_attn; r.K = qd; r.nseg = 1; r.acc = 1; r.rpw = p.rpw_o;
        r.segW[0] = L.wo; r.segY[0] = a.x; r.seg_end[0] = H; r.M = H;
        return r;
    };
    auto ffn_p = [&](const zh_step_layer &L) {
        RingP r = {};
        r.x = a.x; r.norm_w = L.ffn_norm; r.eps = a.eps;
        r.K = H; r.nseg = 1; r.acc = 0; r.rpw = p.rpw_ffn;
        r.segW[0] = L.gate; r.W2 = L.up; r.segY[0] = a.s; r.seg_end[0] = a.ffn; r.M = a.ffn;
        r.xq_out = a.xq_s; r.grp_cnt = a.grp_cnt;
        return r;
    };
    auto down_p = [&](const zh_step_layer &L) {
        Ring6P r = {};
        r.W = L.down; r.xq = a.xq_s; r.y = a.x; r.M = H; r.acc = 1; r.rpw = p.rpw_down;
        return r;
    };
    uint32_t nbar = 0;
    // layer l0's Q/K/V tiles (no barrier before the first phase)
    uint32_t pre = q4k_ring_prefetch<NBH, LPB_PLAIN>(qkv_p(a.layers[a.l0]), wg, lds);
    for (uint32_t l = a.l0; l < a.l1; l++) {
        const zh_step_layer &L = a.layers[l];
        STEP_TRACE(l - 1, 10);
        STEP_TRACE(l, 0);
        q4k_ring_body<NBH, LPB_PLAIN, 1, true>(qkv_p(L), wg, lds, pre);
        STEP_TRACE(l, 1);
        // ---- barrier, the attention's first K/V sub-chunks copied meanwhile
        grid_arrive(a.ctl, ++nbar, wg, nwg);
        pre = chunk < p.nd ? attn_ring_prefetch<G, 8>(attn_p(L), kvh, chunk, lds, true) : 0u;
        grid_wait(a.ctl, p.err, nbar, wg, nwg);
        STEP_TRACE(l, 2);
        if (chunk < p.nd) attn_ring_body<G, true, 8, true>(attn_p(L), kvh, chunk, lds, pre);
        STEP_TRACE(l, 3);
        grid_arrive(a.ctl, ++nbar, wg, nwg);
        pre = q4k_ring_prefetch<NBH, LPB_PLAIN>(o_p(L), wg, lds);
        grid_wait(a.ctl, p.err, nbar, wg, nwg);
        STEP_TRACE(l, 4);
        q4k_ring_body<NBH, LPB_PLAIN, 2, true>(o_p(L), wg, lds, pre);
        STEP_TRACE(l, 5);
        grid_arrive(a.ctl, ++nbar, wg, nwg);
        pre = q4k_ring_prefetch<NBH, LPB_GATE_UP>(ffn_p(L), wg, lds);
        grid_wait(a.ctl, p.err, nbar, wg, nwg);
        STEP_TRACE(l, 6);
        q4k_ring_body<NBH, LPB_GATE_UP, 1, true>(ffn_p(L), wg, lds, pre);
        STEP_TRACE(l, 7);
        grid_arrive(a.ctl, ++nbar, wg, nwg);
        pre = q6k_ring_prefetch<NBF>(down_p(L), wg, lds);
        grid_wait(a.ctl, p.err, nbar, wg, nwg);
        STEP_TRACE(l, 8);
        q6k_ring_body<NBF, true>(down_p(L), wg, lds, pre);
        STEP_TRACE(l, 9);
        if (l + 1 < a.l1) {
            grid_arrive(a.ctl, ++nbar, wg, nwg);
            pre = q4k_ring_prefetch<NBH, LPB_PLAIN>(qkv_p(a.layers[l + 1]), wg, lds);
            grid_wait(a.ctl, p.err, nbar, wg, nwg);
        }
    }
    // ---- every workgroup is past its last barrier wait: the last one to
    // get here clears the barrier words for the next launch
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0 &&
        __hip_atomic_fetch_add(a.ctl + ST_DONE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nwg - 1) {
        for (uint32_t g = 0; g < ST_GROUPS; g++) {
            __hip_atomic_store(a.ctl + ST_GC + g * 64, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.ctl + ST_FLAG + g * 64, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __hip_atomic_store(a.ctl + ST_ROOT, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.ctl + ST_DONE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int NBH, int NBF, int G>
constexpr uint32_t step_lds() {
    constexpr uint32_t a = RG_LDS_COH, b = ar_lds_bytes<G, 8>(), c = R6<NBF>::LDS;
    return a > b ? (a > c ? a : c) : (b > c ? b : c);
}

// with the kernel's static LDS (the attention merge's ~6 KB) within 160 KB
static_assert(step_lds<16, 56, 4>() <= 150u * 1024 && step_lds<16, 48, 4>() <= 150u * 1024, "LDS budget");

template <int NBH, int NBF, int G>
static int launch_step(zh_ctx *c, const StepP &p) {
    static bool attr = false;
    constexpr uint32_t lds = step_lds<NBH, NBF, G>();
    if (!attr) {
        ZH_HIP(c, hipFuncSetAttribute((const void *)k_step_layers<NBH, NBF, G>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr = true;
    }
    hipLaunchKernelGGL((k_step_layers<NBH, NBF, G>), dim3(c->cu_count), dim3(ST_T), lds, c->stream, p);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1) / b; }

}  // namespace

uint64_t zh_step_ctl_bytes() { return 4ull * ST_CTL_WORDS; }

bool zhk_step_supported(zh_ctx *c, const zh_step_args &a) {
    if (zh_knob("ZH_NO_STEP") || c->concurrent || c->cu_count < 64) return false;
    const uint32_t cus = (uint32_t)c->cu_count;
    if ((a.hidden != 2048 && a.hidden != 4096) || a.n_heads * FD_HD != a.hidden) return false;
    if (a.n_kv_heads == 0 || a.n_kv_heads > 64 || a.n_heads != 4 * a.n_kv_heads) return false;
    if (a.ffn != 12288 && a.ffn != 14336) return false;
    const uint32_t nd = attn_nd(a.n_kv_heads, c->cu_count);
    if ((uint64_t)(a.max_ctx + nd - 1) / nd > 16ull * AR_MAXPG || a.max_ctx % 16) return false;
    const uint32_t qkv = a.hidden + 2 * a.n_kv_heads * FD_HD;
    if (ceil_div(qkv, cus) > RG_MAXROWS || ceil_div(a.hidden, cus) > R6_MAXROWS) return false;
    const uint32_t rf = ceil_div(a.ffn, cus);
    if (rf > RG_MAXROWS || a.ffn % 32 || rf / 32 + 2 > LPB_XQ_MAX_GROUPS) return false;
    return true;
}

int zhk_step_layers(zh_ctx *c, const zh_step_args &a) {
    if (!zhk_step_supported(c, a)) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "step kernel: unsupported shape");
    const uint32_t cus = (uint32_t)c->cu_count;
    StepP p = {};
    p.a = a;
    p.err = c->err_dev;
    p.nd = attn_nd(a.n_kv_heads, c->cu_count);
    p.rpw_qkv = ceil_div(a.hidden + 2 * a.n_kv_heads * FD_HD, cus);
    p.rpw_o = ceil_div(a.hidden, cus);
    p.rpw_ffn = ceil_div(a.ffn, cus);
    p.rpw_down = ceil_div(a.hidden, cus);
    if (a.hidden == 4096) return a.ffn == 12288 ? launch_step<16, 48, 4>(c, p) : launch_step<16, 56, 4>(c, p);
    return a.ffn == 12288 ? launch_step<8, 48, 4>(c, p) : launch_step<8, 56, 4>(c, p);
}
