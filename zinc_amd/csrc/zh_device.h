// zh_device.h — device-side helpers shared by the gfx950 kernels.
//
// Conventions:
//  * wave64 everywhere (gfx950); workgroups are multiples of 64 lanes.
//  * Weight buffers are raw GGUF blocks addressed by byte offsets, exactly as
//    the reference's DmmvPushConstants (src/compute/dmmv.zig:21-28).
//  * Activations feeding a DMMV are block-quantised once into "XQ" form (see
//    below) so the mat-vec inner loop runs on v_dot4_i32_i8 instead of
//    per-weight int->float conversion plus FMA.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));  // dword-aligned 128-bit load
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define ZH_DEV static __device__ __forceinline__
#define ZH_DEVM __device__ __forceinline__  // for static member functions

// Debug build only (-DZH_DEBUG_TRACE): thread 0 of each of the first 8192
// workgroups of a launch stores s_memrealtime (100 MHz) at numbered points
// 0..15 of a kernel into this source file's g_zh_trace, read back with the
// file's zh_debug_trace_<file> entry. The product build compiles the points
// away.
#ifdef ZH_DEBUG_TRACE
static __device__ uint64_t g_zh_trace[8192 * 16];
#define ZH_TRACE_POINT(slot)                                                                          \
    do {                                                                                              \
        const uint32_t bl_ = blockIdx.x + blockIdx.y * gridDim.x;                                     \
        if (threadIdx.x == 0 && bl_ < 8192 && (slot) < 16) g_zh_trace[bl_ * 16 + (slot)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
// a value instead of a time stamp (e.g. the workgroup's XCD), in slot 15
#define ZH_TRACE_VALUE(v)                                                                             \
    do {                                                                                              \
        const uint32_t bl_ = blockIdx.x + blockIdx.y * gridDim.x;                                     \
        if (threadIdx.x == 0 && bl_ < 8192) g_zh_trace[bl_ * 16 + 15] = (uint64_t)(v);                \
    } while (0)
#define ZH_TRACE_DUMP_FN(name)                                                                        \
    extern "C" int name(uint64_t *host, uint32_t n) {                                                 \
        static uint64_t zeros[8192 * 16];                                                             \
        int rc = (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_zh_trace), (size_t)n * 8, 0, hipMemcpyDeviceToHost); \
        return rc | (int)hipMemcpyToSymbol(HIP_SYMBOL(g_zh_trace), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice); \
    }
#else
#define ZH_TRACE_POINT(slot) do { } while (0)
#define ZH_TRACE_VALUE(v) do { } while (0)
#define ZH_TRACE_DUMP_FN(name)
#endif

// ---------------------------------------------------------------------------
// XQ activation format.
// A vector of K floats (K % 32 == 0) is cut into K/32 blocks. Block j stores
//   limb[j][3][32] int8 : X_i = L0 + 256*L1 + 65536*L2, |X_i| < 2^22
//   xs[j]  float        : x_i ~= X_i * xs[j], xs = 2^(E-22), max|x| < 2^E
//   xsum[j][2] float    : sum of the quantised x over each 16-element half
// X carries 22 magnitude bits relative to the block maximum, so the
// representation error (<= 2^-23 of the block max per element) is below the
// rounding of an f32 serial dot product. Dot products against 4..8-bit
// weight codes accumulate exactly in int32.
// ---------------------------------------------------------------------------
typedef _Float16 half4 __attribute__((ext_vector_type(4)));  // MFMA f16 operand fragment
typedef float floatx4 __attribute__((ext_vector_type(4)));    // MFMA 16x16 accumulator fragment

struct XQView {
    int8_t *limb;   // [nblk][3][32]
    float *xs;      // [nblk]
    float *xsum;    // [nblk][2]
};
ZH_DEV XQView xq_view(void *base, uint32_t nblk) {
    XQView v;
    v.limb = (int8_t *)base;
    v.xs = (float *)((char *)base + (size_t)nblk * 96);
    v.xsum = v.xs + nblk;
    return v;
}

ZH_DEV float bits_f(uint32_t u) { return __uint_as_float(u); }

// Quantise one value given the block's inverse scale 2^(22-E).
ZH_DEV int xq_quant(float x, float inv) {
    int X = (int)__builtin_rintf(x * inv);  // power-of-two scaling is exact
    X = X > 4194303 ? 4194303 : (X < -4194303 ? -4194303 : X);
    return X;
}
// Block exponent for max|x|: returns inverse scale 2^(22-E) and scale 2^(E-22)
// with max|x| < 2^E. amax == 0 (or denormal) gives zero scales.
ZH_DEV void xq_scales(float amax, float &inv, float &scale) {
    uint32_t eb = __float_as_uint(amax) >> 23;  // biased exponent of amax
    if (eb == 0) { inv = 0.f; scale = 0.f; return; }
    int E = (int)eb - 126;                     // amax < 2^E
    int ei = 22 - E + 127, es = E - 22 + 127;
    ei = ei < 1 ? 1 : (ei > 254 ? 254 : ei);
    es = es < 1 ? 1 : (es > 254 ? 254 : es);
    inv = __uint_as_float((uint32_t)ei << 23);
    scale = __uint_as_float((uint32_t)es << 23);
}
// Split X into three balanced int8 limbs.
ZH_DEV void xq_limbs(int X, int &l0, int &l1, int &l2) {
    l0 = (int)(int8_t)(X & 0xFF);
    int X1 = (X - l0) >> 8;
    l1 = (int)(int8_t)(X1 & 0xFF);
    l2 = (X1 - l1) >> 8;
}
ZH_DEV uint32_t pack4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xFF) | ((uint32_t)(b & 0xFF) << 8) | ((uint32_t)(c & 0xFF) << 16) |
           ((uint32_t)(d & 0xFF) << 24);
}

ZH_DEV int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// ---------------------------------------------------------------------------
// Wave64 reductions (DPP/permute lowered by the compiler).
// ---------------------------------------------------------------------------
template <int WIDTH>
ZH_DEV float team_sum(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
// Butterfly exchanges across rows, lane l with lane l ^ 16 / l ^ 32, as
// VALU permlane swaps (no LDS round trip): swapping v with itself leaves the
// lower lane's value in r[0] and the upper lane's in r[1] in both lanes of a
// pair, so both compute op(lower, upper) -- the same bits in both lanes.
ZH_DEV float xor16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
ZH_DEV float xor32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
ZH_DEV float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
ZH_DEV float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// DPP lane exchanges inside a 16-lane row and readlane across rows: a few
// cycles each instead of an LDS-crossbar round trip. All 64 lanes of the
// wave must be active. Controls: quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] =
// 0x4E, row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
ZH_DEV float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
ZH_DEV float lane_f(float v, int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l)); }
ZH_DEV float row8_sum(float v) {  // sum over each aligned group of 8 lanes, in every lane of it
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    return v + dpp_f<0x141>(v);
}
ZH_DEV float row8_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    return fmaxf(v, dpp_f<0x141>(v));
}
ZH_DEV float row16_sum(float v) { v = row8_sum(v); return v + dpp_f<0x140>(v); }
ZH_DEV float row16_max(float v) { v = row8_max(v); return fmaxf(v, dpp_f<0x140>(v)); }
// v uniform within each 16-lane row -> wave-uniform total
ZH_DEV float rows_sum(float v) { return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48)); }
ZH_DEV float rows_max(float v) { return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48))); }
ZH_DEV float wave_sum(float v) { return rows_sum(row16_sum(v)); }
// Sum over aligned teams of TL lanes (TL = 4..64), result in every lane of
// the team. All lanes of the wave active.
template <int TL>
ZH_DEV float team_sum_dpp(float v) {
    if (TL == 4) {
        v += dpp_f<0xB1>(v);
        return v + dpp_f<0x4E>(v);
    }
    if (TL == 8) return row8_sum(v);
    v = row16_sum(v);
    if (TL == 32) return xor16_sum(v);
    if (TL >= 64) return rows_sum(v);
    return v;
}
ZH_DEV float wave_max(float v) { return rows_max(row16_max(v)); }

ZH_DEV float h2f(uint32_t h16) { return (float)__ushort_as_half((unsigned short)(h16 & 0xFFFF)); }
// f32 -> f16 round-to-nearest-even in integer arithmetic (subnormals kept,
// overflow to inf), independent of the hardware's fp16 denormal mode.
ZH_DEV uint16_t f2h_rn(float f) {
    uint32_t u = __float_as_uint(f);
    uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (a > 0x7F800000u ? 0x200u : 0u));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (a < 0x38800000u) {
        if (a < 0x33000000u) return (uint16_t)sign;
        uint32_t e = a >> 23, man = (a & 0x7FFFFFu) | 0x800000u, shift = 126u - e;
        uint32_t q = man >> shift, rem = man & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (a - 0x38000000u) >> 13, rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

// Load n dwords starting at an arbitrary byte address (byte-aligned) using
// dword-aligned loads and v_alignbyte. `out` receives n dwords.
template <int N>
ZH_DEV void load_unaligned(const uint8_t *p, uint32_t *out) {
    uintptr_t a = (uintptr_t)p;
    const uint32_t *q = (const uint32_t *)(a & ~(uintptr_t)3);
    uint32_t sh = (uint32_t)(a & 3);
    uint32_t t[N + 1];
#pragma unroll
    for (int i = 0; i < N + 1; i++) t[i] = q[i];
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __builtin_amdgcn_alignbyte(t[i + 1], t[i], sh);
}

// Device-scope (all XCDs) store / load: coherent across the XCDs' L2s
// without writing back or invalidating other data (an agent-scope fence
// writes back / invalidates a whole XCD L2).
ZH_DEV void st_dev(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
ZH_DEV float ld_dev(const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
ZH_DEV uint64_t ld_dev64(const float *p) {  // two floats, 8-byte aligned
    return __hip_atomic_load((const uint64_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Quantises one 32-element block held one value per lane by 32 consecutive
// lanes (l = lane & 31). Each 32-lane half of the wave is either fully
// active or fully inactive.
ZH_DEV float half_max(float v) {  // max over each 32-lane half, in every lane of it
    v = row16_max(v);
    const float lo = fmaxf(lane_f(v, 0), lane_f(v, 16)), hi = fmaxf(lane_f(v, 32), lane_f(v, 48));
    return (threadIdx.x & 32) ? hi : lo;
}
ZH_DEV void xq_store_block32(float xi, int l, XQView v, uint32_t blk) {
    float a = half_max(fabsf(xi));
    float inv, sc;
    xq_scales(a, inv, sc);
    int X = xq_quant(xi, inv);
    int l0, l1, l2;
    xq_limbs(X, l0, l1, l2);
    v.limb[blk * 96 + l] = (int8_t)l0;
    v.limb[blk * 96 + 32 + l] = (int8_t)l1;
    v.limb[blk * 96 + 64 + l] = (int8_t)l2;
    // integer sum over each 16-lane row: the block's two 16-element sums
    int s = X;
    s += __builtin_amdgcn_update_dpp(0, s, 0xB1, 0xF, 0xF, false);
    s += __builtin_amdgcn_update_dpp(0, s, 0x4E, 0xF, 0xF, false);
    s += __builtin_amdgcn_update_dpp(0, s, 0x141, 0xF, 0xF, false);
    s += __builtin_amdgcn_update_dpp(0, s, 0x140, 0xF, 0xF, false);
    if (l == 0) v.xs[blk] = sc;
    if ((l & 15) == 0) v.xsum[blk * 2 + (l >> 4)] = (float)s * sc;
}

// xq_store_block32 for a consumer in another workgroup of the same launch:
// every word at device scope (each 4-lane group's limb bytes packed into a
// dword first).
ZH_DEV void xq_store_block32_dev(float xi, int l, XQView v, uint32_t blk) {
    float a = half_max(fabsf(xi));
    float inv, sc;
    xq_scales(a, inv, sc);
    int X = xq_quant(xi, inv);
    int l0, l1, l2;
    xq_limbs(X, l0, l1, l2);
    const uint32_t b = ((uint32_t)(uint8_t)l0) | ((uint32_t)(uint8_t)l1 << 8) | ((uint32_t)(uint8_t)l2 << 16);
    const uint32_t b1 = __shfl_down(b, 1, 64), b2 = __shfl_down(b, 2, 64), b3 = __shfl_down(b, 3, 64);
    if ((l & 3) == 0) {
        uint32_t *limb = (uint32_t *)(v.limb + (size_t)blk * 96);
#pragma unroll
        for (int k = 0; k < 3; k++) {
            const uint32_t w = ((b >> (8 * k)) & 0xFF) | (((b1 >> (8 * k)) & 0xFF) << 8) |
                               (((b2 >> (8 * k)) & 0xFF) << 16) | (((b3 >> (8 * k)) & 0xFF) << 24);
            __hip_atomic_store(limb + k * 8 + l / 4, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    int s = X;
    s += __builtin_amdgcn_update_dpp(0, s, 0xB1, 0xF, 0xF, false);
    s += __builtin_amdgcn_update_dpp(0, s, 0x4E, 0xF, 0xF, false);
    s += __builtin_amdgcn_update_dpp(0, s, 0x141, 0xF, 0xF, false);
    s += __builtin_amdgcn_update_dpp(0, s, 0x140, 0xF, 0xF, false);
    if (l == 0) st_dev(v.xs + blk, sc);
    if ((l & 15) == 0) st_dev(v.xsum + blk * 2 + (l >> 4), (float)s * sc);
}

// Argmax: first (lowest-index) maximum; NaN never compares greater, as the
// reference's strict `>` scan (forward.zig:10348-10356).
ZH_DEV void am_better(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}
ZH_DEV void am_wave(float &bv, uint32_t &bi) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float ov = __shfl_xor(bv, o, 64);
        uint32_t oi = (uint32_t)__shfl_xor((int)bi, o, 64);
        am_better(bv, bi, ov, oi);
    }
}

// Router top-k with softmax over the selected logits (softmax_topk_v2.comp,
// topKSoftmax forward.zig:496-537), in one wave: lane l holds logits l,
// l+64, l+128, l+192 (n <= 256). Exact f32 comparisons, the lowest index wins
// ties; routing = [ids u32 x k][weights f32 x k] with weights
// exp(sel_j - sel_0) / sum.
ZH_DEV void topk_softmax_wave(const float (&vals)[4], uint32_t n, uint32_t k, uint32_t *routing) {
    const uint32_t lane = threadIdx.x & 63;
    bool avail[4];
#pragma unroll
    for (int i = 0; i < 4; i++) avail[i] = lane + 64 * i < n;
    float mysel = 0.f, m0 = 0.f;
    for (uint32_t j = 0; j < k; j++) {
        // best remaining (value desc, index asc) in this lane
        float bv = -INFINITY;
        uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (avail[i] && (bi == 0xFFFFFFFFu || vals[i] > bv)) { bv = vals[i]; bi = lane + 64 * i; }
        // wave maximum, then the lowest index holding it (indices < 256 are
        // exact as floats; DPP reductions, no LDS crossbar)
        const float m = wave_max(bv);
        const float candf = (bi != 0xFFFFFFFFu && bv == m) ? (float)bi : INFINITY;
        const float cmin = -wave_max(-candf);
        const uint32_t cand = cmin == INFINITY ? 0xFFFFFFFFu : (uint32_t)cmin;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (lane + 64 * i == cand) avail[i] = false;
        if (lane == 0) routing[j] = cand;
        if (lane == j) mysel = m;
        if (j == 0) m0 = m;
    }
    const float my = lane < k ? expf(mysel - m0) : 0.f;
    const float s = wave_sum(my);
    if (lane < k) ((float *)routing)[k + lane] = my / s;
}

// ---------------------------------------------------------------------------
// Asynchronous HBM -> LDS copies (gfx950 global_load_lds_dwordx4). Each is
// issued from inline assembly, so the compiler tracks none of them: the
// kernels that use them issue no compiler-visible global loads while copies
// are in flight (a compiler-generated wait for such a load would be
// vmcnt(0) and drain every copy) and wait explicitly with wait_vm.
// ---------------------------------------------------------------------------
ZH_DEV uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
// 64 lanes x 16 bytes from per-lane global addresses into LDS at the
// wave-uniform byte address `lds` + 16 * lane.
ZH_DEV void dma16(const void *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
// The same copy at system scope: it reads past this XCD's L2, for data that
// another workgroup of the same launch (perhaps on another XCD) stored at
// device scope.
ZH_DEV void dma16_sys(const void *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off sc0 sc1" ::"v"(g), "s"(lds)
                 : "memory", "m0");
}
template <bool COH>
ZH_DEV void dma16_act(const void *g, uint32_t lds) {
    if (COH) dma16_sys(g, lds);
    else dma16(g, lds);
}
template <int N>
ZH_DEV void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Waits until at most n of this wave's vector-memory instructions are
// outstanding (n <= 40; larger counts wait for everything).
ZH_DEV void wait_vm_dyn(uint32_t n) {
    switch (n) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<1>(); break;
    case 2: wait_vm<2>(); break;
    case 3: wait_vm<3>(); break;
    case 4: wait_vm<4>(); break;
    case 5: wait_vm<5>(); break;
    case 6: wait_vm<6>(); break;
    case 7: wait_vm<7>(); break;
    case 8: wait_vm<8>(); break;
    case 9: wait_vm<9>(); break;
    case 10: wait_vm<10>(); break;
    case 11: wait_vm<11>(); break;
    case 12: wait_vm<12>(); break;
    case 13: wait_vm<13>(); break;
    case 14: wait_vm<14>(); break;
    case 15: wait_vm<15>(); break;
    case 16: wait_vm<16>(); break;
    case 17: wait_vm<17>(); break;
    case 18: wait_vm<18>(); break;
    case 19: wait_vm<19>(); break;
    case 20: wait_vm<20>(); break;
    case 21: wait_vm<21>(); break;
    case 22: wait_vm<22>(); break;
    case 23: wait_vm<23>(); break;
    case 24: wait_vm<24>(); break;
    case 25: wait_vm<25>(); break;
    case 26: wait_vm<26>(); break;
    case 27: wait_vm<27>(); break;
    case 28: wait_vm<28>(); break;
    case 29: wait_vm<29>(); break;
    case 30: wait_vm<30>(); break;
    case 31: wait_vm<31>(); break;
    case 32: wait_vm<32>(); break;
    case 33: wait_vm<33>(); break;
    case 34: wait_vm<34>(); break;
    case 35: wait_vm<35>(); break;
    case 36: wait_vm<36>(); break;
    case 37: wait_vm<37>(); break;
    case 38: wait_vm<38>(); break;
    case 39: wait_vm<39>(); break;
    case 40: wait_vm<40>(); break;
    default: wait_vm<0>(); break;  // conservative: everything
    }
}
// The thread index, opaque to the optimiser: what a phase of the persistent
// kernel derives from it is recomputed in that phase instead of being
// hoisted out of the layer loop (where it would stay live in registers
// through every other phase).
ZH_DEV uint32_t phase_tid() {
    uint32_t t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}
// Barrier for LDS data: this wave's LDS accesses complete, then s_barrier.
// Unlike __syncthreads it does not drain the wave's DMAs in flight.
ZH_DEV void lds_bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
