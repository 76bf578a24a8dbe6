// zh_xcd.h — helpers for launches whose workgroups exchange data inside one
// XCD (zh_qkv_attn.hip, zh_ffn_xcd.hip): the workgroup's XCD, device-scope
// DMA, and the bounded wait for an XCD's flag words.
//
// Every launch of these kernels has 256 workgroups, one per CU of an MI355X
// (8 XCDs x 32 CUs). The dispatcher deals a launch's workgroups round robin
// over the XCDs, starting where the previous launch stopped (measured:
// workgroup w lands on XCD (w + s) % 8 for a launch-dependent s; the engine
// checks this once per context with zhk_xcd_round_robin). A workgroup reads
// its XCD from the XCC_ID register and takes slot j = w / 8 of it: every run
// of 8 consecutive workgroups covers the 8 XCDs once, so the (XCD, j) pairs
// are all distinct.
//
// Exchange protocol inside an XCD: plain stores (they land in the XCD's L2),
// s_waitcnt vmcnt(0) for their acknowledgement, then a plain store of the
// flag word carrying the launch's epoch; consumers poll the flags with
// device-scope loads and read the data with device-scope loads or DMA, or
// with plain loads of lines they have not read before in the launch.
#pragma once
#include "zh_device.h"
#include "zh_internal.h"

constexpr uint32_t XCD_N = 8, XCD_PER = 32;  // XCDs, workgroups per XCD

ZH_DEV uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 0xFu;
}

// 16 B per lane into LDS at device scope: data another workgroup of this XCD
// stored in the shared L2
ZH_DEV void dma16_dev(const void *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off sc1" ::"v"(g), "s"(lds)
                 : "memory", "m0");
}

// Waits (bounded by ctl[1] ticks) until flag words f[0 .. n) reach epoch E;
// wave `pw` polls, one word per lane (its outstanding vector-memory
// operations drain on the first poll). Returns false after giving up (and
// sets ZH_DEVERR_ATTN_WAIT). Every thread of the workgroup calls it; DMA copies the
// other waves issued before it stay in flight.
ZH_DEV bool xcd_wait(const uint32_t *f, uint32_t n, uint32_t E, uint32_t *ctl, uint32_t tid, uint32_t pw = 0) {
    __shared__ uint32_t s_ok;
    if (tid / 64 == pw) {
        const uint32_t lane = tid & 63;
        bool ok = true;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        const uint64_t limit = __hip_atomic_load(ctl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        while (true) {
            const uint32_t v = lane < n ? __hip_atomic_load(f + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : E;
            if (__builtin_amdgcn_ballot_w64((int32_t)(v - E) < 0) == 0 && limit != 0) break;
            if (__builtin_amdgcn_s_memrealtime() - t0 >= limit) {
                ok = false;
                if (lane == 0) __hip_atomic_fetch_or(ctl, ZH_DEVERR_ATTN_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
        if (lane == 0) s_ok = ok ? 1u : 0u;
    }
    lds_bar();  // (not __syncthreads: its fence may wait for the callers' copies in flight)
    return s_ok != 0;
}

// Tagged exchange: a value published as one 64-bit atomic word, the epoch in
// the high half, so a reader polls the words themselves — no store
// acknowledgement before a flag, no flag, no second read. (64-bit atomic
// loads and stores are single-copy atomic.)
ZH_DEV void tag_store(uint64_t *p, float v, uint32_t E) {
    __hip_atomic_store(p, ((uint64_t)E << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// One wave: lane l reads words p[l + 64 i] (i < N) until all carry epoch E,
// bounded by ctl[1] ticks as xcd_wait (a zero limit gives up at once). On
// giving up the missing values are NaN, ZH_DEVERR_ATTN_WAIT is set and the
// result is false (wave-uniform).
template <int N>
ZH_DEV bool tag_wait(const uint64_t *p, uint32_t E, uint32_t *ctl, float (&v)[N]) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    const uint64_t limit = __hip_atomic_load(ctl + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t got = 0;
    while (true) {
        // every word is re-read each round, so the N loads are issued
        // together and meet at one wait (a load per not-yet-seen word would
        // put a branch, and so a wait, between them: N round trips a round)
        uint64_t w[N];
#pragma unroll
        for (int i = 0; i < N; i++) w[i] = __hip_atomic_load(p + lane + 64 * i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < N; i++) {
            if (!((got >> i) & 1u) && (uint32_t)(w[i] >> 32) == E) {
                v[i] = __uint_as_float((uint32_t)w[i]);
                got |= 1u << i;
            }
        }
        if (__builtin_amdgcn_ballot_w64(got != (1u << N) - 1u) == 0 && limit != 0) return true;
        if (__builtin_amdgcn_s_memrealtime() - t0 >= limit) {
#pragma unroll
            for (int i = 0; i < N; i++)
                if (!((got >> i) & 1u)) v[i] = __builtin_nanf("");
            if (lane == 0) __hip_atomic_fetch_or(ctl, ZH_DEVERR_ATTN_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
    }
}

// The split residual's atomic part (zh_engine.hip step_xcd): 64-bit fixed
// point in units of 2^-24. Integer adds commute, so the sum of a row's
// contributions (one per XCD or expert) does not depend on the order the
// atomics land in, and the decode step is deterministic; each contribution
// is rounded once, to 2^-24 absolute (finer than f32 above magnitude 1).
// Sums must stay below 2^37 in magnitude (the synthetic 8B-shape model's
// residual reaches ~2^31): a NaN or out-of-range contribution adds a poison
// value (-2^38 in value) that reads back as NaN while at most three of them
// meet in one element. (The launches also write NaN into the plain part of
// the residual when a wait gives up, which carries it whatever the
// accumulator holds.) (zh_fix: zh_internal.h)
ZH_DEV void fix_add(zh_fix *p, float v) {
    const double s = (double)v * 16777216.0;
    const long long q = fabs(s) < 0x1p61 ? (long long)__builtin_rint(s) : (long long)(-0x1p62);
    __hip_atomic_fetch_add(p, q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
ZH_DEV float fix_to_f(zh_fix q) {
    const int hi = (int)(q >> 32);  // units of 2^8
    const uint32_t lo = (uint32_t)q;
    if ((uint32_t)hi + (1u << 29) >= (1u << 30)) return __builtin_nanf("");  // |value| >= 2^37
    return fmaf((float)lo, 0x1p-24f, (float)hi * 256.f);
}

