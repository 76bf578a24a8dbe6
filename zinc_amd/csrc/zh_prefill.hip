// zh_prefill.hip — batched prefill: dequant-GEMM on the MFMA units.
//
// Y[n][m] (+)= sum_k X[n][k] * W[m][k] for N tokens at once
// (dispatchProjectionBatched, forward.zig:8147-8216; recordMulMmQ4K,
// dmmv.zig:1045-1094, mul_mm_q4k.comp). X is token-major fp16 (the reference
// keeps X column-major K x N in f32, dmmv.zig:139-155 — the same element
// order), Y token-major f32. W stays in GGUF Q4_K / Q6_K blocks; each
// K-step dequantises one super-block column of a 128-row tile into LDS as
// fp16 (value computed in f32 exactly as dequantRow, then rounded to
// nearest even) and the four waves run v_mfma_f32_16x16x32_f16 with f32
// accumulation.
//
// MFMA 16x16x32 f16 operand layout (lane l): A[i][k] with i = l % 16,
// k = 8*(l/16)..+7; B[k][j] with j = l % 16, same k; D[i][j] with j = l % 16,
// i = 4*(l/16) + r, r = 0..3. Tokens are the i dimension, weight rows the j
// dimension, so each output row segment is written by 16 consecutive lanes.
#include "zh_device.h"
#include "zh_internal.h"
#include <type_traits>

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4v __attribute__((ext_vector_type(4)));

constexpr int GT = 256;         // threads (4 waves)
constexpr int TI = 128;         // tokens per tile
constexpr int KS = 128;         // k per step: half a super-block
// halfs per LDS row: 288 B (measured on the 512-token prefill: 15.45 ms
// against 15.88 for 272 B rows, 24.6 for unpadded 256 B rows; strides that
// are not a multiple of 16 B split the 16-byte reads; unpadded rows with the
// 16-byte chunks XOR-swizzled by the row: 15.97)
constexpr int LDR = KS + 16;

struct GemmP {
    // up to three stacked weight matrices sharing X (Q/K/V, gate/up): rows
    // [seg_end[s-1], seg_end[s]) come from segW[s] and go to segY[s] (row
    // stride segLdy[s]); segment sizes are multiples of the row tile
    uint32_t nseg;
    const uint8_t *segW[3];
    float *segY[3];
    uint32_t segLdy[3], seg_end[3];
    uint64_t row_bytes;
    const _Float16 *X;       // [N][ldx]
    const float *x_unscale;  // optional [N]: row n of X was stored times 1/x_unscale[n] (a power of two)
    uint32_t M, K, N, ldx, acc;
    // split-K (one segment only): workgroup z of ksplit takes K-steps
    // [z nst / ksplit, (z+1) nst / ksplit) and writes its f32 sums to
    // part[z][N][M]; k_gemm_reduce adds them up in order
    uint32_t ksplit;
    float *part;
};

// f32 -> fp16, round to nearest even, from the f32 value: the empty asm
// keeps the compiler from fusing the conversion into the producing
// multiply-add (v_fma_mix rounds the exact result to fp16 once, which
// differs from rounding the f32 value when that lands on an fp16 tie)
ZH_DEV _Float16 to_h(float v) {
    asm("" : "+v"(v));
    return (_Float16)v;
}

// Raw bytes of one dequantisation unit -- 32 elements of one weight row --
// loaded a K-step ahead.
struct RawQ4K {  // header 16 B + qs[32p .. 32p+31] of sub-pair p
    u32x4 hdr, q[2];
};
struct RawQ6K {  // dword-aligned covers of the 32 ql / 32 qh bytes of group g, the half's scales, d
    uint32_t ql[9], qh[9], sc[3], dw[2], sh;
};

ZH_DEV void load_q4k_unit(const uint8_t *blk, uint32_t p, RawQ4K &r) {
    r.hdr = *(const u32x4 *)blk;
    const u32x4 *q4 = (const u32x4 *)(blk + 16 + 32 * p);
    r.q[0] = q4[0];
    r.q[1] = q4[1];
}
// group g of half h: ql[64h + 32(g&1) .. +32], qh[32h .. +32], sc[8h .. 8h+8]
ZH_DEV void load_q6k_unit(const uint8_t *blk, uint32_t h, uint32_t g, RawQ6K &r) {
    const uintptr_t a = (uintptr_t)blk;
    r.sh = (uint32_t)(a & 3);
    const uint32_t *base = (const uint32_t *)(a & ~(uintptr_t)3);
#pragma unroll
    for (int i = 0; i < 9; i++) r.ql[i] = base[16 * h + 8 * (g & 1) + i];
#pragma unroll
    for (int i = 0; i < 9; i++) r.qh[i] = base[32 + 8 * h + i];
#pragma unroll
    for (int i = 0; i < 3; i++) r.sc[i] = base[48 + 2 * h + i];
    r.dw[0] = base[52];
    r.dw[1] = base[53];
}

// Q4_K sub-block j = 2p + nib (32 elements: nibble nib of qs[32p .. 32p+31])
// into LDS. dequantRow Q4_K (forward.zig:370-409): dj = d*sc[j],
// mj = dmin*m[j], out = dj*q - mj in f32, then to fp16 (nearest even). dj
// and mj (an 11-bit f16 times a 6-bit integer) and dj*q (times a 4-bit q)
// are exact in f32, so the f32 multiply-add the compiler forms rounds once,
// exactly where dequantRow's subtraction does; to_h then rounds that f32
// value.
ZH_DEV void deq_q4k_unit(const RawQ4K &r, uint32_t p, uint32_t nib, _Float16 *dst) {
    const uint32_t w0 = r.hdr.x, w1 = r.hdr.y, w2 = r.hdr.z, w3 = r.hdr.w;
    const float d = h2f(w0), dmin = h2f(w0 >> 16);
    const uint32_t scA = w1 & 0x3F3F3F3Fu, mA = w2 & 0x3F3F3F3Fu;
    const uint32_t scB = (w3 & 0x0F0F0F0Fu) | ((w1 >> 2) & 0x30303030u);
    const uint32_t mB = ((w3 >> 4) & 0x0F0F0F0Fu) | ((w2 >> 2) & 0x30303030u);
    const uint32_t j = 2 * p + nib;
    const uint32_t scw = p < 2 ? scA : scB, mw = p < 2 ? mA : mB;
    const float dj = __fmul_rn(d, (float)((scw >> (8 * (j & 3))) & 0xFF));
    const float mj = __fmul_rn(dmin, (float)((mw >> (8 * (j & 3))) & 0xFF));
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const u32x4 qv = r.q[c];
        const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
        half8 o[2];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            uint32_t n4 = (qw[w] >> (4 * nib)) & 0x0F0F0F0Fu;
            // (kept as one word: each element is then a byte conversion,
            // v_cvt_f32_ubyteN, instead of a bit-field extract and a
            // conversion)
            asm volatile("" : "+v"(n4));
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int e = 4 * w + b;
                o[e >> 3][e & 7] = to_h(__fsub_rn(__fmul_rn(dj, (float)((n4 >> (8 * b)) & 0xFF)), mj));
            }
        }
        *(half8 *)(dst + 16 * c) = o[0];
        *(half8 *)(dst + 16 * c + 8) = o[1];
    }
}

// Q6_K group g of half h (dequantRow Q6_K, forward.zig:276-325): element
// 128h + 32g + l: q6 = (ql[64h + l + 32(g&1)] >> 4(g>>1)) & 15 |
// ((qh[32h + l] >> 2g) & 3) << 4; out = (d * sc[8h + l/16 + 2g]) * (q6 - 32).
// The block may start 2-byte aligned: its bytes are realigned with alignbyte.
// Four 6-bit values are assembled per dword (masks on the packed bytes); each
// element is then one byte conversion and fma(ds, q6, -32 ds), which equals
// the rounded product ds * (q6 - 32) (-32 ds is exact), then fp16.
ZH_DEV void deq_q6k_unit(const RawQ6K &r, uint32_t g, _Float16 *dst) {
    const uint32_t sh = r.sh;
    const float d = h2f(__builtin_amdgcn_alignbyte(r.dw[1], r.dw[0], sh));
    const uint32_t s0 = __builtin_amdgcn_alignbyte(r.sc[1], r.sc[0], sh), s1 = __builtin_amdgcn_alignbyte(r.sc[2], r.sc[1], sh);
    const uint32_t i0 = 2 * g, i1 = 2 * g + 1;
    const float ds0 = __fmul_rn(d, (float)(int8_t)(((i0 < 4 ? s0 : s1) >> (8 * (i0 & 3))) & 0xFF));
    const float ds1 = __fmul_rn(d, (float)(int8_t)(((i1 < 4 ? s0 : s1) >> (8 * (i1 & 3))) & 0xFF));
    const uint32_t nsh = 4 * (g >> 1), hsh = 2 * g;
#pragma unroll
    for (int c = 0; c < 4; c++) {  // 8 elements l = 8c .. 8c+7
        const float ds = c < 2 ? ds0 : ds1, nb = -32.f * ds;
        uint32_t q[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t qlw = __builtin_amdgcn_alignbyte(r.ql[2 * c + h + 1], r.ql[2 * c + h], sh);
            const uint32_t qhw = __builtin_amdgcn_alignbyte(r.qh[2 * c + h + 1], r.qh[2 * c + h], sh);
            q[h] = ((qlw >> nsh) & 0x0F0F0F0Fu) | (((qhw >> hsh) & 0x03030303u) << 4);
        }
        half8 o;
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = to_h(fmaf(ds, (float)((q[e >> 2] >> (8 * (e & 3))) & 0xFF), nb));
        *(half8 *)(dst + 8 * c) = o;
    }
}

// Tile = TI tokens x TJ weight rows, K in steps of KS = half a super-block.
// Waves 2 x 2: wave (wi, wj) owns tokens 64 wi .. +63 and rows TJ/2 wj ..
// +TJ/2 (4 x TJ/32 MFMA tiles). Each step the threads dequantise the tile's
// TJ x 4 units of 32 elements (UPT per thread) into LDS while the X chunks
// of the next step and the raw weight bytes of the next two steps are in
// flight in registers. 74 KB of
// LDS (TJ = 128): two workgroups per CU, so one's dequantisation overlaps
// the other's MFMAs.
template <int QT, int TJ>
__global__ __launch_bounds__(GT, 2) void k_gemm(GemmP p) {
    extern __shared__ __align__(16) uint8_t lds[];
    _Float16 *xs = (_Float16 *)lds;       // [TI][LDR]
    _Float16 *ws = xs + TI * LDR;          // [TJ][LDR]
    constexpr int WJ = TJ / 2;             // weight rows per wave
    constexpr int NJ = WJ / 16, NI = 64 / 16;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t wi = wave & 1, wj = wave >> 1;
    const uint32_t n0 = blockIdx.y * TI;
    // segment of this row tile
    const uint32_t jg = blockIdx.x * TJ;
    const uint32_t sg = (jg >= p.seg_end[0] ? 1u : 0u) + (p.nseg > 2 && jg >= p.seg_end[1] ? 1u : 0u);
    const uint32_t seg_start = sg ? p.seg_end[sg - 1] : 0u, Ms = p.seg_end[sg] - seg_start;
    const uint32_t j0 = jg - seg_start;
    const uint8_t *Wseg = p.segW[sg];
    const uint32_t nst_all = p.K / KS, z = blockIdx.z;
    const uint32_t st_begin = z * nst_all / p.ksplit, nst = (z + 1) * nst_all / p.ksplit;
    const uint32_t bpb = QT == ZH_Q4_K ? 144 : 210;
    f32x4v acc[NI][NJ];
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};
    constexpr int XC = TI * KS / 8 / GT;  // 16-byte X chunks per thread per step
    constexpr int UPT = TJ * 4 / GT;      // units (row, 32-element group u4) per thread per step
    half8 xr[XC];
    typedef typename std::conditional<QT == ZH_Q4_K, RawQ4K, RawQ6K>::type Raw;
    // the raw weight bytes (HBM) are requested two K-steps ahead, in two
    // register sets with fixed roles (steps alternate between them, so no
    // register copy waits for bytes still in flight); X (L2-resident) one
    // step ahead
    Raw wa[UPT], wb[UPT];
    auto load_x = [&](uint32_t st) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < XC; c++) {
            const uint32_t idx = c * GT + tid, t = idx / (KS / 8), ch = idx % (KS / 8);
            const uint32_t tok = min(n0 + t, p.N - 1);
            xr[c] = *(const half8 *)(p.X + (size_t)tok * p.ldx + (size_t)st * KS + ch * 8);
        }
    };
    auto load_w = [&](uint32_t st, Raw (&wr)[UPT]) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < UPT; k++) {
            const uint32_t u = k * GT + tid, r = u >> 2, u4 = u & 3;
            const uint32_t row = min(j0 + r, Ms - 1);  // rows past the segment: loaded clamped, never written
            const uint8_t *blk = Wseg + (size_t)row * p.row_bytes + (size_t)(st >> 1) * bpb;
            if constexpr (QT == ZH_Q4_K) load_q4k_unit(blk, 2 * (st & 1) + (u4 >> 1), wr[k]);
            else load_q6k_unit(blk, st & 1, u4, wr[k]);
        }
    };
    // one K-step: X and the dequantised weights into LDS, the next loads,
    // the MFMAs
    auto step = [&](uint32_t st, Raw (&wr)[UPT]) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < XC; c++) {
            const uint32_t idx = c * GT + tid, t = idx / (KS / 8), ch = idx % (KS / 8);
            *(half8 *)(xs + t * LDR + ch * 8) = xr[c];
        }
#pragma unroll
        for (int k = 0; k < UPT; k++) {
            const uint32_t u = k * GT + tid, r = u >> 2, u4 = u & 3;
            // Q4_K: u4 = (sub-pair within the half, nibble) -> elements 32 u4 of the step
            if constexpr (QT == ZH_Q4_K) deq_q4k_unit(wr[k], 2 * (st & 1) + (u4 >> 1), u4 & 1, ws + r * LDR + 32 * u4);
            else deq_q6k_unit(wr[k], u4, ws + r * LDR + 32 * u4);
        }
        __syncthreads();
        // X first: a wave's loads complete in order, so waiting for this X
        // next step does not wait for the weight bytes requested after it
        if (st + 1 < nst) load_x(st + 1);
        if (st + 2 < nst) load_w(st + 2, wr);
#pragma unroll
        for (int kk = 0; kk < KS / 32; kk++) {
            const uint32_t ko = kk * 32 + 8 * (lane / 16);
            half8 b[NJ];
#pragma unroll
            for (int j = 0; j < NJ; j++) b[j] = *(const half8 *)(ws + (wj * WJ + j * 16 + lane % 16) * LDR + ko);
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const half8 a = *(const half8 *)(xs + (wi * 64 + i * 16 + lane % 16) * LDR + ko);
#pragma unroll
                for (int j = 0; j < NJ; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[j], acc[i][j], 0, 0, 0);
            }
        }
        __syncthreads();
    };
    load_w(st_begin, wa);
    if (st_begin + 1 < nst) load_w(st_begin + 1, wb);
    load_x(st_begin);
    for (uint32_t st = st_begin; st < nst; st += 2) {
        step(st, wa);
        if (st + 1 < nst) step(st + 1, wb);
    }
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const uint32_t row = j0 + wj * WJ + j * 16 + lane % 16;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t tok = n0 + wi * 64 + i * 16 + 4 * (lane / 16) + r;
                if (p.ksplit > 1) {
                    if (tok < p.N && row < Ms) p.part[((size_t)z * p.N + tok) * p.M + seg_start + row] = acc[i][j][r];
                } else if (tok < p.N && row < Ms) {
                    float *yp = p.segY[sg] + (size_t)tok * p.segLdy[sg] + row;
                    const float v = p.x_unscale ? acc[i][j][r] * p.x_unscale[tok] : acc[i][j][r];  // exact
                    *yp = p.acc ? *yp + v : v;
                }
            }
        }
}

// Split-K epilogue: Y[n][m] (+)= (sum over z of part[z][n][m]) * unscale[n],
// the partial sums added in split order.
__global__ __launch_bounds__(256) void k_gemm_reduce(const float *__restrict__ part, uint32_t ksplit, uint32_t N,
                                                     uint32_t M, float *__restrict__ Y, uint32_t ldy, uint32_t acc,
                                                     const float *__restrict__ x_unscale) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)N * M) return;
    const uint32_t n = (uint32_t)(i / M), m = (uint32_t)(i % M);
    float v = part[i];
    for (uint32_t z = 1; z < ksplit; z++) v += part[(size_t)z * N * M + i];
    if (x_unscale) v *= x_unscale[n];  // exact: a power of two
    float *yp = Y + (size_t)n * ldy + m;
    *yp = acc ? *yp + v : v;
}

// The same over stacked segments: column m of part goes to the segment
// holding row m.
__global__ __launch_bounds__(256) void k_gemm_reduce_seg(GemmP p) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (uint64_t)p.N * p.M) return;
    const uint32_t n = (uint32_t)(i / p.M), m = (uint32_t)(i % p.M);
    float v = p.part[i];
    for (uint32_t z = 1; z < p.ksplit; z++) v += p.part[(size_t)z * p.N * p.M + i];
    if (p.x_unscale) v *= p.x_unscale[n];  // exact: a power of two
    const uint32_t sg = (m >= p.seg_end[0] ? 1u : 0u) + (p.nseg > 2 && m >= p.seg_end[1] ? 1u : 0u);
    float *yp = p.segY[sg] + (size_t)n * p.segLdy[sg] + (m - (sg ? p.seg_end[sg - 1] : 0u));
    *yp = p.acc ? *yp + v : v;
}

// The split-K epilogue of the stacked q | k | v projection (acc 0, no
// unscale) fused with the q/k RMSNorm, RoPE and the KV-cache write of
// k_qk_norm_rope_kv (zh_ops.hip; cpuRmsNormMul + applyRope, the same f32
// operations in the same order), one workgroup per token: wave w takes
// heads w, w + 4, ... of the 40 (q, then k, then v), lane dims lane and
// lane + 64 (a RoPE pair).
__global__ __launch_bounds__(256) void k_reduce_qkv_rope(GemmP p, zh_gemm_rope r) {
    constexpr uint32_t HD = 128;
    const uint32_t n = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t pos = r.pos0 + n;
    const uint32_t slot = pos / 16;
    bool ok = slot < r.n_pages;
    const uint32_t phys = ok ? r.pages[slot] * 16 + pos % 16 : 0;
    ok = ok && phys < r.cache_tokens;
    const float *pn = p.part + (size_t)n * p.M;
    const size_t zs = (size_t)p.N * p.M;
    for (uint32_t hh = wave; hh < r.nq + 2 * r.nkv; hh += 4) {  // uniform per wave
        const uint32_t c0 = hh * HD;
        float a = pn[c0 + lane], b = pn[c0 + lane + 64];
        for (uint32_t z = 1; z < p.ksplit; z++) {
            a += pn[z * zs + c0 + lane];
            b += pn[z * zs + c0 + lane + 64];
        }
        if (hh < r.nq + r.nkv) {
            const bool is_q = hh < r.nq;
            const uint32_t head = is_q ? hh : hh - r.nq;
            float sq = 0.f;
            sq = fmaf(a, a, sq);
            sq = fmaf(b, b, sq);
            sq = wave_sum(sq);
            const float rms_inv = 1.0f / sqrtf(sq / (float)HD + r.eps);
            const float *wt = is_q ? r.q_norm : r.k_norm;
            const uint32_t i = lane;
            const float lo = wt[i] * (a * rms_inv);
            const float hi = wt[i + 64] * (b * rms_inv);
            const float th = (float)pos * r.inv_freq[i];
            float sn, co;
            sincosf(th, &sn, &co);
            const float rlo = lo * co - hi * sn;
            const float rhi = lo * sn + hi * co;
            if (is_q) {
                float *qo = p.segY[0] + (size_t)n * p.segLdy[0] + (size_t)head * HD;
                qo[i] = rlo;
                qo[i + 64] = rhi;
            } else if (ok) {
                uint16_t *kdst = r.kc + ((size_t)head * r.cache_tokens + phys) * HD;
                kdst[i] = f2h_rn(rlo);
                kdst[i + 64] = f2h_rn(rhi);
            }
        } else if (ok) {
            uint16_t *vdst = r.vc + ((size_t)(hh - r.nq - r.nkv) * r.cache_tokens + phys) * HD;
            vdst[lane] = f2h_rn(a);
            vdst[lane + 64] = f2h_rn(b);
        }
    }
}

// The same split-K epilogue fused with the RMSNorm the next GEMM takes as
// its input, one workgroup per token row (M <= 16384, M % 4 == 0, Y rows M
// apart): row n of Y (+)= (sum over z of part[z][n], in split order) *
// unscale[n], exactly as k_gemm_reduce, then out[n] = fp16(w * (y * rms_inv))
// with the sums of squares in k_rms_norm_rows_f16's order (cpuRmsNormMul,
// forward.zig:618-626).
constexpr int RN_RV = 16;
__global__ __launch_bounds__(256) void k_reduce_rms_rows_f16(const float *__restrict__ part, uint32_t ksplit,
                                                             uint32_t N, uint32_t M, float *__restrict__ Y,
                                                             uint32_t acc, const float *__restrict__ x_unscale,
                                                             const float *__restrict__ w, _Float16 *__restrict__ out,
                                                             float eps) {
    const uint32_t r = blockIdx.x, t = threadIdx.x;
    __shared__ float red[4];
    f32x4 v[RN_RV];
    float sq = 0.f;
    const float us = x_unscale ? x_unscale[r] : 1.0f;
#pragma unroll
    for (int j = 0; j < RN_RV; j++) {
        const uint32_t i = 4 * (t + 256 * j);
        if (i < M) {
            const size_t o = (size_t)r * M + i;
            f32x4 s = *(const f32x4 *)(part + o);
            for (uint32_t z = 1; z < ksplit; z++) {
                const f32x4 pz = *(const f32x4 *)(part + (size_t)z * N * M + o);
                s.x += pz.x; s.y += pz.y; s.z += pz.z; s.w += pz.w;
            }
            if (x_unscale) {  // exact: a power of two
                s.x *= us; s.y *= us; s.z *= us; s.w *= us;
            }
            f32x4 y = s;
            if (acc) {
                const f32x4 yo = *(const f32x4 *)(Y + o);
                y = f32x4{yo.x + s.x, yo.y + s.y, yo.z + s.z, yo.w + s.w};
            }
            *(f32x4 *)(Y + o) = y;
            v[j] = y;
        } else {
            v[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        sq = fmaf(v[j].x, v[j].x, fmaf(v[j].y, v[j].y, fmaf(v[j].z, v[j].z, fmaf(v[j].w, v[j].w, sq))));
    }
    sq = wave_sum(sq);
    if ((t & 63) == 0) red[t >> 6] = sq;
    __syncthreads();
    const float rms_inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)M + eps);
#pragma unroll
    for (int j = 0; j < RN_RV; j++) {
        const uint32_t i = 4 * (t + 256 * j);
        if (i < M) {
            const f32x4 wv = *(const f32x4 *)(w + i);
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            *(h4 *)(out + (size_t)r * M + i) =
                h4{(_Float16)(wv.x * (v[j].x * rms_inv)), (_Float16)(wv.y * (v[j].y * rms_inv)),
                   (_Float16)(wv.z * (v[j].z * rms_inv)), (_Float16)(wv.w * (v[j].w * rms_inv))};
        }
    }
}

}  // namespace

int zhk_gemm_multi(zh_ctx *c, uint32_t qtype, uint32_t nseg, const uint8_t *const *W, const _Float16 *X, uint32_t ldx,
                   float *const *Y, const uint32_t *ldy, const uint32_t *M, uint32_t K, uint32_t N, uint32_t acc,
                   const float *x_unscale, const float *norm_w, _Float16 *norm_out, float eps,
                   const zh_gemm_rope *rope) {
    if ((qtype != ZH_Q4_K && qtype != ZH_Q6_K) || K % 256 || N == 0 || nseg < 1 || nseg > 3)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "gemm: qtype %u K %u N %u nseg %u", qtype, K, N, nseg);
    GemmP p = {};
    if (norm_out && (nseg != 1 || !norm_w || ldy[0] != M[0] || M[0] % 4 || M[0] > 4u * 256u * RN_RV))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "gemm: fused norm needs one matrix of rows %u apart", M[0]);
    if (rope && (nseg != 3 || acc || x_unscale || M[0] != rope->nq * 128u || M[1] != rope->nkv * 128u ||
                 M[2] != rope->nkv * 128u || ldy[0] != M[0] || ldy[1] != M[1] || ldy[2] != M[2]))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "gemm: the q | k | v epilogue needs head_dim 128 rows");
    p.nseg = nseg; p.row_bytes = zh_tensor_bytes(qtype, 1, K); p.X = X; p.x_unscale = x_unscale;
    p.K = K; p.N = N; p.ldx = ldx; p.acc = acc;
    uint32_t end = 0;
    for (uint32_t s = 0; s < nseg; s++) {
        if (M[s] == 0) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "gemm: empty segment");
        p.segW[s] = W[s]; p.segY[s] = Y[s]; p.segLdy[s] = ldy[s];
        end += M[s];
        p.seg_end[s] = end;
    }
    for (uint32_t s = nseg; s < 3; s++) p.seg_end[s] = end;
    p.M = end;
    const uint32_t ni = (N + TI - 1) / TI;
    // 128-row tiles, K split when there are fewer tiles than two per CU
    // (below); 64-row tiles only where a segment boundary needs them (every
    // segment but the last is a whole number of tiles)
    bool small = zh_knob("ZH_GEMM_TJ64");
    for (uint32_t s = 0; s + 1 < nseg; s++)
        if (M[s] % 128) small = true;
    for (uint32_t s = 0; s + 1 < nseg; s++)
        if (M[s] % 64) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "gemm: segment rows %u not a multiple of 64", M[s]);
    const uint32_t TJv = small ? 64 : 128;
    const uint32_t lds = (TI + TJv) * LDR * 2;
    // Fewer tiles than two per CU (O, down, the stacked Q/K/V): split K so
    // two workgroups share each CU (one's dequantisation overlapping the
    // other's MFMAs), within one round of resident workgroups (rounding the
    // split up measured slower for Q/K/V: 576 workgroups for 512 slots); at
    // least 8 K-steps per split.
    const uint64_t tiles = (uint64_t)((end + TJv - 1) / TJv) * ni, slots = 2ull * (uint64_t)c->cu_count;
    p.ksplit = 1;
    if (tiles < slots && !zh_knob("ZH_NO_SPLITK")) {
        uint32_t sk = (uint32_t)(slots / tiles);
        while (sk > 1 && K / KS < 8 * sk) sk--;
        p.ksplit = sk;
    }
    if (p.ksplit > 1) {
        void *scr = nullptr;
        int rc = zh_scratch(c, 4ull * p.ksplit * N * end, &scr);
        if (rc) return rc;
        p.part = (float *)scr;
    }
    dim3 grid((end + TJv - 1) / TJv, ni, p.ksplit);
#define GL(Q, J) hipLaunchKernelGGL((k_gemm<Q, J>), grid, dim3(GT), lds, c->stream, p)
    if (qtype == ZH_Q4_K) { if (small) GL(ZH_Q4_K, 64); else GL(ZH_Q4_K, 128); }
    else { if (small) GL(ZH_Q6_K, 64); else GL(ZH_Q6_K, 128); }
#undef GL
    if (rope && p.ksplit > 1) {
        hipLaunchKernelGGL(k_reduce_qkv_rope, dim3(N), dim3(256), 0, c->stream, p, *rope);
        ZH_LAUNCH_CHECK(c);
        return ZH_OK;
    }
    if (rope) {  // (K not split: the sums are in Y already)
        ZH_LAUNCH_CHECK(c);
        return zhk_qk_norm_rope_kv(c, Y[0], rope->q_norm, Y[1], rope->k_norm, Y[2], rope->inv_freq, rope->kc, rope->vc,
                                   rope->pages, rope->n_pages, rope->cache_tokens, rope->nq, rope->nkv, 128,
                                   zh_pos_src{rope->pos0, nullptr}, rope->eps, N);
    }
    if (p.ksplit > 1 && norm_out) {
        hipLaunchKernelGGL(k_reduce_rms_rows_f16, dim3(N), dim3(256), 0, c->stream, p.part, p.ksplit, N, end, Y[0],
                           acc, x_unscale, norm_w, norm_out, eps);
    } else if (p.ksplit > 1 && nseg > 1) {
        const uint64_t n = (uint64_t)N * end;
        hipLaunchKernelGGL(k_gemm_reduce_seg, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, c->stream, p);
    } else if (p.ksplit > 1) {
        const uint64_t n = (uint64_t)N * end;
        hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, c->stream, p.part, p.ksplit,
                           N, end, Y[0], ldy[0], acc, x_unscale);
    } else if (norm_out) {
        ZH_LAUNCH_CHECK(c);
        return zhk_rms_norm_rows_f16(c, Y[0], norm_w, norm_out, end, N, eps);
    }
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

int zhk_gemm(zh_ctx *c, uint32_t qtype, const uint8_t *W, const _Float16 *X, uint32_t ldx, float *Y, uint32_t ldy,
             uint32_t M, uint32_t K, uint32_t N, uint32_t acc, const float *x_unscale) {
    return zhk_gemm_multi(c, qtype, 1, &W, X, ldx, &Y, &ldy, &M, K, N, acc, x_unscale);
}

int zhk_gemm_norm(zh_ctx *c, uint32_t qtype, const uint8_t *W, const _Float16 *X, uint32_t ldx, float *Y, uint32_t M,
                  uint32_t K, uint32_t N, uint32_t acc, const float *x_unscale, const float *norm_w,
                  _Float16 *norm_out, float eps) {
    return zhk_gemm_multi(c, qtype, 1, &W, X, ldx, &Y, &M, &M, K, N, acc, x_unscale, norm_w, norm_out, eps);
}

// Y[n][m] (+)= X[n][:] . W[m][:], X fp16 token-major, Y f32 token-major
// (dispatchProjectionBatched, forward.zig:8147-8216).
extern "C" int zh_gemm_xw(zh_ctx *c, uint32_t qtype, const zh_buf *W, uint64_t a_off, const zh_buf *X,
                          uint64_t x_off, zh_buf *Y, uint64_t y_off, uint32_t M, uint32_t K, uint32_t N,
                          uint32_t acc_mode) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (qtype != ZH_Q4_K && qtype != ZH_Q6_K)
        return zh_set_err(c, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "gemm qtype %u", qtype);
    if (K == 0 || K % 256 || M == 0 || N == 0 || (x_off & 15))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "gemm shape M %u K %u N %u / x_off alignment", M, K, N);
    if (!W || !X || !Y || a_off + zh_tensor_bytes(qtype, M, K) > W->size || x_off + 2ull * K * N > X->size ||
        y_off + 4ull * M * N > Y->size)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "gemm range");
    return zhk_gemm(c, qtype, (const uint8_t *)W->ptr + a_off, (const _Float16 *)((const char *)X->ptr + x_off), K,
                    (float *)((char *)Y->ptr + y_off), M, M, K, N, acc_mode, nullptr);
}

// ---------------------------------------------------------------------------
// Batched prefill support kernels (prefillBatched, forward.zig:9330-9735).
// ---------------------------------------------------------------------------
namespace {

// Row kernels: one workgroup per token row, the row held in registers
// between the reduction and the write (RV 16-byte chunks per thread cover
// n <= 1024 RV elements; n a multiple of 4).
constexpr int RV = 16;
typedef _Float16 half4 __attribute__((ext_vector_type(4)));

// RMSNorm of `rows` rows of n (cpuRmsNormMul, forward.zig:618-626:
// w[i] * (x[i] * (1/sqrt(sum x^2 / n + eps)))), written as fp16 GEMM input.
__global__ __launch_bounds__(256) void k_rms_norm_rows_f16(const float *__restrict__ x, const float *__restrict__ w,
                                                           _Float16 *__restrict__ out, uint32_t n, float eps) {
    const uint32_t r = blockIdx.x, t = threadIdx.x;
    const float *xr = x + (size_t)r * n;
    __shared__ float red[4];
    f32x4 v[RV];
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < RV; j++) {
        const uint32_t i = 4 * (t + 256 * j);
        v[j] = i < n ? *(const f32x4 *)(xr + i) : f32x4{0.f, 0.f, 0.f, 0.f};
        sq = fmaf(v[j].x, v[j].x, fmaf(v[j].y, v[j].y, fmaf(v[j].z, v[j].z, fmaf(v[j].w, v[j].w, sq))));
    }
    sq = wave_sum(sq);
    if ((t & 63) == 0) red[t >> 6] = sq;
    __syncthreads();
    const float rms_inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)n + eps);
#pragma unroll
    for (int j = 0; j < RV; j++) {
        const uint32_t i = 4 * (t + 256 * j);
        if (i < n) {
            const f32x4 wv = *(const f32x4 *)(w + i);
            *(half4 *)(out + (size_t)r * n + i) =
                half4{(_Float16)(wv.x * (v[j].x * rms_inv)), (_Float16)(wv.y * (v[j].y * rms_inv)),
                      (_Float16)(wv.z * (v[j].z * rms_inv)), (_Float16)(wv.w * (v[j].w * rms_inv))};
        }
    }
}

// SwiGLU (cpuSwiGLU, forward_metal.zig:6567-6572), one row per workgroup, to
// fp16 with a per-row power-of-two scale: the row maximum maps into
// [2^14, 2^15) so no value overflows fp16 and small rows keep 11 bits;
// unscale[row] = 1/scale multiplies the GEMM result back exactly.
ZH_DEV float silu_mul_f(float g, float u) { return (g / (1.0f + expf(-g))) * u; }
__global__ __launch_bounds__(256) void k_swiglu_rows_f16(const float *__restrict__ g, const float *__restrict__ u,
                                                         _Float16 *__restrict__ out, float *__restrict__ unscale,
                                                         uint32_t n) {
    const uint32_t r = blockIdx.x, t = threadIdx.x;
    const float *gr = g + (size_t)r * n, *ur = u + (size_t)r * n;
    __shared__ float red[4];
    f32x4 v[RV];
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < RV; j++) {
        const uint32_t i = 4 * (t + 256 * j);
        if (i < n) {
            const f32x4 gv = *(const f32x4 *)(gr + i), uv = *(const f32x4 *)(ur + i);
            v[j] = f32x4{silu_mul_f(gv.x, uv.x), silu_mul_f(gv.y, uv.y), silu_mul_f(gv.z, uv.z), silu_mul_f(gv.w, uv.w)};
        } else {
            v[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    }
    mx = wave_max(mx);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // scale = 2^(14 - E) with mx = m * 2^E, m in [1, 2); mx == 0 (or not finite) -> 1
    int E = 0;
    if (mx > 0.f && mx < INFINITY) E = (int)((__float_as_uint(mx) >> 23) & 0xFF) - 127;
    E = max(-100, min(E, 100));
    const float sc = ldexpf(1.0f, 14 - E), inv = ldexpf(1.0f, E - 14);
    if (t == 0) unscale[r] = (mx > 0.f && mx < INFINITY) ? inv : 1.0f;
    const float s2 = (mx > 0.f && mx < INFINITY) ? sc : 1.0f;
#pragma unroll
    for (int j = 0; j < RV; j++) {
        const uint32_t i = 4 * (t + 256 * j);
        if (i < n)
            *(half4 *)(out + (size_t)r * n + i) =
                half4{(_Float16)(v[j].x * s2), (_Float16)(v[j].y * s2), (_Float16)(v[j].z * s2), (_Float16)(v[j].w * s2)};
    }
}

// Causal prefill attention on the MFMA units (flash attention): workgroup =
// one q head x AQ = 64 queries (16 per wave), key blocks of AK = 64 staged in
// LDS (K row-major, V transposed to [d][key]). Per block each wave computes
// S = Q K^T (16 x 64, v_mfma_f32_16x16x32_f16 over d), scales and masks it,
// updates the running row maximum and sum (online softmax, f32), writes
// P = exp(S - m) as fp16 to its own LDS tile (the D layout of S holds 4 rows
// per lane; the A layout of the next product holds 8 keys of one row) and
// accumulates O += P V (16 x 128). Q, K, V and P are fp16 operands with f32
// accumulation. Query tiles run longest first (causal: tile t sees t + 1
// blocks).
constexpr int AQ = 64, AK = 64;
constexpr int AKLD = 128 + 8;  // halfs per K row (272 B)
constexpr int AVLD = AK + 8;   // halfs per P row (144 B)
// V transposed, [d][key] with 64 keys per row (128 B, no padding): the 16-byte
// chunk of keys 8c .. 8c + 7 of row d sits at chunk c ^ ((d / 8) % 8), so the
// 16 lanes that store one key's 16 chunks of dims (2-byte stores) spread over
// 8 bank groups instead of one, and a B fragment is still one 16-byte read
ZH_DEV uint32_t vt_at(uint32_t d, uint32_t key) { return d * AK + ((((key >> 3) ^ (d >> 3)) & 7) << 3) + (key & 7); }
__global__ __launch_bounds__(256) void k_attn_prefill_mfma(const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                                           const uint16_t *__restrict__ vc,
                                                           const uint32_t *__restrict__ pages, uint32_t n_pages,
                                                           uint32_t cache_tokens, uint32_t nq, uint32_t nkv,
                                                           uint32_t pos0, uint32_t N, float scale,
                                                           _Float16 *__restrict__ out) {
    constexpr int HD = 128;
    __shared__ __align__(16) _Float16 ks[AK * AKLD];
    __shared__ __align__(16) uint16_t vt[HD * AK];
    __shared__ __align__(16) _Float16 pl[4][16 * AVLD];
    const uint32_t h = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t i0 = (gridDim.y - 1 - blockIdx.y) * AQ;  // longest tiles first
    const uint32_t kvh = h / (nq / nkv), li = lane % 16, lg = lane / 16;
    const uint16_t *kh = kc + (size_t)kvh * cache_tokens * HD;
    const uint16_t *vh = vc + (size_t)kvh * cache_tokens * HD;
    // Q fragments (A operand): row i0 + 16 wave + li, d = 32 ks + 8 lg .. +7
    half8 qa[4];
    {
        const float *qp = q + (size_t)min(i0 + 16 * wave + li, N - 1) * nq * HD + (size_t)h * HD + 8 * lg;
#pragma unroll
        for (int k4 = 0; k4 < 4; k4++) {
            const f32x4 a = *(const f32x4 *)(qp + 32 * k4), b = *(const f32x4 *)(qp + 32 * k4 + 4);
            qa[k4] = half8{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                           (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
        }
    }
    f32x4v o[8];
#pragma unroll
    for (int db = 0; db < 8; db++) o[db] = f32x4v{0.f, 0.f, 0.f, 0.f};
    float m[4], l[4];
#pragma unroll
    for (int r = 0; r < 4; r++) { m[r] = -INFINITY; l[r] = 0.f; }
    const uint32_t kmax = pos0 + min(i0 + AQ, N) - 1;  // last key any query of the workgroup sees
    const uint32_t qpos = pos0 + i0 + 16 * wave + 4 * lg;  // position of this lane's row r = 0
    _Float16 *pw = pl[wave];
    // the key block's K and V chunks (16 B of one key each: 4 per thread)
    // wait in registers, requested while the previous block computes; rows
    // past kmax are loaded clamped and masked below
    u32x4 pk[4], pv[4];
    auto load_kv = [&](uint32_t kb) __attribute__((always_inline)) {
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const uint32_t c = tid + 256 * it, key = c / 16, ch = c % 16, t = min(kb * AK + key, kmax);
            uint32_t ph = pages[min(t / 16, n_pages - 1)] * 16 + t % 16;
            ph = ph < cache_tokens ? ph : 0u;
            pk[it] = *(const u32x4 *)(kh + (size_t)ph * HD + ch * 8);
            pv[it] = *(const u32x4 *)(vh + (size_t)ph * HD + ch * 8);
        }
    };
    load_kv(0);
    for (uint32_t kb = 0; kb * AK <= kmax; kb++) {
        // stage the key block: K rows as they are, V transposed
#pragma unroll
        for (int it = 0; it < 4; it++) {
            const uint32_t c = tid + 256 * it, key = c / 16, ch = c % 16;
            *(u32x4 *)(ks + key * AKLD + ch * 8) = pk[it];
            const uint32_t w[4] = {pv[it].x, pv[it].y, pv[it].z, pv[it].w};
#pragma unroll
            for (int e = 0; e < 8; e++) vt[vt_at(ch * 8 + e, key)] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
        }
        __syncthreads();
        if ((kb + 1) * AK <= kmax) load_kv(kb + 1);
        f32x4v sc[4];
#pragma unroll
        for (int jb = 0; jb < 4; jb++) {
            sc[jb] = f32x4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k4 = 0; k4 < 4; k4++) {
                const half8 b = *(const half8 *)(ks + (16 * jb + li) * AKLD + 32 * k4 + 8 * lg);
                sc[jb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[k4], b, sc[jb], 0, 0, 0);
            }
        }
        float mb[4], f[4], ls[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            mb[r] = -INFINITY;
#pragma unroll
            for (int jb = 0; jb < 4; jb++) {
                const uint32_t key = kb * AK + 16 * jb + li;
                const float v = key <= qpos + r ? sc[jb][r] * scale : -INFINITY;
                sc[jb][r] = v;
                mb[r] = fmaxf(mb[r], v);
            }
            // block 0 holds key 0, visible to every row: m is finite from then on
            const float mn = fmaxf(m[r], row16_max(mb[r]));
            f[r] = expf(m[r] - mn);
            m[r] = mn;
            ls[r] = 0.f;
        }
#pragma unroll
        for (int jb = 0; jb < 4; jb++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = expf(sc[jb][r] - m[r]);
                ls[r] += p;
                pw[(4 * lg + r) * AVLD + 16 * jb + li] = (_Float16)p;
            }
#pragma unroll
        for (int r = 0; r < 4; r++) l[r] = fmaf(l[r], f[r], row16_sum(ls[r]));
#pragma unroll
        for (int db = 0; db < 8; db++)
#pragma unroll
            for (int r = 0; r < 4; r++) o[db][r] *= f[r];
        // the wave reads back its own P tile (LDS operations of a wave complete in order)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int k2 = 0; k2 < 2; k2++) {
            const half8 a = *(const half8 *)(pw + li * AVLD + 32 * k2 + 8 * lg);
#pragma unroll
            for (int db = 0; db < 8; db++) {
                const half8 b = *(const half8 *)(vt + vt_at(16 * db + li, 32 * k2 + 8 * lg));
                o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, o[db], 0, 0, 0);
            }
        }
        __syncthreads();  // the block's K / V tiles are rewritten next
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint32_t i = i0 + 16 * wave + 4 * lg + r;
        if (i < N) {
            const float inv = 1.0f / l[r];
            _Float16 *op = out + (size_t)i * nq * HD + (size_t)h * HD + li;
#pragma unroll
            for (int db = 0; db < 8; db++) op[16 * db] = (_Float16)(o[db][r] * inv);
        }
    }
}

}  // namespace

int zhk_rms_norm_rows_f16(zh_ctx *c, const float *x, const float *w, _Float16 *out, uint32_t n, uint32_t rows,
                          float eps) {
    if (n % 4 || n > 1024u * RV) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "rms_norm_rows n %u", n);
    hipLaunchKernelGGL(k_rms_norm_rows_f16, dim3(rows), dim3(256), 0, c->stream, x, w, out, n, eps);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
int zhk_swiglu_rows_f16(zh_ctx *c, const float *g, const float *u, _Float16 *out, float *unscale, uint32_t n,
                        uint32_t rows) {
    if (n % 4 || n > 1024u * RV) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "swiglu_rows n %u", n);
    hipLaunchKernelGGL(k_swiglu_rows_f16, dim3(rows), dim3(256), 0, c->stream, g, u, out, unscale, n);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
int zhk_attn_prefill(zh_ctx *c, const float *q, const uint16_t *kc, const uint16_t *vc, const uint32_t *pages,
                     uint32_t n_pages, uint32_t cache_tokens, uint32_t nq, uint32_t nkv, uint32_t hd, uint32_t pos0,
                     uint32_t N, float scale, _Float16 *out) {
    if (hd != 128 || nkv == 0 || nq % nkv) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "attn_prefill heads");
    hipLaunchKernelGGL(k_attn_prefill_mfma, dim3(nq, (N + AQ - 1) / AQ), dim3(256), 0, c->stream, q, kc, vc, pages,
                       n_pages, cache_tokens, nq, nkv, pos0, N, scale, out);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

// recordFlashAttnBatched (attention.zig:240-316) over caller buffers.
extern "C" int zh_flash_attn_batched(zh_ctx *c, const zh_buf *q, const zh_buf *kc, const zh_buf *vc,
                                     const zh_buf *pages, uint32_t n_pages, uint32_t cache_tokens, zh_buf *out,
                                     uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t seq_start, uint32_t nq_tok,
                                     float attn_scale) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (!q || !kc || !vc || !pages || !out || hd != 128 || nkv == 0 || nh % nkv || nq_tok == 0)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "flash_attn_batched: heads %u/%u head_dim %u n %u", nh, nkv, hd,
                          nq_tok);
    if ((uint64_t)seq_start + nq_tok > 16ull * n_pages)
        return zh_set_err(c, ZH_ERR_CONTEXT_LENGTH_EXCEEDED, "positions %u + %u", seq_start, nq_tok);
    const uint64_t row = (uint64_t)nh * hd;
    if (4ull * row * nq_tok > q->size || 2ull * row * nq_tok > out->size ||
        2ull * nkv * cache_tokens * hd > kc->size || 2ull * nkv * cache_tokens * hd > vc->size ||
        4ull * n_pages > pages->size)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "flash_attn_batched range");
    const float scale = attn_scale != 0.f ? attn_scale : 1.0f / sqrtf((float)hd);
    return zhk_attn_prefill(c, (const float *)q->ptr, (const uint16_t *)kc->ptr, (const uint16_t *)vc->ptr,
                            (const uint32_t *)pages->ptr, n_pages, cache_tokens, nh, nkv, hd, seq_start, nq_tok, scale,
                            (_Float16 *)out->ptr);
}
