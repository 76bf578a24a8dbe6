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
constexpr int KS = 256;         // k per step: one super-block
constexpr int LDR = KS + 8;     // halfs per LDS row (528 B: conflict-free 16 B reads)

struct GemmP {
    const uint8_t *W;
    uint64_t row_bytes;
    const _Float16 *X;       // [N][ldx]
    const float *x_unscale;  // optional [N]: row n of X was stored times 1/x_unscale[n] (a power of two)
    float *Y;                // [N][ldy]
    uint32_t M, K, N, ldx, ldy, acc;
};

ZH_DEV _Float16 to_h(float v) { return (_Float16)v; }  // round to nearest even

// Raw bytes of one row's half super-block, loaded a K-step ahead.
struct RawQ4K {  // header 16 B + qs[64h .. 64h+63]
    u32x4 hdr, q[4];
};
struct RawQ6K {  // dword-aligned cover of ql[64h..+64], qh[32h..+32], sc[8h..+8], d
    uint32_t ql[17], qh[9], sc[3], dw[2], sh;
};

ZH_DEV void load_q4k_half(const uint8_t *blk, uint32_t h, RawQ4K &r) {
    r.hdr = *(const u32x4 *)blk;
    const u32x4 *q4 = (const u32x4 *)(blk + 16 + 64 * h);
#pragma unroll
    for (int c = 0; c < 4; c++) r.q[c] = q4[c];
}
ZH_DEV void load_q6k_half(const uint8_t *blk, uint32_t h, RawQ6K &r) {
    const uintptr_t a = (uintptr_t)blk;
    r.sh = (uint32_t)(a & 3);
    const uint32_t *base = (const uint32_t *)(a & ~(uintptr_t)3);
#pragma unroll
    for (int i = 0; i < 17; i++) r.ql[i] = base[16 * h + i];
#pragma unroll
    for (int i = 0; i < 9; i++) r.qh[i] = base[32 + 8 * h + i];
#pragma unroll
    for (int i = 0; i < 3; i++) r.sc[i] = base[48 + 2 * h + i];
    r.dw[0] = base[52];
    r.dw[1] = base[53];
}

// Q4_K half super-block h (elements 128h..128h+127) into LDS.
// dequantRow Q4_K (forward.zig:370-409): sub-pair p, d1 = d*sc[2p],
// m1 = dmin*m[2p]: out[64p+l] = d1*(q&15) - m1, out[64p+32+l] = d2*(q>>4) - m2;
// f32 operations rounded one by one (no contraction), then to fp16.
ZH_DEV void deq_q4k_half(const RawQ4K &r, uint32_t h, _Float16 *dst) {
    const uint32_t w0 = r.hdr.x, w1 = r.hdr.y, w2 = r.hdr.z, w3 = r.hdr.w;
    const float d = h2f(w0), dmin = h2f(w0 >> 16);
    const uint32_t scA = w1 & 0x3F3F3F3Fu, mA = w2 & 0x3F3F3F3Fu;
    const uint32_t scB = (w3 & 0x0F0F0F0Fu) | ((w1 >> 2) & 0x30303030u);
    const uint32_t mB = ((w3 >> 4) & 0x0F0F0F0Fu) | ((w2 >> 2) & 0x30303030u);
#pragma unroll
    for (int pp = 0; pp < 2; pp++) {
        const uint32_t p = 2 * h + pp;  // sub-pair
        const uint32_t j0 = 2 * p, j1 = 2 * p + 1;
        const uint32_t scw = p < 2 ? scA : scB, mw = p < 2 ? mA : mB;
        const float d1 = __fmul_rn(d, (float)((scw >> (8 * (j0 & 3))) & 0xFF));
        const float m1 = __fmul_rn(dmin, (float)((mw >> (8 * (j0 & 3))) & 0xFF));
        const float d2 = __fmul_rn(d, (float)((scw >> (8 * (j1 & 3))) & 0xFF));
        const float m2 = __fmul_rn(dmin, (float)((mw >> (8 * (j1 & 3))) & 0xFF));
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const u32x4 qv = r.q[2 * pp + c];
            const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
            half8 lo[2], hi[2];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const uint32_t byte = (qw[e >> 2] >> (8 * (e & 3))) & 0xFF;
                lo[e >> 3][e & 7] = to_h(__fsub_rn(__fmul_rn(d1, (float)(byte & 15)), m1));
                hi[e >> 3][e & 7] = to_h(__fsub_rn(__fmul_rn(d2, (float)(byte >> 4)), m2));
            }
            // elements 64p + 16c + 0..15 (low nibbles), 64p + 32 + 16c + 0..15 (high)
            *(half8 *)(dst + 64 * pp + 16 * c) = lo[0];
            *(half8 *)(dst + 64 * pp + 16 * c + 8) = lo[1];
            *(half8 *)(dst + 64 * pp + 32 + 16 * c) = hi[0];
            *(half8 *)(dst + 64 * pp + 32 + 16 * c + 8) = hi[1];
        }
    }
}

// Q6_K half super-block h (dequantRow Q6_K, forward.zig:276-325): element
// 128h + 32g + l: q = (ql[64h + l + 32(g&1)] >> 4(g>>1)) & 15 |
// ((qh[32h + l] >> 2g) & 3) << 4; out = (d * sc[8h + l/16 + 2g]) * (q - 32).
// The block may start 2-byte aligned: its bytes are realigned with alignbyte.
ZH_DEV void deq_q6k_half(const RawQ6K &r, _Float16 *dst) {
    const uint32_t sh = r.sh;
    const float d = h2f(__builtin_amdgcn_alignbyte(r.dw[1], r.dw[0], sh));
    const uint32_t s0 = __builtin_amdgcn_alignbyte(r.sc[1], r.sc[0], sh), s1 = __builtin_amdgcn_alignbyte(r.sc[2], r.sc[1], sh);
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const float ds0 = __fmul_rn(d, (float)(int8_t)((((2 * g) < 4 ? s0 : s1) >> (8 * ((2 * g) & 3))) & 0xFF));
        const float ds1 = __fmul_rn(d, (float)(int8_t)((((2 * g + 1) < 4 ? s0 : s1) >> (8 * ((2 * g + 1) & 3))) & 0xFF));
#pragma unroll
        for (int c = 0; c < 4; c++) {  // 8 elements l = 8c .. 8c+7
            const uint32_t qlw0 = __builtin_amdgcn_alignbyte(r.ql[(g & 1) * 8 + 2 * c + 1], r.ql[(g & 1) * 8 + 2 * c], sh);
            const uint32_t qlw1 = __builtin_amdgcn_alignbyte(r.ql[(g & 1) * 8 + 2 * c + 2], r.ql[(g & 1) * 8 + 2 * c + 1], sh);
            const uint32_t qhw0 = __builtin_amdgcn_alignbyte(r.qh[2 * c + 1], r.qh[2 * c], sh);
            const uint32_t qhw1 = __builtin_amdgcn_alignbyte(r.qh[2 * c + 2], r.qh[2 * c + 1], sh);
            half8 o;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t lb = ((e < 4 ? qlw0 : qlw1) >> (8 * (e & 3))) & 0xFF;
                const uint32_t hb = ((e < 4 ? qhw0 : qhw1) >> (8 * (e & 3))) & 0xFF;
                const int q = (int)(((lb >> (4 * (g >> 1))) & 15) | (((hb >> (2 * g)) & 3) << 4));
                o[e] = to_h(__fmul_rn(c < 2 ? ds0 : ds1, (float)(q - 32)));
            }
            *(half8 *)(dst + 32 * g + 8 * c) = o;
        }
    }
}

template <int QT, int TJ>
__global__ __launch_bounds__(GT, 1) void k_gemm(GemmP p) {
    extern __shared__ __align__(16) uint8_t lds[];
    _Float16 *xs = (_Float16 *)lds;       // [TI][LDR]
    _Float16 *ws = xs + TI * LDR;          // [TJ][LDR]
    constexpr int JW = TJ / 4;             // weight rows per wave
    constexpr int NJ = JW / 16, NI = TI / 16;
    const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t j0 = blockIdx.x * TJ, n0 = blockIdx.y * TI;
    const uint32_t nb = p.K / KS;
    const uint32_t bpb = QT == ZH_Q4_K ? 144 : 210;
    f32x4v acc[NI][NJ];
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = f32x4v{0.f, 0.f, 0.f, 0.f};
    // Software pipeline: the next K-step's X chunks and raw weight bytes are
    // loaded into registers while the current step's MFMAs run.
    constexpr int XC = TI * 32 / GT;          // 16-byte X chunks per thread per step
    constexpr int WU = (TJ * 2 + GT - 1) / GT;  // (row, half) units per thread
    half8 xr[XC];
    typedef typename std::conditional<QT == ZH_Q4_K, RawQ4K, RawQ6K>::type Raw;
    Raw wr[WU];
    auto load_step = [&](uint32_t sb) {
#pragma unroll
        for (int c = 0; c < XC; c++) {
            const uint32_t idx = c * GT + tid, t = idx / 32, ch = idx % 32;
            const uint32_t tok = min(n0 + t, p.N - 1);
            xr[c] = *(const half8 *)(p.X + (size_t)tok * p.ldx + (size_t)sb * KS + ch * 8);
        }
#pragma unroll
        for (int w = 0; w < WU; w++) {
            const uint32_t u = min(w * GT + tid, (uint32_t)TJ * 2 - 1), r = u >> 1, h = u & 1;
            const uint32_t row = min(j0 + r, p.M - 1);
            const uint8_t *blk = p.W + (size_t)row * p.row_bytes + (size_t)sb * bpb;
            if constexpr (QT == ZH_Q4_K) load_q4k_half(blk, h, wr[w]);
            else load_q6k_half(blk, h, wr[w]);
        }
    };
    load_step(0);
    for (uint32_t sb = 0; sb < nb; sb++) {
#pragma unroll
        for (int c = 0; c < XC; c++) {
            const uint32_t idx = c * GT + tid, t = idx / 32, ch = idx % 32;
            *(half8 *)(xs + t * LDR + ch * 8) = xr[c];
        }
#pragma unroll
        for (int w = 0; w < WU; w++) {
            const uint32_t u = w * GT + tid;
            if (u < (uint32_t)TJ * 2) {
                const uint32_t r = u >> 1, h = u & 1;
                if constexpr (QT == ZH_Q4_K) deq_q4k_half(wr[w], h, ws + r * LDR + 128 * h);
                else deq_q6k_half(wr[w], ws + r * LDR + 128 * h);
            }
        }
        __syncthreads();
        if (sb + 1 < nb) load_step(sb + 1);
#pragma unroll
        for (int kk = 0; kk < KS / 32; kk++) {
            const uint32_t ko = kk * 32 + 8 * (lane / 16);
            half8 b[NJ];
#pragma unroll
            for (int j = 0; j < NJ; j++) b[j] = *(const half8 *)(ws + (wave * JW + j * 16 + lane % 16) * LDR + ko);
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const half8 a = *(const half8 *)(xs + (i * 16 + lane % 16) * LDR + ko);
#pragma unroll
                for (int j = 0; j < NJ; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[j], acc[i][j], 0, 0, 0);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const uint32_t row = j0 + wave * JW + j * 16 + lane % 16;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t tok = n0 + i * 16 + 4 * (lane / 16) + r;
                if (tok < p.N && row < p.M) {
                    float *yp = p.Y + (size_t)tok * p.ldy + row;
                    const float v = p.x_unscale ? acc[i][j][r] * p.x_unscale[tok] : acc[i][j][r];  // exact
                    *yp = p.acc ? *yp + v : v;
                }
            }
        }
}

}  // namespace

int zhk_gemm(zh_ctx *c, uint32_t qtype, const uint8_t *W, const _Float16 *X, uint32_t ldx, float *Y, uint32_t ldy,
             uint32_t M, uint32_t K, uint32_t N, uint32_t acc, const float *x_unscale) {
    if ((qtype != ZH_Q4_K && qtype != ZH_Q6_K) || K % KS || M == 0 || N == 0)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "gemm: qtype %u M %u K %u N %u", qtype, M, K, N);
    GemmP p;
    p.W = W; p.row_bytes = zh_tensor_bytes(qtype, 1, K); p.X = X; p.x_unscale = x_unscale; p.Y = Y;
    p.M = M; p.K = K; p.N = N; p.ldx = ldx; p.ldy = ldy; p.acc = acc;
    const uint32_t ni = (N + TI - 1) / TI;
    // 64-row tiles when 128-row tiles would leave CUs idle
    const bool small = (uint64_t)((M + 127) / 128) * ni < (uint64_t)c->cu_count;
    const uint32_t TJv = small ? 64 : 128;
    const uint32_t lds = (TI + TJv) * LDR * 2;
    dim3 grid((M + TJv - 1) / TJv, ni);
#define GL(Q, J) hipLaunchKernelGGL((k_gemm<Q, J>), grid, dim3(GT), lds, c->stream, p)
    if (qtype == ZH_Q4_K) { if (small) GL(ZH_Q4_K, 64); else GL(ZH_Q4_K, 128); }
    else { if (small) GL(ZH_Q6_K, 64); else GL(ZH_Q6_K, 128); }
#undef GL
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
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

// RMSNorm of `rows` rows of n (cpuRmsNormMul, forward.zig:618-626:
// w[i] * (x[i] * (1/sqrt(sum x^2 / n + eps)))), written as fp16 GEMM input.
__global__ __launch_bounds__(256) void k_rms_norm_rows_f16(const float *__restrict__ x, const float *__restrict__ w,
                                                           _Float16 *__restrict__ out, uint32_t n, float eps) {
    const uint32_t r = blockIdx.x, t = threadIdx.x;
    const float *xr = x + (size_t)r * n;
    __shared__ float red[4];
    float sq = 0.f;
    for (uint32_t i = t; i < n; i += 256) sq = fmaf(xr[i], xr[i], sq);
    sq = wave_sum(sq);
    if ((t & 63) == 0) red[t >> 6] = sq;
    __syncthreads();
    const float rms_inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)n + eps);
    for (uint32_t i = t; i < n; i += 256) out[(size_t)r * n + i] = (_Float16)(w[i] * (xr[i] * rms_inv));
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
    float mx = 0.f;
    for (uint32_t i = t; i < n; i += 256) mx = fmaxf(mx, fabsf(silu_mul_f(gr[i], ur[i])));
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
    for (uint32_t i = t; i < n; i += 256) out[(size_t)r * n + i] = (_Float16)(silu_mul_f(gr[i], ur[i]) * s2);
}

// Causal attention for a batch of queries (flash_attn_batched.comp; per query
// the arithmetic of cpuAttention, forward_metal.zig:6600-6646: score =
// dot(q, k) * scale, softmax, P * V). Workgroup = (q head, 16 queries): wave w
// owns queries 4w..4w+3; keys go 64 per chunk (lane = key) with an online
// softmax; P * V with lane = 2 output dims. Query i sits at position pos0 + i
// and sees keys 0..pos0+i of the paged fp16 cache. Output fp16 [N][nq*128].
constexpr int AP_Q = 16;
__global__ __launch_bounds__(256) void k_attn_prefill(const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                                      const uint16_t *__restrict__ vc, const uint32_t *__restrict__ pages,
                                                      uint32_t n_pages, uint32_t cache_tokens, uint32_t nq, uint32_t nkv,
                                                      uint32_t pos0, uint32_t N, float scale, _Float16 *__restrict__ out) {
    constexpr int HD = 128;
    const uint32_t h = blockIdx.x, i0 = blockIdx.y * AP_Q, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t kvh = h / (nq / nkv);
    __shared__ float qs[AP_Q][HD];
    __shared__ float ps[4][4][64];
    for (uint32_t e = tid; e < AP_Q * HD; e += 256) {
        const uint32_t qi = e / HD, d = e % HD;
        qs[qi][d] = q[(size_t)min(i0 + qi, N - 1) * nq * HD + (size_t)h * HD + d];
    }
    __syncthreads();
    const uint16_t *kh = kc + (size_t)kvh * cache_tokens * HD;
    const uint16_t *vh = vc + (size_t)kvh * cache_tokens * HD;
    const uint32_t kmax = pos0 + min(i0 + AP_Q, N) - 1;  // last key any query of the workgroup sees
    float m[4], l[4], acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; a++) { m[a] = -INFINITY; l[a] = 0.f; acc[a][0] = acc[a][1] = 0.f; }
    for (uint32_t c0 = 0; c0 <= kmax; c0 += 64) {
        const uint32_t t = min(c0 + lane, kmax);
        const uint32_t pg = min(t / 16, n_pages - 1);
        uint32_t ph = pages[pg] * 16 + t % 16;
        ph = ph < cache_tokens ? ph : 0u;
        const u32x4 *kr = (const u32x4 *)(kh + (size_t)ph * HD);
        float s[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
        for (int c = 0; c < HD / 8; c++) {
            const u32x4 kv = kr[c];
            const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float kf = h2f(kw[e >> 1] >> (16 * (e & 1)));
#pragma unroll
                for (int a = 0; a < 4; a++) s[a] = fmaf(qs[4 * wave + a][8 * c + e], kf, s[a]);
            }
        }
#pragma unroll
        for (int a = 0; a < 4; a++) {
            const uint32_t qpos = pos0 + i0 + 4 * wave + a;
            const float sv = (c0 + lane <= qpos) ? s[a] * scale : -INFINITY;
            const float mn = fmaxf(m[a], wave_max(sv));  // finite: key 0 is always visible
            const float pr = expf(sv - mn), f = expf(m[a] - mn);
            l[a] = fmaf(l[a], f, wave_sum(pr));
            acc[a][0] *= f;
            acc[a][1] *= f;
            m[a] = mn;
            ps[wave][a][lane] = pr;
        }
        // the wave's own LDS writes are visible to it after the wait the compiler inserts
        const uint32_t nk = min(64u, kmax + 1 - c0);
        for (uint32_t j = 0; j < nk; j++) {
            const uint32_t tj = c0 + j;
            const uint32_t pgj = min(tj / 16, n_pages - 1);
            uint32_t phj = pages[pgj] * 16 + tj % 16;
            phj = phj < cache_tokens ? phj : 0u;
            const uint32_t vv = *(const uint32_t *)(vh + (size_t)phj * HD + 2 * lane);
            const float v0 = h2f(vv), v1 = h2f(vv >> 16);
#pragma unroll
            for (int a = 0; a < 4; a++) {
                acc[a][0] = fmaf(ps[wave][a][j], v0, acc[a][0]);
                acc[a][1] = fmaf(ps[wave][a][j], v1, acc[a][1]);
            }
        }
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const uint32_t i = i0 + 4 * wave + a;
        if (i < N) {
            _Float16 *o = out + (size_t)i * nq * HD + (size_t)h * HD + 2 * lane;
            o[0] = (_Float16)(acc[a][0] / l[a]);
            o[1] = (_Float16)(acc[a][1] / l[a]);
        }
    }
}

}  // namespace

int zhk_rms_norm_rows_f16(zh_ctx *c, const float *x, const float *w, _Float16 *out, uint32_t n, uint32_t rows,
                          float eps) {
    hipLaunchKernelGGL(k_rms_norm_rows_f16, dim3(rows), dim3(256), 0, c->stream, x, w, out, n, eps);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
int zhk_swiglu_rows_f16(zh_ctx *c, const float *g, const float *u, _Float16 *out, float *unscale, uint32_t n,
                        uint32_t rows) {
    hipLaunchKernelGGL(k_swiglu_rows_f16, dim3(rows), dim3(256), 0, c->stream, g, u, out, unscale, n);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
int zhk_attn_prefill(zh_ctx *c, const float *q, const uint16_t *kc, const uint16_t *vc, const uint32_t *pages,
                     uint32_t n_pages, uint32_t cache_tokens, uint32_t nq, uint32_t nkv, uint32_t hd, uint32_t pos0,
                     uint32_t N, float scale, _Float16 *out) {
    if (hd != 128 || nkv == 0 || nq % nkv) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "attn_prefill heads");
    hipLaunchKernelGGL(k_attn_prefill, dim3(nq, (N + AP_Q - 1) / AP_Q), dim3(256), 0, c->stream, q, kc, vc, pages,
                       n_pages, cache_tokens, nq, nkv, pos0, N, scale, out);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}
