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
constexpr int LDR = KS + 8;     // halfs per LDS row (272 B: 16-byte reads of 8 rows hit distinct banks)

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

ZH_DEV _Float16 to_h(float v) { return (_Float16)v; }  // round to nearest even

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
// mj = dmin*m[j], out = dj*q - mj; the f32 operations rounded one by one (no
// contraction), then to fp16 (nearest even).
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
            const uint32_t n4 = (qw[w] >> (4 * nib)) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; b++) {  // byte-to-float conversions (v_cvt_f32_ubyteN)
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
// and raw weight bytes of the next step are in flight in registers. 70 KB of
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
    Raw wr[UPT];
    auto load_step = [&](uint32_t st) {
#pragma unroll
        for (int c = 0; c < XC; c++) {
            const uint32_t idx = c * GT + tid, t = idx / (KS / 8), ch = idx % (KS / 8);
            const uint32_t tok = min(n0 + t, p.N - 1);
            xr[c] = *(const half8 *)(p.X + (size_t)tok * p.ldx + (size_t)st * KS + ch * 8);
        }
#pragma unroll
        for (int k = 0; k < UPT; k++) {
            const uint32_t u = k * GT + tid, r = u >> 2, u4 = u & 3;
            const uint32_t row = min(j0 + r, Ms - 1);  // rows past the segment: loaded clamped, never written
            const uint8_t *blk = Wseg + (size_t)row * p.row_bytes + (size_t)(st >> 1) * bpb;
            if constexpr (QT == ZH_Q4_K) load_q4k_unit(blk, 2 * (st & 1) + (u4 >> 1), wr[k]);
            else load_q6k_unit(blk, st & 1, u4, wr[k]);
        }
    };
    load_step(st_begin);
    for (uint32_t st = st_begin; st < nst; st++) {
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
        if (st + 1 < nst) load_step(st + 1);
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
                    if (tok < p.N && row < Ms) p.part[((size_t)z * p.N + tok) * p.M + row] = acc[i][j][r];
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

}  // namespace

int zhk_gemm_multi(zh_ctx *c, uint32_t qtype, uint32_t nseg, const uint8_t *const *W, const _Float16 *X, uint32_t ldx,
                   float *const *Y, const uint32_t *ldy, const uint32_t *M, uint32_t K, uint32_t N, uint32_t acc,
                   const float *x_unscale) {
    if ((qtype != ZH_Q4_K && qtype != ZH_Q6_K) || K % 256 || N == 0 || nseg < 1 || nseg > 3)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "gemm: qtype %u K %u N %u nseg %u", qtype, K, N, nseg);
    GemmP p = {};
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
    // Stacked matrices: 64-row tiles when 128-row tiles would leave CUs idle;
    // every segment but the last must then be a whole number of tiles. A
    // single matrix keeps 128-row tiles and splits K instead (below).
    bool small = (uint64_t)((end + 127) / 128) * ni < (uint64_t)c->cu_count &&
                 (nseg > 1 || getenv("ZH_GEMM_TJ64"));
    for (uint32_t s = 0; s + 1 < nseg; s++)
        if (M[s] % 128) small = true;
    for (uint32_t s = 0; s + 1 < nseg; s++)
        if (M[s] % 64) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "gemm: segment rows %u not a multiple of 64", M[s]);
    const uint32_t TJv = small ? 64 : 128;
    const uint32_t lds = (TI + TJv) * LDR * 2;
    // A single matrix with fewer tiles than two per CU (O, down) splits K so
    // two workgroups share each CU (one's dequantisation overlapping the
    // other's MFMAs); at least 8 K-steps per split.
    const uint64_t tiles = (uint64_t)((end + TJv - 1) / TJv) * ni, slots = 2ull * (uint64_t)c->cu_count;
    p.ksplit = 1;
    if (nseg == 1 && tiles < slots && !getenv("ZH_NO_SPLITK")) {
        uint32_t sk = (uint32_t)((slots + tiles - 1) / tiles);
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
    if (p.ksplit > 1) {
        const uint64_t n = (uint64_t)N * end;
        hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, c->stream, p.part, p.ksplit,
                           N, end, Y[0], ldy[0], acc, x_unscale);
    }
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

int zhk_gemm(zh_ctx *c, uint32_t qtype, const uint8_t *W, const _Float16 *X, uint32_t ldx, float *Y, uint32_t ldy,
             uint32_t M, uint32_t K, uint32_t N, uint32_t acc, const float *x_unscale) {
    return zhk_gemm_multi(c, qtype, 1, &W, X, ldx, &Y, &ldy, &M, K, N, acc, x_unscale);
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
