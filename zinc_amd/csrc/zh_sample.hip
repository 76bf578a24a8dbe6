// Token sampling on the device: sampleFromLogits (src/compute/forward.zig
// :10261-10334) with repetition penalty (adjustedLogit :10241-10245), top-k,
// temperature and top-p, and the greedy scans it falls back to
// (argmaxFromLogits :10247-10259).
//
// The reference reads the whole logits vector back and scans it on the host;
// here two kernels select on the device and only the token comes back.
//  1. k_sample_slices: NB workgroups each take a slice of at most 4096
//     logits, apply the penalty (history tokens of the slice marked in an LDS
//     bitmap), turn every candidate into a 64-bit key
//        (order-preserving f32 bits) << 32 | (0xFFFFFFFF - token)
//     (larger value first, equal values: earlier token first, the
//     reference's insertion order) and bitonic-sort the slice in LDS; the
//     first K keys go out.
//  2. k_sample_pick: one workgroup sorts the NB x K keys (at most 8192) in
//     LDS, then one lane runs the reference's f64 weighting, top-p cut and
//     draw over the K best.
// Non-candidates (non-finite logits when sampling, NaN when scanning for the
// maximum) get key 0 and sort last.
#include "zh_device.h"
#include "zh_internal.h"

namespace {

constexpr int SL_T = 1024;       // threads per workgroup
constexpr int SL_N = 4096;       // keys per slice sort
constexpr int PK_N = 8192;       // keys of the final sort
constexpr uint32_t MAX_K = 128;  // sampleFromLogits' max_candidates

// f32 -> u32 with the float order (negative values reversed below positive)
__device__ __forceinline__ uint32_t ord_f32(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float unord_f32(uint32_t o) {
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

// Bitonic sort of n (a power of two) keys in LDS into descending order.
__device__ void sort_desc(uint64_t *k, uint32_t n) {
    for (uint32_t size = 2; size <= n; size <<= 1) {
        for (uint32_t j = size >> 1; j > 0; j >>= 1) {
            for (uint32_t i = threadIdx.x; i < n / 2; i += SL_T) {
                const uint32_t l = (i / j) * 2 * j + (i % j), r = l + j;
                const uint64_t a = k[l], b = k[r];
                // blocks with (l & size) == 0 run descending; the last pass
                // (size == n) is one descending block
                const bool desc = (l & size) == 0;
                if (desc ? (a < b) : (a > b)) {
                    k[l] = b;
                    k[r] = a;
                }
            }
            __syncthreads();
        }
    }
}

struct SampleP {
    const float *logits;
    uint32_t V, slice, nb, K;
    const uint32_t *hist;
    uint32_t nh;
    float pen;          // repetition penalty (<= 1.0001: none)
    uint32_t greedy;    // 1: argmaxFromLogits (NaN never a candidate, +-inf are); 0: finite logits only
    float temperature, top_p;
    double u;
    uint64_t *keys;     // [nb][K]
    uint32_t *out;
};

__global__ __launch_bounds__(SL_T) void k_sample_slices(SampleP p) {
    __shared__ uint64_t keys[SL_N];
    __shared__ uint32_t seen[SL_N / 32];
    const uint32_t tid = threadIdx.x, lo = blockIdx.x * p.slice;
    for (uint32_t i = tid; i < SL_N / 32; i += SL_T) seen[i] = 0;
    __syncthreads();
    if (p.pen > 1.0001f)
        for (uint32_t i = tid; i < p.nh; i += SL_T) {
            const uint32_t t = p.hist[i] - lo;  // tokenSeen: history tokens of this slice
            if (t < p.slice) atomicOr(&seen[t / 32], 1u << (t % 32));
        }
    __syncthreads();
    for (uint32_t e = tid; e < SL_N; e += SL_T) {
        const uint32_t idx = lo + e;
        uint64_t key = 0;
        if (e < p.slice && idx < p.V) {
            const float raw = p.logits[idx];
            float v = raw;
            if (p.pen > 1.0001f && (seen[e / 32] >> (e % 32) & 1u))
                v = v >= 0.f ? __fdiv_rn(v, p.pen) : __fmul_rn(v, p.pen);
            const bool cand = p.greedy ? !isnan(v) : isfinite(raw);
            if (cand) key = ((uint64_t)ord_f32(v) << 32) | (uint64_t)(0xFFFFFFFFu - idx);
        }
        keys[e] = key;
    }
    __syncthreads();
    sort_desc(keys, SL_N);
    for (uint32_t j = tid; j < p.K; j += SL_T) p.keys[(size_t)blockIdx.x * p.K + j] = keys[j];
}

__global__ __launch_bounds__(SL_T) void k_sample_pick(SampleP p) {
    __shared__ uint64_t keys[PK_N];
    const uint32_t tid = threadIdx.x, n = p.nb * p.K;
    uint32_t np2 = 1;
    while (np2 < n) np2 <<= 1;
    for (uint32_t i = tid; i < np2; i += SL_T) keys[i] = i < n ? p.keys[i] : 0ull;
    __syncthreads();
    sort_desc(keys, np2);
    if (tid != 0) return;
    uint32_t tok = 0;
    if (p.greedy) {
        // the scan starts from logits[0]: a NaN there is never replaced
        if (!isnan(p.logits[0]) && keys[0] != 0) tok = 0xFFFFFFFFu - (uint32_t)keys[0];
        *p.out = tok;
        return;
    }
    uint32_t cnt = 0;
    while (cnt < p.K && keys[cnt] != 0) cnt++;
    if (cnt == 0) { *p.out = 0; return; }
    auto id_of = [&](uint32_t i) { return 0xFFFFFFFFu - (uint32_t)keys[i]; };
    auto val_of = [&](uint32_t i) { return unord_f32((uint32_t)(keys[i] >> 32)); };
    if (cnt == 1) { *p.out = id_of(0); return; }
    // weights exp(l / T - l0 / T) in f64 (forward.zig:10300-10307)
    const double T = (double)p.temperature, m0 = (double)val_of(0) / T;
    double total = 0.0;
    for (uint32_t i = 0; i < cnt; i++) total += exp((double)val_of(i) / T - m0);
    if (!(total > 0.0) || !isfinite(total)) { *p.out = id_of(0); return; }
    uint32_t keep = cnt;
    if (p.top_p < 0.9999f) {
        double cum = 0.0;
        for (uint32_t i = 0; i < cnt; i++) {
            cum += exp((double)val_of(i) / T - m0) / total;
            keep = i + 1;
            if (cum >= (double)p.top_p && i > 0) break;
        }
    }
    double kept = 0.0;
    for (uint32_t i = 0; i < keep; i++) kept += exp((double)val_of(i) / T - m0);
    if (!(kept > 0.0) || !isfinite(kept)) { *p.out = id_of(0); return; }
    const double target = p.u * kept;
    double cum = 0.0;
    tok = id_of(keep - 1);
    for (uint32_t i = 0; i < keep; i++) {
        cum += exp((double)val_of(i) / T - m0);
        if (target <= cum) { tok = id_of(i); break; }
    }
    *p.out = tok;
}

}  // namespace

bool zhk_sampling_requires_readback(const zh_sampling_params *s) {
    return s->temperature > 0.0001f || s->top_p < 0.9999f || s->repetition_penalty > 1.0001f;
}

// sampleFromLogits over n device logits; hist (device, nh tokens) is the
// generated history; the token lands in out (device). Stream ordered.
int zhk_sample(zh_ctx *c, const float *logits, uint32_t n, const uint32_t *hist, uint32_t nh,
               const zh_sampling_params *s, double u, uint64_t *keys, uint32_t *out) {
    if (n == 0 || n > zhk_sample_max_vocab()) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "sample: %u logits", n);
    SampleP p = {};
    p.logits = logits;
    p.V = n;
    p.hist = hist;
    p.nh = nh;
    p.out = out;
    p.keys = keys;
    const bool readback = zhk_sampling_requires_readback(s);
    // greedy unless sampling: argmaxFromLogits with the penalty when the
    // temperature is off, without it when nothing needs the logits
    p.greedy = !readback || s->temperature <= 0.0001f;
    p.pen = readback ? s->repetition_penalty : 1.0f;
    p.K = p.greedy ? 1u : (s->top_k < 1 ? 1u : s->top_k > MAX_K ? MAX_K : s->top_k);
    p.temperature = s->temperature > 0.0001f ? s->temperature : 0.0001f;
    p.top_p = s->top_p < 0.f ? 0.f : s->top_p > 1.f ? 1.f : s->top_p;
    p.u = u;
    // slices of at most SL_N logits, at most PK_N / K of them
    p.nb = (n + SL_N - 1) / SL_N;
    const uint32_t want = (n + 2047) / 2048;  // about 2048 logits per slice when that fits
    if (want > p.nb && want * p.K <= (uint32_t)PK_N) p.nb = want;
    p.slice = (n + p.nb - 1) / p.nb;
    if (p.nb * p.K > (uint32_t)PK_N || p.slice > (uint32_t)SL_N)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "sample: %u logits with top_k %u", n, p.K);
    hipLaunchKernelGGL(k_sample_slices, dim3(p.nb), dim3(SL_T), 0, c->stream, p);
    hipLaunchKernelGGL(k_sample_pick, dim3(1), dim3(SL_T), 0, c->stream, p);
    ZH_LAUNCH_CHECK(c);
    return ZH_OK;
}

uint32_t zhk_sample_max_vocab() { return (uint32_t)PK_N / MAX_K * SL_N; }

// Scratch layout: token word, keys (PK_N), history.
int zhk_sample_host(zh_ctx *c, const float *logits, uint32_t n, const zh_sampling_params *s, const uint32_t *history,
                    uint32_t nh, double u, uint32_t *token) {
    if (!s || !token || (nh && !history)) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "sample: null argument");
    const bool pen = zhk_sampling_requires_readback(s) && s->repetition_penalty > 1.0001f;
    const uint64_t hist_n = pen ? nh : 0;
    void *scr = nullptr;
    int rc = zh_scratch(c, 256 + 8ull * PK_N + 4ull * hist_n + 4, &scr);
    if (rc) return rc;
    uint32_t *out = (uint32_t *)scr;
    uint64_t *keys = (uint64_t *)((char *)scr + 256);
    uint32_t *hd = (uint32_t *)((char *)scr + 256 + 8ull * PK_N);
    if (hist_n) ZH_HIP(c, hipMemcpyAsync(hd, history, 4ull * hist_n, hipMemcpyHostToDevice, c->stream));
    rc = zhk_sample(c, logits, n, hd, (uint32_t)hist_n, s, u, keys, out);
    if (rc) return rc;
    ZH_HIP(c, hipMemcpyAsync(token, out, 4, hipMemcpyDeviceToHost, c->stream));
    ZH_HIP(c, hipStreamSynchronize(c->stream));
    return ZH_OK;
}

extern "C" int zh_sample_logits(zh_ctx *c, const zh_buf *logits, uint64_t off, uint32_t n,
                                const zh_sampling_params *s, const uint32_t *history, uint32_t n_history, double u,
                                uint32_t *token) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (!logits || off % 4 || off + 4ull * n > zh_buf_size(logits))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "sample: logits range");
    return zhk_sample_host(c, (const float *)((const char *)zh_buf_device_ptr(logits) + off), n, s, history,
                           n_history, u, token);
}
