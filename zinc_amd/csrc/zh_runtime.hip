// zh_runtime.hip — context, buffers, timing and the seeded synthetic-data
// generator of libzinc_hip.so.
#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include "zh_device.h"
#include "zh_internal.h"

int zh_set_err(zh_ctx *ctx, int code, const char *fmt, ...) {
    if (ctx) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        ctx->err = buf;
    }
    return code;
}

extern "C" const char *zh_status_string(int s) {
    switch (s) {
    case ZH_OK: return "ok";
    case ZH_ERR_UNSUPPORTED_QUANT_TYPE: return "UnsupportedQuantType";
    case ZH_ERR_INVALID_ARGUMENT: return "InvalidArgument";
    case ZH_ERR_HIP: return "HipError";
    case ZH_ERR_CONTEXT_LENGTH_EXCEEDED: return "ContextLengthExceeded";
    case ZH_ERR_OUT_OF_MEMORY: return "OutOfMemory";
    case ZH_ERR_TENSOR_NOT_FOUND: return "TensorNotFound";
    case ZH_ERR_INVALID_MAGIC: return "InvalidMagic";
    case ZH_ERR_UNKNOWN_METADATA_TYPE: return "UnknownMetadataType";
    case ZH_ERR_UNSUPPORTED_ARCHITECTURE: return "UnsupportedArchitecture";
    case ZH_ERR_TRUNCATED_FILE: return "TruncatedFile";
    case ZH_ERR_IO: return "IoError";
    case ZH_ERR_NOT_FOUND: return "NotFound";
    case ZH_ERR_KV_CACHE_EXHAUSTED: return "KvCacheExhausted";
    case ZH_ERR_WAIT_TIMEOUT: return "WaitTimeout";
    default: return "unknown";
    }
}

extern "C" int zh_init(int device, zh_ctx **out) {
    if (!out) return ZH_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= device || device < 0) return ZH_ERR_HIP;
    if (hipSetDevice(device) != hipSuccess) return ZH_ERR_HIP;
    zh_ctx *c = new zh_ctx();
    c->device = device;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) { delete c; return ZH_ERR_HIP; }
    c->cu_count = prop.multiProcessorCount;
    // Default-priority, non-blocking stream (one per engine/context).
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) { delete c; return ZH_ERR_HIP; }
    for (int i = 0; i < 64; i++)
        if (hipEventCreate(&c->ev[i]) != hipSuccess) { delete c; return ZH_ERR_HIP; }
    const uint32_t ctl[2] = {0u, ZH_ATTN_WAIT_TICKS};
    if (hipMalloc((void **)&c->err_dev, 256) != hipSuccess ||
        hipMemcpy(c->err_dev, ctl, sizeof ctl, hipMemcpyHostToDevice) != hipSuccess) {
        zh_destroy(c);
        return ZH_ERR_HIP;
    }
    *out = c;
    return ZH_OK;
}

extern "C" void zh_destroy(zh_ctx *c) {
    if (!c) return;
    hipSetDevice(c->device);
    hipStreamSynchronize(c->stream);
    if (c->scratch) hipFree(c->scratch);
    if (c->err_dev) hipFree(c->err_dev);
    for (int i = 0; i < 64; i++) if (c->ev[i]) hipEventDestroy(c->ev[i]);
    hipStreamDestroy(c->stream);
    delete c;
}

extern "C" const char *zh_last_error(const zh_ctx *c) { return c ? c->err.c_str() : "no context"; }

extern "C" int zh_device_info(zh_ctx *c, char *name, size_t name_len, int *cu, uint64_t *hbm) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    hipDeviceProp_t p;
    ZH_HIP(c, hipGetDeviceProperties(&p, c->device));
    if (name && name_len) snprintf(name, name_len, "%s (%s)", p.name, p.gcnArchName);
    if (cu) *cu = p.multiProcessorCount;
    if (hbm) *hbm = p.totalGlobalMem;
    return ZH_OK;
}

extern "C" int zh_sync(zh_ctx *c) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    ZH_HIP(c, hipStreamSynchronize(c->stream));
    // input a kernel had to clamp since the last zh_sync
    uint32_t e = 0;
    ZH_HIP(c, hipMemcpy(&e, c->err_dev, 4, hipMemcpyDeviceToHost));
    if (e) {
        ZH_HIP(c, hipMemset(c->err_dev, 0, 4));
        if (e & (ZH_DEVERR_ATTN_WAIT | ZH_DEVERR_STEP_BARRIER)) {
            for (const auto &w : c->xwords) ZH_HIP(c, hipMemset(w.p, 0, w.bytes));
            ZH_HIP(c, hipDeviceSynchronize());
            // check the workgroup placement again (here, outside any graph
            // capture: the probe synchronises); engines re-record their step
            c->xcd_rr = -1;
            zhk_xcd_round_robin(c);
            c->place_gen++;
        }
        if (e & ZH_DEVERR_STEP_BARRIER)
            return zh_set_err(c, ZH_ERR_WAIT_TIMEOUT, "a grid barrier of the decode-layers kernel gave up waiting "
                                                      "(its workgroups were not all resident); the step's output "
                                                      "is not valid");
        if (e & ZH_DEVERR_ATTN_WAIT)
            return zh_set_err(c, ZH_ERR_WAIT_TIMEOUT, "a decode-attention merger gave up waiting for the other "
                                                      "chunks of its kv head; that head's output is NaN");
        if (e & ZH_DEVERR_EXPERT_ID)
            return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "an expert id at or past the weights' expert count "
                                                          "(zh_dmmv_moe clamped it to the last expert)");
    }
    return ZH_OK;
}

extern "C" int zh_set_attn_wait_limit(zh_ctx *c, uint32_t microseconds) {
    if (!c) return ZH_ERR_INVALID_ARGUMENT;
    if (microseconds > 40000000u) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "wait limit above 40 s");
    const uint32_t ticks = microseconds * 100u;
    ZH_HIP(c, hipStreamSynchronize(c->stream));
    ZH_HIP(c, hipMemcpy(c->err_dev + 1, &ticks, 4, hipMemcpyHostToDevice));
    return ZH_OK;
}

int zh_scratch(zh_ctx *c, uint64_t bytes, void **out) {
    if (bytes > c->scratch_size) {
        if (c->scratch) {
            ZH_HIP(c, hipStreamSynchronize(c->stream));
            ZH_HIP(c, hipFree(c->scratch));
            c->scratch = nullptr;
        }
        uint64_t sz = bytes < (1u << 20) ? (1u << 20) : bytes + 256;
        ZH_HIP(c, hipMalloc(&c->scratch, sz));
        c->scratch_size = sz;
    }
    *out = c->scratch;
    return ZH_OK;
}

// ---------------------------------------------------------------- buffers
extern "C" int zh_buf_alloc(zh_ctx *c, uint64_t size, zh_buf **out) {
    if (!c || !out) return ZH_ERR_INVALID_ARGUMENT;
    *out = nullptr;
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, size + 256);
    if (e != hipSuccess)
        return zh_set_err(c, ZH_ERR_OUT_OF_MEMORY, "hipMalloc(%llu): %s", (unsigned long long)size,
                          hipGetErrorString(e));
    // Zero the pad so over-reads are deterministic.
    ZH_HIP(c, hipMemsetAsync((char *)p + size, 0, 256, c->stream));
    zh_buf *b = new zh_buf{p, size};
    *out = b;
    return ZH_OK;
}

extern "C" void zh_buf_free(zh_ctx *c, zh_buf *b) {
    if (!b) return;
    if (c) hipStreamSynchronize(c->stream);
    hipFree(b->ptr);
    delete b;
}
extern "C" uint64_t zh_buf_size(const zh_buf *b) { return b ? b->size : 0; }
extern "C" void *zh_buf_device_ptr(const zh_buf *b) { return b ? b->ptr : nullptr; }

extern "C" int zh_buf_upload(zh_ctx *c, zh_buf *b, uint64_t off, const void *src, uint64_t n) {
    if (!c || !b || !src || off + n > b->size)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "upload out of range");
    ZH_HIP(c, hipMemcpyAsync((char *)b->ptr + off, src, n, hipMemcpyHostToDevice, c->stream));
    ZH_HIP(c, hipStreamSynchronize(c->stream));
    return ZH_OK;
}
extern "C" int zh_buf_download(zh_ctx *c, const zh_buf *b, uint64_t off, void *dst, uint64_t n) {
    if (!c || !b || !dst || off + n > b->size)
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "download out of range");
    ZH_HIP(c, hipMemcpyAsync(dst, (char *)b->ptr + off, n, hipMemcpyDeviceToHost, c->stream));
    ZH_HIP(c, hipStreamSynchronize(c->stream));
    return ZH_OK;
}
extern "C" int zh_buf_fill_u8(zh_ctx *c, zh_buf *b, uint64_t off, uint8_t v, uint64_t n) {
    if (!c || !b || off + n > b->size) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "fill out of range");
    ZH_HIP(c, hipMemsetAsync((char *)b->ptr + off, v, n, c->stream));
    return ZH_OK;
}

extern "C" int zh_event_record(zh_ctx *c, int slot) {
    if (!c || slot < 0 || slot >= 64) return ZH_ERR_INVALID_ARGUMENT;
    ZH_HIP(c, hipEventRecord(c->ev[slot], c->stream));
    return ZH_OK;
}
extern "C" int zh_event_elapsed_ms(zh_ctx *c, int a, int b, float *ms) {
    if (!c || a < 0 || b < 0 || a >= 64 || b >= 64 || !ms) return ZH_ERR_INVALID_ARGUMENT;
    ZH_HIP(c, hipEventSynchronize(c->ev[b]));
    ZH_HIP(c, hipEventElapsedTime(ms, c->ev[a], c->ev[b]));
    return ZH_OK;
}

// ---------------------------------------------------------------------------
// Seeded synthetic data. Same specification as oracle/zinc_oracle.c
// (zo_rand / zo_normal / zo_synth_tensor): splitmix64 finaliser over
// (seed, stream, counter); Irwin-Hall(4) normal standardised by one f32
// multiply; f16 by round-to-nearest-even. Every float op is a single
// correctly rounded operation (explicit _rn intrinsics: no contraction), so
// the bytes are identical to the host generator's.
// ---------------------------------------------------------------------------
ZH_DEV uint64_t fmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
ZH_DEV uint64_t synth_key(uint64_t seed, uint64_t stream) { return fmix64(seed ^ (stream * 0xD1B54A32D192ED03ull)); }
ZH_DEV uint64_t synth_rand(uint64_t key, uint64_t ctr) { return fmix64(key + (ctr + 1) * 0x9E3779B97F4A7C15ull); }
ZH_DEV float synth_normal(uint64_t r) {
    int s = (int)(r & 0xFFFF) + (int)((r >> 16) & 0xFFFF) + (int)((r >> 32) & 0xFFFF) +
            (int)((r >> 48) & 0xFFFF) - 131070;
    return __fmul_rn((float)s, 2.6429573e-05f);
}
ZH_DEV uint16_t synth_scale_f16(uint64_t r) { return f2h_rn(__fmul_rn(fabsf(synth_normal(r)), 0.02f)); }

// qtype | ZH_SYNTH_CENTERED selects the model-init variant of Q4_K / Q5_K:
// dmin = f16(7.5 * d) / f16(15.5 * d) (the mean 4- / 5-bit code), which makes
// every sub-block's expected weight zero-mean over random (sc, m), so mat-vec
// outputs carry no common mode.
#define ZH_SYNTH_CENTERED 0x100u
// qtype | ZH_SYNTH_ROUTER | e << 12 (Q8_0): a router, d = f16(d * 2^-e), e from
// zh_router_shift(K): the router logits of an RMS-normed input are then about
// N(0,1), not O(sqrt(K)) as the other projections'.
#define ZH_SYNTH_ROUTER 0x200u
__global__ void k_synth_tensor(uint8_t *dst, uint32_t qtype_flags, uint64_t b0, uint64_t b1, uint64_t key) {
    uint64_t b = b0 + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= b1) return;
    const uint32_t qtype = qtype_flags & 0xFFu;
    const bool centered = (qtype_flags & ZH_SYNTH_CENTERED) != 0;
    switch (qtype) {
    case ZH_Q4_K: {
        uint8_t *o = dst + b * 144;
        uint16_t d = synth_scale_f16(synth_rand(key, b * 32 + 0));
        uint16_t dm = centered ? f2h_rn(__fmul_rn(h2f(d), 7.5f)) : synth_scale_f16(synth_rand(key, b * 32 + 1));
        o[0] = d & 0xFF; o[1] = d >> 8; o[2] = dm & 0xFF; o[3] = dm >> 8;
        for (int i = 0; i < 140; i++) {
            uint64_t r = synth_rand(key, b * 32 + 2 + i / 8);
            o[4 + i] = (uint8_t)(r >> (8 * (i % 8)));
        }
        break;
    }
    case ZH_Q5_K: {  // as Q4_K, then 172 uniform bytes (scales, qh, qs)
        uint8_t *o = dst + b * 176;
        uint16_t d = synth_scale_f16(synth_rand(key, b * 32 + 0));
        uint16_t dm = centered ? f2h_rn(__fmul_rn(h2f(d), 15.5f)) : synth_scale_f16(synth_rand(key, b * 32 + 1));
        o[0] = d & 0xFF; o[1] = d >> 8; o[2] = dm & 0xFF; o[3] = dm >> 8;
        for (int i = 0; i < 172; i++) {
            uint64_t r = synth_rand(key, b * 32 + 2 + i / 8);
            o[4 + i] = (uint8_t)(r >> (8 * (i % 8)));
        }
        break;
    }
    case ZH_Q6_K: {
        uint8_t *o = dst + b * 210;
        for (int i = 0; i < 192; i++) {
            uint64_t r = synth_rand(key, b * 32 + 1 + i / 8);
            o[i] = (uint8_t)(r >> (8 * (i % 8)));
        }
        for (int i = 0; i < 16; i++) {
            uint64_t r = synth_rand(key, b * 32 + 25 + i / 8);
            uint8_t byte = (uint8_t)(r >> (8 * (i % 8)));
            o[192 + i] = (uint8_t)(int8_t)((int)(byte & 63) - 32);
        }
        uint16_t d = synth_scale_f16(synth_rand(key, b * 32 + 0));
        o[208] = d & 0xFF; o[209] = d >> 8;
        break;
    }
    case ZH_Q8_0: {
        uint8_t *o = dst + b * 34;
        uint16_t d = synth_scale_f16(synth_rand(key, b * 16 + 0));
        if (qtype_flags & ZH_SYNTH_ROUTER) d = f2h_rn(ldexpf(h2f(d), -(int)((qtype_flags >> 12) & 15u)));
        o[0] = d & 0xFF; o[1] = d >> 8;
        for (int i = 0; i < 32; i++) {
            uint64_t r = synth_rand(key, b * 16 + 1 + i / 4);
            uint32_t u = (uint32_t)(r >> (16 * (i % 4))) & 0xFFFF;
            o[2 + i] = (uint8_t)(int8_t)((int)(u % 255u) - 127);
        }
        break;
    }
    case ZH_MXFP4: {
        uint8_t *o = dst + b * 17;
        uint64_t r0 = synth_rand(key, b * 4 + 0);
        o[0] = (uint8_t)(118 + (r0 % 13));
        for (int i = 0; i < 16; i++) {
            uint64_t r = synth_rand(key, b * 4 + 1 + i / 8);
            o[1 + i] = (uint8_t)(r >> (8 * (i % 8)));
        }
        break;
    }
    case ZH_F32: {
        float v = synth_normal(synth_rand(key, b));
        ((float *)dst)[b] = v;
        break;
    }
    case ZH_F16: {
        ((uint16_t *)dst)[b] = f2h_rn(synth_normal(synth_rand(key, b)));
        break;
    }
    }
}

__global__ void k_synth_vector(void *dst, uint32_t kind, uint64_t i0, uint64_t i1, float scale,
                               uint64_t key) {
    uint64_t i = i0 + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= i1) return;
    uint64_t r = synth_rand(key, i);
    if (kind == 0) {
        ((float *)dst)[i] = __fmul_rn(synth_normal(r), scale);
    } else if (kind == 1) {
        ((uint16_t *)dst)[i] = f2h_rn(synth_normal(r));
    } else {
        int s = (int)(r & 0xFFFF) - 32768;
        ((float *)dst)[i] = __fadd_rn(1.0f, __fmul_rn((float)s, 3.0517578e-07f));
    }
}

static uint64_t host_synth_key(uint64_t seed, uint64_t stream) {
    uint64_t z = seed ^ (stream * 0xD1B54A32D192ED03ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint32_t zh_router_shift(uint64_t K) {
    // 2^e nearest to 1.466 sqrt(K), 1.466 the standard deviation of the
    // synthetic Q8_0 weights d * q (d = |N(0, .02)|, q uniform -127..127)
    const long e = lround(log2(1.466 * sqrt((double)K)));
    return e < 0 ? 0u : e > 15 ? 15u : (uint32_t)e;
}

int zhk_synth_tensor(zh_ctx *c, uint8_t *dst, uint32_t qtype_flags, uint64_t rows, uint64_t cols,
                     uint64_t seed, uint64_t stream) {
    const uint32_t qtype = qtype_flags & 0xFFu;
    uint64_t nb = rows * (cols / zh_block_size(qtype));
    uint64_t key = host_synth_key(seed, stream);
    const uint64_t chunk = 1ull << 24;
    for (uint64_t b0 = 0; b0 < nb; b0 += chunk) {
        uint64_t n = nb - b0 < chunk ? nb - b0 : chunk;
        hipLaunchKernelGGL(k_synth_tensor, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, c->stream,
                           dst, qtype_flags, b0, b0 + n, key);
        ZH_LAUNCH_CHECK(c);
    }
    return ZH_OK;
}

int zhk_synth_vector(zh_ctx *c, void *dst, uint32_t kind, uint64_t n, float scale, uint64_t seed,
                     uint64_t stream) {
    uint64_t key = host_synth_key(seed, stream);
    const uint64_t chunk = 1ull << 26;
    for (uint64_t i0 = 0; i0 < n; i0 += chunk) {
        uint64_t m = n - i0 < chunk ? n - i0 : chunk;
        hipLaunchKernelGGL(k_synth_vector, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, c->stream,
                           dst, kind, i0, i0 + m, scale, key);
        ZH_LAUNCH_CHECK(c);
    }
    return ZH_OK;
}

extern "C" int zh_synth_tensor(zh_ctx *c, zh_buf *buf, uint64_t off, uint32_t qtype_flags, uint64_t rows,
                               uint64_t cols, uint64_t seed, uint64_t stream) {
    if (!c || !buf) return ZH_ERR_INVALID_ARGUMENT;
    const uint32_t qtype = qtype_flags & 0xFFu;
    if (qtype_flags & ~(0xFFu | ZH_SYNTH_CENTERED | ZH_SYNTH_ROUTER | 0xF000u))
        return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "synth flags");
    uint32_t bs = zh_block_size(qtype), bpb = zh_bytes_per_block(qtype);
    if (bpb == 0) return zh_set_err(c, ZH_ERR_UNSUPPORTED_QUANT_TYPE, "qtype %u", qtype);
    if (cols % bs) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "cols %% block size");
    uint64_t bytes = zh_tensor_bytes(qtype, rows, cols);
    if (off + bytes > buf->size) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "synth out of range");
    return zhk_synth_tensor(c, (uint8_t *)buf->ptr + off, qtype_flags, rows, cols, seed, stream);
}

extern "C" int zh_synth_vector(zh_ctx *c, zh_buf *buf, uint64_t off, uint32_t kind, uint64_t n,
                               float scale, uint64_t seed, uint64_t stream) {
    if (!c || !buf || kind > 2) return ZH_ERR_INVALID_ARGUMENT;
    uint64_t bytes = n * (kind == 1 ? 2 : 4);
    if (off + bytes > buf->size) return zh_set_err(c, ZH_ERR_INVALID_ARGUMENT, "synth out of range");
    return zhk_synth_vector(c, (char *)buf->ptr + off, kind, n, scale, seed, stream);
}

// ---------------------------------------------------------------------------
// Calibration probe (the counterpart of the reference's bandwidth
// microbenchmark, benchmarks/bandwidth.zig): a streaming-read
// kernel that gives the achievable HBM read ceiling.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_stream_read(const u32x4 *__restrict__ p, uint64_t n16, uint32_t *out) {
    uint32_t acc = 0;
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        u32x4 a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + stride);
        u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride), d = __builtin_nontemporal_load(p + i + 3 * stride);
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += stride) {
        u32x4 a = p[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == 0x9E3779B9u) out[0] = acc;  // keeps the loads live; practically never taken
}

// Register-load streaming over per-workgroup contiguous slices: workgroup b
// reads 16-byte words [b per, (b + 1) per) of the buffer, U loads in flight
// per thread (U x 16 B x the workgroup's threads per CU), plain loads.
template <int U>
__global__ __launch_bounds__(256) void k_stream_slice(const u32x4 *__restrict__ p, uint64_t n16, uint64_t per,
                                                       uint32_t *out) {
    const uint64_t b0 = (uint64_t)blockIdx.x * per, b1 = b0 + per < n16 ? b0 + per : n16;
    const uint32_t nt = blockDim.x;
    uint32_t acc = 0;
    uint64_t i = b0 + threadIdx.x;
    for (; i + (U - 1) * (uint64_t)nt < b1; i += (uint64_t)U * nt) {
        u32x4 v[U];
#pragma unroll
        for (int k = 0; k < U; k++) v[k] = p[i + (uint64_t)k * nt];
#pragma unroll
        for (int k = 0; k < U; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    for (; i < b1; i += nt) {
        const u32x4 a = p[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == 0x9E3779B9u) out[0] = acc;  // keeps the loads live; practically never taken
}

// The streaming-read ceiling: the best of three read patterns over the same
// bytes, each timed over `iters` launches (HIP events):
//   0 grid-stride nontemporal 16-byte loads, 8 workgroups of 256 per CU, 4 in flight per thread;
//   1 per-workgroup contiguous slices, 4 workgroups of 256 per CU, 32 loads in flight per thread;
//   2 per-workgroup contiguous slices, 8 workgroups of 256 per CU, 16 loads in flight per thread.
// (Measured on MI355X: 5.8-6.3 TB/s for all of them over 1-4 GB; up to
// 7.3 TB/s over 256 MB, which the 256 MB MALL partly serves.)
extern "C" int zh_stream_read_probe(zh_ctx *c, const zh_buf *buf, uint64_t bytes, uint32_t iters, float *gbs) {
    if (!c || !buf || !gbs || bytes > buf->size || bytes < 16 || iters == 0) return ZH_ERR_INVALID_ARGUMENT;
    void *o;
    int rc = zh_scratch(c, 256, &o);
    if (rc) return rc;
    const u32x4 *src = (const u32x4 *)buf->ptr;
    const uint64_t n16 = bytes / 16;
    const uint32_t cu = (uint32_t)c->cu_count;
    float best = 0.f;
    for (int v = 0; v < 3; v++) {
        auto launch = [&]() {
            if (v == 0) {
                hipLaunchKernelGGL(k_stream_read, dim3(cu * 8), dim3(256), 0, c->stream, src, n16, (uint32_t *)o);
            } else {
                const uint32_t wgs = v == 1 ? 4 * cu : 8 * cu;
                const uint64_t per = (n16 + wgs - 1) / wgs;
                if (v == 1)
                    hipLaunchKernelGGL(k_stream_slice<32>, dim3(wgs), dim3(256), 0, c->stream, src, n16, per, (uint32_t *)o);
                else
                    hipLaunchKernelGGL(k_stream_slice<16>, dim3(wgs), dim3(256), 0, c->stream, src, n16, per, (uint32_t *)o);
            }
        };
        launch();
        ZH_HIP(c, hipEventRecord(c->ev[62], c->stream));
        for (uint32_t k = 0; k < iters; k++) launch();
        ZH_LAUNCH_CHECK(c);
        ZH_HIP(c, hipEventRecord(c->ev[63], c->stream));
        ZH_HIP(c, hipEventSynchronize(c->ev[63]));
        float ms = 0.f;
        ZH_HIP(c, hipEventElapsedTime(&ms, c->ev[62], c->ev[63]));
        const float r = (float)((double)(n16 * 16) * iters / (ms * 1e-3) / 1e9);
        if (r > best) best = r;
    }

    *gbs = best;
    return ZH_OK;
}

