/*
 * zinc_hip.h — C ABI of the MI355X (gfx950) HIP backend for ZINC's per-token
 * decode loop. Built as libzinc_hip.so by hipcc. Every entry point is a plain
 * C function over opaque handles, plain pointers and sizes, returning an int
 * status (ZH_OK == 0). The ABI follows the reference's Metal shim pattern
 * (src/metal/shim.h:23-80: opaque context/buffer handles, create_buffer,
 * dispatch with push-constant style scalars, commit_and_wait) but with one
 * typed entry point per kernel family instead of generic pipelines.
 *
 * Threading: one HIP stream per context; a context is not re-entrant
 * (reference: one command buffer and queue per engine, forward.zig:4361-4363).
 * Ordering: calls enqueue work on the context's stream and return; results are
 * visible to the host after zh_sync (reference: submitAndWait,
 * forward.zig:7757-7772).
 * Buffers: zh_buf_alloc pads every allocation by 256 bytes so kernels may
 * issue dword-aligned 128-bit loads that straddle the logical end.
 */
#ifndef ZINC_HIP_H
#define ZINC_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (map to the reference's Zig error set) ---------------- */
enum {
    ZH_OK = 0,
    ZH_ERR_UNSUPPORTED_QUANT_TYPE = 1, /* error.UnsupportedQuantType  dmmv.zig:722,822 */
    ZH_ERR_INVALID_ARGUMENT = 2,       /* error.InvalidArgument       dmmv.zig:767,944,1065 */
    ZH_ERR_HIP = 3,                    /* device/runtime failure */
    ZH_ERR_CONTEXT_LENGTH_EXCEEDED = 4,/* error.ContextLengthExceeded forward.zig:4300 */
    ZH_ERR_OUT_OF_MEMORY = 5,
    ZH_ERR_TENSOR_NOT_FOUND = 6,       /* error.TensorNotFound        forward.zig:7377 */
    ZH_ERR_INVALID_MAGIC = 7,          /* error.InvalidMagic          gguf.zig:347 */
    ZH_ERR_UNKNOWN_METADATA_TYPE = 8,  /* error.UnknownMetadataType   gguf.zig:513,540 */
    ZH_ERR_UNSUPPORTED_ARCHITECTURE = 9,/* error.UnsupportedArchitecture loader.zig:449 */
    ZH_ERR_TRUNCATED_FILE = 10,        /* a header or tensor runs past the end of the file */
    ZH_ERR_IO = 11,                    /* open / stat / mmap failure (std.fs errors) */
    ZH_ERR_NOT_FOUND = 12,             /* metadata key absent or not of the asked type (null) */
    ZH_ERR_KV_CACHE_EXHAUSTED = 13,    /* error.KvCacheExhausted      kv_cache.zig:73 */
    ZH_ERR_WAIT_TIMEOUT = 14           /* a kernel's bounded cross-workgroup wait gave up */
};

/* ---- GGMLType values used on the path (src/model/gguf.zig:38-69) -------- */
enum { ZH_F32 = 0, ZH_F16 = 1, ZH_Q8_0 = 8, ZH_Q4_K = 12, ZH_Q5_K = 13, ZH_Q6_K = 14, ZH_MXFP4 = 39 };

typedef struct zh_ctx zh_ctx;
typedef struct zh_buf zh_buf;
typedef struct zh_engine zh_engine;
typedef struct zh_kv_pool zh_kv_pool;

/* ---- device lifecycle: replaces Instance.init / mtl_init (shim.h:24-25) -- */
int  zh_init(int device, zh_ctx **out);
void zh_destroy(zh_ctx *ctx);
const char *zh_last_error(const zh_ctx *ctx);
const char *zh_status_string(int status);
/* name (>=64 bytes), CU count, total HBM bytes */
int  zh_device_info(zh_ctx *ctx, char *name, size_t name_len, int *cu_count, uint64_t *hbm_bytes);
int  zh_sync(zh_ctx *ctx);
/* Limit of the bounded wait in the decode attention's in-kernel merge
 * (default 50000 us; 0 = give up at once). No counterpart in the reference,
 * which merges split attention in a dispatch of its own
 * (flash_attn_split_merge.comp); here the first mergers of a kv head wait for
 * its other chunks. A merger that gives up writes NaN for its q head, the
 * launch completes, and the next zh_sync returns ZH_ERR_WAIT_TIMEOUT. Takes
 * effect for later launches, captured graphs included. */
int  zh_set_attn_wait_limit(zh_ctx *ctx, uint32_t microseconds);

/* ---- buffers: replaces Buffer.initDeviceLocal (vulkan/buffer.zig:102) and
 *      mtl_create_buffer / mtl_free_buffer (shim.h:37-41) ----------------- */
int      zh_buf_alloc(zh_ctx *ctx, uint64_t size, zh_buf **out);
void     zh_buf_free(zh_ctx *ctx, zh_buf *buf);
uint64_t zh_buf_size(const zh_buf *buf);
void    *zh_buf_device_ptr(const zh_buf *buf);
int      zh_buf_upload(zh_ctx *ctx, zh_buf *buf, uint64_t offset, const void *src, uint64_t n);
int      zh_buf_download(zh_ctx *ctx, const zh_buf *buf, uint64_t offset, void *dst, uint64_t n);
int      zh_buf_fill_u8(zh_ctx *ctx, zh_buf *buf, uint64_t offset, uint8_t v, uint64_t n);

/* ---- timing (the build's counterpart of the reference's timestamp-query
 *      profiling, forward.zig:2443-2476) ------------------------------- */
int zh_event_record(zh_ctx *ctx, int slot);          /* slot 0..63 */
int zh_event_elapsed_ms(zh_ctx *ctx, int a, int b, float *ms);

/* ---- calibration probe (counterpart of the reference's microbenchmark
 *      benchmarks/bandwidth.zig) ---------------------------------------- */
/* Streaming 128-bit reads over the first `bytes` of buf, `iters` times: GB/s,
 * the best of three read patterns (grid-stride nontemporal loads; per-CU
 * contiguous slices with 32 or 16 register loads in flight per thread). */
int zh_stream_read_probe(zh_ctx *ctx, const zh_buf *buf, uint64_t bytes, uint32_t iters, float *gbs);

/* ---- synthetic data (seeded, bit-identical to oracle/zinc_oracle.c) ----- */
/* Fill rows x cols of `qtype` blocks at `offset` per the BASELINE distributions.
 * qtype | 0x100 (Q4_K / Q5_K): model-init variant with dmin = f16(7.5*d) /
 * f16(15.5*d), so
 * sub-block weights are zero-mean; the synthetic models use it. */
int zh_synth_tensor(zh_ctx *ctx, zh_buf *buf, uint64_t offset, uint32_t qtype,
                    uint64_t rows, uint64_t cols, uint64_t seed, uint64_t stream);
/* kind 0: N(0,1)*scale f32; 1: N(0,1) f16; 2: norm weight 1+U(-.01,.01) f32 */
int zh_synth_vector(zh_ctx *ctx, zh_buf *buf, uint64_t offset, uint32_t kind, uint64_t n,
                    float scale, uint64_t seed, uint64_t stream);

/* ---- quantized DMMV --------------------------------------------------- */
/* y[y_off..] (=, or += when acc_mode==1) = dequant(W[a_off..]) (MxK) * x[x_off..].
 * Replaces DmmvDispatch.recordDispatch (dmmv.zig:806-874) / dispatchDmmvInner
 * (forward.zig:8431-8540) with DmmvPushConstants{M,K,a_offset,x_offset,
 * y_offset,acc_mode} (dmmv.zig:21-28). Offsets are BYTES (4-byte aligned; a_off
 * 16-byte aligned for Q4_K). qtype: Q4_K, Q5_K, Q6_K (K % 256 == 0), Q8_0 and
 * MXFP4 (K % 32 == 0). */
int zh_dmmv(zh_ctx *ctx, uint32_t qtype, const zh_buf *W, uint64_t a_off,
            const zh_buf *x, uint64_t x_off, zh_buf *y, uint64_t y_off,
            uint32_t M, uint32_t K, uint32_t acc_mode);
/* 1 when zh_dmmv / zh_dmmv_xq / zh_dmmv_moe have a kernel for (qtype, K), 0
 * otherwise -- the counterpart of DmmvDispatch.pipelineForType returning null
 * (dmmv.zig:676-690), so a caller can fall back before it calls. */
int zh_dmmv_supported(uint32_t qtype, uint32_t K);
/* Batched DMMV (a skinny GEMM over num_cols activation vectors): replaces
 * DmmvDispatch.recordBatchDispatchPush (dmmv.zig:880-925, BatchDmmvPushConstants
 * {M,K,a_offset,x_offset,y_offset,num_cols} dmmv.zig:31-38; dmmv_q4k_batch.comp /
 * dmmv_q6k_batch.comp). X: f32 [num_cols][K] (column v at X + v*K*4 bytes,
 * 16-byte aligned offset); Y: f32 [num_cols][M] (= or += when acc_mode == 1).
 * qtype Q4_K or Q6_K, K % 256 == 0, num_cols 1..ZH_DMMV_MAX_COLS. The weights
 * stream from HBM once for all columns. */
#define ZH_DMMV_MAX_COLS 16
int zh_dmmv_batched(zh_ctx *ctx, uint32_t qtype, const zh_buf *W, uint64_t a_off, const zh_buf *X, uint64_t x_off,
                    zh_buf *Y, uint64_t y_off, uint32_t M, uint32_t K, uint32_t num_cols, uint32_t acc_mode);
/* (The columns agree with zh_dmmv run per column to the f32 summation
 * floor; bit for bit where zh_dmmv runs the same tile kernels, i.e. not for
 * Q4_K at K = 2048 / 4096, which zh_dmmv streams with another summation
 * order.) */
/* Y[v] = silu(Wg X[v]) * (Wu X[v]) for v < num_cols (Q4_K), the batched form of
 * zh_dmmv_fused_gate_up_swiglu below; layouts as zh_dmmv_batched. */
int zh_dmmv_fused_gate_up_swiglu_batched(zh_ctx *ctx, uint32_t qtype, const zh_buf *Wg, uint64_t g_off,
                                         const zh_buf *Wu, uint64_t u_off, const zh_buf *X, uint64_t x_off,
                                         zh_buf *Y, uint64_t y_off, uint32_t M, uint32_t K, uint32_t num_cols);
/* y = silu(Wg x) * (Wu x): dispatchDmmvFusedGateUpSwiglu (forward.zig:8237-8273,
 * dmmv_q4k_fused_gate_up_swiglu.comp). Both matrices share qtype. */
int zh_dmmv_fused_gate_up_swiglu(zh_ctx *ctx, uint32_t qtype, const zh_buf *Wg, uint64_t g_off,
                                 const zh_buf *Wu, uint64_t u_off, const zh_buf *x, uint64_t x_off,
                                 zh_buf *y, uint64_t y_off, uint32_t M, uint32_t K);
/* Expert-gathered DMMV (recordMoeDispatch, dmmv.zig:709; MoeDmmvPushConstants
 * dmmv.zig:41-48; dmmv_q4k_moe_kpar.comp:56-95): for slot s < n_used,
 * e = routing[s] (u32 ids at the start of `routing`),
 * y[y_off + s*M*4 ..] = W[e*expert_stride ..] * x[x_off + s*x_expert_stride*4 ..].
 * The ids are read on the device only (the call enqueues and returns): an id
 * at or past the experts W holds is clamped to the last one, and the next
 * zh_sync returns ZH_ERR_INVALID_ARGUMENT for it. */
int zh_dmmv_moe(zh_ctx *ctx, uint32_t qtype, const zh_buf *W, uint64_t expert_stride,
                const zh_buf *routing, const zh_buf *x, uint32_t x_expert_stride, uint64_t x_off,
                zh_buf *y, uint64_t y_off, uint32_t M, uint32_t K, uint32_t n_used);
/* Pre-quantised activations ("XQ": per 32-element block, three int8 limbs of
 * a 22-bit fixed-point value plus an f32 power-of-two scale and partial
 * sums; zh_xq_bytes(K) bytes per vector). A caller that feeds one activation
 * to several matrices (Q/K/V, gate/up) quantises once; the reference has no
 * counterpart (its shaders read f32 x directly, dmmv_q4k.comp:90-104).
 * x_stride: floats between vectors; vector v goes to xq_off + v*zh_xq_bytes(K). */
uint64_t zh_xq_bytes(uint32_t K);
int zh_quantize_activation(zh_ctx *ctx, const zh_buf *x, uint64_t x_off, uint32_t K, uint32_t n_vec,
                           uint32_t x_stride, zh_buf *xq, uint64_t xq_off);
/* zh_dmmv / zh_dmmv_fused_gate_up_swiglu over an XQ activation. */
int zh_dmmv_xq(zh_ctx *ctx, uint32_t qtype, const zh_buf *W, uint64_t a_off, const zh_buf *xq, uint64_t xq_off,
               zh_buf *y, uint64_t y_off, uint32_t M, uint32_t K, uint32_t acc_mode);
int zh_dmmv_fused_gate_up_swiglu_xq(zh_ctx *ctx, uint32_t qtype, const zh_buf *Wg, uint64_t g_off,
                                    const zh_buf *Wu, uint64_t u_off, const zh_buf *xq, uint64_t xq_off,
                                    zh_buf *y, uint64_t y_off, uint32_t M, uint32_t K);
/* Bit-exact dequantisation of rows [row0, row0+n_rows) to f32 (dequantRow,
 * forward.zig:242-465), used for the embedding gather and for parity tests. */
int zh_dequant_rows(zh_ctx *ctx, uint32_t qtype, const zh_buf *W, uint64_t a_off,
                    uint32_t row0, uint32_t n_rows, uint32_t K, zh_buf *out, uint64_t out_off);

/* ---- elementwise / norm / rope / attention / routing / sampling --------- */
/* rms_norm_mul.comp via dispatchRmsNorm (forward.zig:3408); cpuRmsNormMul
 * (forward.zig:618-626): out = w[i % w_len] * (x * 1/sqrt(mean(x^2)+eps)). */
int zh_rms_norm(zh_ctx *ctx, const zh_buf *x, uint64_t x_off, const zh_buf *w, uint32_t w_len,
                zh_buf *out, uint64_t out_off, uint32_t n, uint32_t n_groups, float eps);
/* swiglu.comp / cpuSwiGLU (forward_metal.zig:6567-6572) */
int zh_swiglu(zh_ctx *ctx, const zh_buf *g, uint64_t g_off, const zh_buf *u, uint64_t u_off,
              zh_buf *out, uint64_t out_off, uint32_t n);
/* Fused per-head Q/K RMSNorm + NeoX RoPE + fp16 KV write
 * (qk_norm_rope_kv_write.comp, dispatchQkNormRopeKvWrite forward.zig:4008).
 * q (f32, n_q_heads*head_dim) is normed+rotated in place; k is normed+rotated
 * and, with raw v, stored as fp16 into the caches at the physical slot of
 * logical token `position` (page table of 16-token pages, forward.zig:677-698).
 * Cache layout: [n_kv_heads][cache_tokens][head_dim] fp16. inv_freq holds
 * head_dim/2 f32 inverse frequencies (forward.zig:1495-1500). */
int zh_qk_norm_rope_kv_write(zh_ctx *ctx, zh_buf *q, const zh_buf *q_norm_w, const zh_buf *k,
                             const zh_buf *k_norm_w, const zh_buf *v, const zh_buf *inv_freq,
                             zh_buf *k_cache, zh_buf *v_cache, const zh_buf *page_table,
                             uint32_t n_pages, uint32_t cache_tokens, uint32_t n_q_heads,
                             uint32_t n_kv_heads, uint32_t head_dim, uint32_t position, float eps);
/* Paged GQA flash-decode over the fp16 cache, split along context with a
 * log-sum-exp merge (flash_attn.comp + flash_attn_split_merge.comp via
 * AttentionDispatch.recordFlashAttnSplit/SplitMerge, attention.zig:199-316;
 * oracle cpuAttention forward_metal.zig:6600-6646). out: f32[n_heads*head_dim].
 * attn_scale 0 => 1/sqrt(head_dim). */
int zh_flash_decode(zh_ctx *ctx, const zh_buf *q, const zh_buf *k_cache, const zh_buf *v_cache,
                    const zh_buf *page_table, uint32_t n_pages, uint32_t cache_tokens, zh_buf *out,
                    uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t seq_len,
                    float attn_scale);
/* zh_flash_decode that allocates nothing (no counterpart in the reference;
 * for callers that cannot allocate: code under HIP graph capture, serving
 * loops that forbid allocation). Same arguments and result as
 * zh_flash_decode, bit for bit. The split-K partials and merge counters live
 * in a 2 MiB device array per GPU, held until the process ends, instead of
 * the context's scratch; a shape whose partials exceed it is rejected with
 * ZH_ERR_INVALID_ARGUMENT (head_dim 128, GQA group <= 8 and <= 256 CUs always
 * fit). Every call on one GPU shares that array: calls that overlap on one
 * GPU (other streams, other contexts) race. */
int zh_flash_decode_noalloc(zh_ctx *ctx, const zh_buf *q, const zh_buf *k_cache, const zh_buf *v_cache,
                            const zh_buf *page_table, uint32_t n_pages, uint32_t cache_tokens, zh_buf *out,
                            uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t seq_len,
                            float attn_scale);
/* Causal batched attention for prefill (flash_attn_batched.comp via
 * AttentionDispatch.recordFlashAttnBatched, attention.zig:240-316): queries
 * seq_start .. seq_start+n_queries-1 (q: f32 [n_queries][n_heads*head_dim],
 * normed and roped), each over cache positions 0 .. its own, through the page
 * table. out: fp16 [n_queries][n_heads*head_dim] (the O projection's GEMM
 * input). fp16 operands on the MFMA units, f32 softmax and accumulation.
 * head_dim 128; attn_scale 0 => 1/sqrt(head_dim). */
int zh_flash_attn_batched(zh_ctx *ctx, const zh_buf *q, const zh_buf *k_cache, const zh_buf *v_cache,
                          const zh_buf *page_table, uint32_t n_pages, uint32_t cache_tokens, zh_buf *out,
                          uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim, uint32_t seq_start,
                          uint32_t n_queries, float attn_scale);
/* softmax_topk_v2.comp / topKSoftmax (forward.zig:496-537): routing gets
 * [ids u32 x k][weights f32 x k]. n <= 256, k <= 16. */
int zh_softmax_topk(zh_ctx *ctx, const zh_buf *logits, uint32_t n, uint32_t k, zh_buf *routing);
/* moe_weighted_acc.comp:23-33: a[i] += sum_j w_j * b[j*src_stride + i] with
 * w_j read from routing[k + j]. */
int zh_moe_weighted_acc(zh_ctx *ctx, zh_buf *a, const zh_buf *b, const zh_buf *routing,
                        uint32_t n, uint32_t n_used, uint32_t src_stride);
/* ArgmaxDispatch.record (argmax.zig:66-87): first (lowest-index) maximum,
 * as sampleGreedy's CPU scan (forward.zig:10343-10356). result: u32. */
int zh_argmax(zh_ctx *ctx, const zh_buf *logits, uint32_t n, zh_buf *result, uint64_t result_off);

/* ---- engine: InferenceEngine surface (forward.zig:1226-10983) ---------- */
/* Batched prefill projection (dispatchProjectionBatched, forward.zig:8147-8216;
 * recordMulMmQ4K dmmv.zig:1045-1094 / mul_mm_q4k.comp): Y[n][m] (+= when
 * acc_mode == 1) sum_k X[n][k] * W[m][k] for N tokens, on the MFMA units.
 * X: fp16, token-major [N][K] (16-byte aligned offset); Y: f32 token-major
 * [N][M]; W: Q4_K or Q6_K rows (K % 256 == 0), dequantised to fp16 tiles,
 * f32 accumulation. */
int zh_gemm_xw(zh_ctx *ctx, uint32_t qtype, const zh_buf *W, uint64_t a_off, const zh_buf *X, uint64_t x_off,
               zh_buf *Y, uint64_t y_off, uint32_t M, uint32_t K, uint32_t N, uint32_t acc_mode);

typedef struct zh_model_config {
    uint32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab;
    uint32_t n_experts, n_experts_used, expert_ffn; /* n_experts == 0 => dense */
    uint32_t max_ctx;                               /* KV capacity in tokens */
    uint32_t type_attn, type_ffn_gate_up, type_ffn_down, type_lm_head, type_embd, type_router;
    float rope_base, eps;
    uint64_t seed;                                  /* synthetic weights seed */
    /* 0: off. Else the layers llama.cpp's Q4_K_M / Q5_K_M recipe gives more
     * bits (use_more_bits: the first and last eighth of the layers and every
     * third layer between) hold attn_v and ffn_down (dense or expert) in this
     * type; the other layers use type_attn / type_ffn_down. */
    uint32_t type_more_bits, reserved;
} zh_model_config;

/* InferenceEngine.init (forward.zig:1226) on a seeded random-init model whose
 * tensors use the same stream numbering as the oracle. */
int zh_engine_create(zh_ctx *ctx, const zh_model_config *cfg, zh_engine **out);
void zh_engine_destroy(zh_engine *eng);                 /* deinit forward.zig:10849 */
/* Fill KV positions [0, n_tokens) with seeded N(0,1) fp16 values. */
int zh_engine_prefill_kv_random(zh_engine *eng, uint32_t n_tokens, uint64_t seed);
/* decodeStep(state, token, collect_output) (forward.zig:4299): runs one token
 * at `position`; with collect_output the greedy token is produced on device. */
int zh_engine_decode_step(zh_engine *eng, uint32_t token, uint32_t position, int collect_output);
/* prefillBatched(state, tokens) (forward.zig:9330-9735): tokens at positions
 * start_pos .. start_pos+n-1 as MFMA dequant-GEMM batches of up to 512 tokens
 * (fp16 operands, f32 accumulation); writes their K/V and leaves the last
 * token's hidden state as the decode state. With collect, its logits and
 * greedy token are produced (read them with zh_engine_sample_greedy /
 * zh_engine_logits). MoE models run the decode step per token. */
int zh_engine_prefill(zh_engine *eng, const uint32_t *tokens, uint32_t n, uint32_t start_pos, int collect);
/* sampleGreedy (forward.zig:10338): waits and returns the last argmax token. */
int zh_engine_sample_greedy(zh_engine *eng, uint32_t *token);
/* generate (forward.zig:10983-11192): feed prompt tokens from `start_pos`,
 * then greedy-decode max_tokens tokens (stopping after eos if eos != UINT32_MAX).
 * out_tokens receives up to max_tokens ids; *n_out the count. The decode
 * loop feeds each argmax back on device (no host round trip per token). */
int zh_engine_generate(zh_engine *eng, const uint32_t *prompt, uint32_t n_prompt, uint32_t start_pos,
                       uint32_t max_tokens, uint32_t eos, uint32_t *out_tokens, uint32_t *n_out);
/* Batched greedy decode of n_seq sequences in lockstep, one token each per
 * step: the decode batch of the reference's scheduler (src/scheduler/
 * scheduler.zig:27-110 activeDecoding, each request a generate(),
 * forward.zig:10983) on one weight stream. engines[v] (distinct) share the
 * weights of engines[0] and its context (zh_engine_create_shared(ctx, base,
 * ...) with base's own ctx); prompts [n_seq][n_prompt]; all sequences start
 * at start_pos; out_tokens [n_seq][max_tokens] (no EOS stop). The Q/K/V, O,
 * gate/up, down and LM-head mat-vecs run as batched DMMV launches
 * (zh_dmmv_batched), attention per sequence. Dense models whose projections
 * are Q4_K / Q6_K (ZH_ERR_UNSUPPORTED_QUANT_TYPE otherwise). */
int zh_engine_generate_batch(zh_engine *const *engines, uint32_t n_seq, const uint32_t *prompts, uint32_t n_prompt,
                             uint32_t start_pos, uint32_t max_tokens, uint32_t *out_tokens);
/* Copy the last logits (vocab f32) to host. */
int zh_engine_logits(zh_engine *eng, float *dst);
/* Copy the hidden state (hidden f32) after the last step to host. */
int zh_engine_hidden(zh_engine *eng, float *dst);
/* No counterpart in the reference (inspection, for parity tests): the
 * n_experts_used expert ids and routing weights the last decode step's router
 * top-k selected in `layer` (MoE models; ZH_ERR_INVALID_ARGUMENT otherwise). */
int zh_engine_routing(zh_engine *eng, uint32_t layer, uint32_t *ids, float *weights);
/* No counterpart in the reference (test hook): make the per-XCD MoE launch run
 * the given experts (ids [n_layers][n_experts_used], n = their count) instead
 * of its own selection, weighted by the softmax over their router logits; the
 * selection it computed is still what zh_engine_routing returns. ids = NULL
 * switches it off. ZH_ERR_INVALID_ARGUMENT for models that do not take that
 * launch. For parity tests that follow another implementation's routing
 * through near ties. */
int zh_engine_force_routing(zh_engine *eng, const uint32_t *ids, uint32_t n);
/* Weight tensor by oracle stream id ((layer+1)<<8 | kind, or 1/2/3 globals). */
int zh_engine_tensor(zh_engine *eng, uint64_t stream, zh_buf **buf, uint64_t *offset, uint64_t *bytes);
/* Gather n logical tokens of layer `layer` K (which=0) or V (1) as fp16,
 * logical-token-major [t][kv_head][head_dim] (the oracle's layout). */
/* The sequence's KV page table: logical 16-token page i of every layer's
 * cache lives in physical page pages[i] (logicalTokenToPhysicalToken,
 * forward.zig:677-698). n == max_ctx / 16, entries < max_ctx / 16. Replaces
 * handing the request's KvPagePool pages to the engine (the reference keeps
 * the table in a device buffer, forward.zig:1312). An identity table keeps
 * the lookup-free attention kernel; any other selects the paged kernel. */
int zh_engine_set_pages(zh_engine *eng, const uint32_t *pages, uint32_t n);
/* Run the decode step's layers as one persistent launch (on != 0) instead of
 * per-phase kernels, where the model takes it (dense, Q4_K attention and
 * gate/up, Q6_K down, hidden 2048 / 4096, FFN 12288 / 14336, 4 q heads per
 * kv head; no engine sharing the device); elsewhere the per-phase kernels
 * run. No counterpart in the reference, which records one dispatch per
 * operation (decodeStep, forward.zig:4299). Default off. */
int zh_engine_set_persistent(zh_engine *eng, int on);
/* Run attn_norm + Q/K/V projections and the decode attention of each layer as
 * one launch (on != 0, the default) where it applies, on a device of 8 XCDs x
 * 32 CUs where each XCD owns 4 q heads (so the projection's outputs, the
 * split-K partials and their flags are exchanged through that XCD's L2): 8
 * kv heads of 128 dims with Q4_K Q/K/V over hidden 4096, or 4 kv heads of 8
 * q heads with Q8_0 Q/K/V over hidden 2048; identity page table, max_ctx <=
 * 65536, no engine sharing the device; elsewhere the two launches of
 * ZH_GROUP_QKV and ZH_GROUP_ATTN run. Replaces the reference's Q/K/V DMMV
 * dispatches plus its fused norm/RoPE/KV-write and flash-decode dispatches
 * (forward.zig:4776-4800, attention.zig:199-316). */
int zh_engine_set_fused_attn(zh_engine *eng, int on);
/* The dense FFN (ffn_norm, gate/up + SwiGLU, down + residual) as one launch
 * split by XCD (default on): XCD h computes FFN rows [1536 h, +1536), its
 * workgroups exchange the SwiGLU slice through the XCD's L2 and add the
 * down projection of that slice into the residual with device atomics.
 * Applies where the O projection runs inside the fused attention launch and
 * the layer is hidden 4096 / FFN 12288 / Q4_K gate, up / Q6_K down; the
 * residual stream is then carried between launches as a sum of two vectors.
 * Replaces the reference's ffn_norm, gate/up/SwiGLU and down dispatches
 * (forward.zig:8237-8290). */
int zh_engine_set_fused_ffn(zh_engine *eng, int on);

/* ---- KV page pool: KvPagePool (src/scheduler/kv_cache.zig:43-125) ------ */
int      zh_kv_pool_create(uint32_t total_pages, uint32_t page_size, zh_kv_pool **out);  /* init */
void     zh_kv_pool_destroy(zh_kv_pool *pool);                                            /* deinit */
/* allocPages: pops `count` ids off the free stack (a fresh pool hands out
 * total_pages-1, total_pages-2, ...); ZH_ERR_KV_CACHE_EXHAUSTED if too few. */
int      zh_kv_pool_alloc(zh_kv_pool *pool, uint64_t request_id, uint32_t count, uint32_t *page_ids);
void     zh_kv_pool_free(zh_kv_pool *pool, uint64_t request_id);                          /* freePages */
uint32_t zh_kv_pool_free_count(const zh_kv_pool *pool);                                  /* freeCount */
uint32_t zh_kv_pool_max_context(const zh_kv_pool *pool, uint32_t page_count);            /* maxContext */
int zh_engine_read_kv(zh_engine *eng, uint32_t layer, uint32_t which, uint32_t t0, uint32_t n,
                      uint16_t *dst);
/* Model bytes touched per decoded token at context length L (weights + fp16
 * KV + activations), the numerator of the bandwidth roofline. */
uint64_t zh_engine_bytes_per_token(zh_engine *eng, uint32_t L);

/* ---- sampling: SamplingParams / sampleFromLogits / sample
 *      (src/compute/forward.zig:95-105, 10229-10367) -------------------- */
typedef struct zh_sampling_params {
    float temperature;        /* 0: greedy */
    float top_p;              /* 1: off */
    float repetition_penalty; /* 1: off */
    uint32_t top_k;           /* candidates, clamped to 1..128 */
} zh_sampling_params;
/* sampleFromLogits over n f32 logits in a device buffer, on the device (the
 * reference reads the logits back and scans them on the host; here only the
 * token returns). history: the generated tokens (host memory; read only when
 * a repetition penalty applies). u: the value the reference draws with
 * random.float(f64) at that point, in [0, 1), used only when the choice is
 * random. No final-logit softcap (the models on the path have none).
 * n at most 262144. */
int zh_sample_logits(zh_ctx *ctx, const zh_buf *logits, uint64_t offset, uint32_t n, const zh_sampling_params *p,
                     const uint32_t *history, uint32_t n_history, double u, uint32_t *token);
/* InferenceEngine.sample (forward.zig:10360-10367) on the last step's logits:
 * sampleGreedy when the params need no logits, else sampleFromLogits. */
int zh_engine_sample(zh_engine *eng, const zh_sampling_params *p, const uint32_t *history, uint32_t n_history,
                     double u, uint32_t *token);

/* ---- GGUF model files: src/model/gguf.zig (parse) and src/model/loader.zig
 *      (extractConfig, load) --------------------------------------------- */
typedef struct zh_gguf zh_gguf;
/* Metadata value tags (GGUFType, gguf.zig:20-35). */
enum { ZH_GGUF_U8 = 0, ZH_GGUF_I8 = 1, ZH_GGUF_U16 = 2, ZH_GGUF_I16 = 3, ZH_GGUF_U32 = 4, ZH_GGUF_I32 = 5,
       ZH_GGUF_F32 = 6, ZH_GGUF_BOOL = 7, ZH_GGUF_STRING = 8, ZH_GGUF_ARRAY = 9, ZH_GGUF_U64 = 10,
       ZH_GGUF_I64 = 11, ZH_GGUF_F64 = 12 };
/* gguf.parse over a read-only private mmap of `path` (loader.zig:420-445,
 * gguf.zig:340-419): header, metadata map, tensor table; tensor data starts at
 * the next general.alignment boundary (default 32). Unlike the reference,
 * every read is bounds-checked: ZH_ERR_TRUNCATED_FILE instead of a fault. */
int  zh_gguf_open(const char *path, zh_gguf **out);
void zh_gguf_close(zh_gguf *f);
const char *zh_gguf_last_error(const zh_gguf *f);  /* detail of the last failure on f (or of open) */
uint32_t zh_gguf_version(const zh_gguf *f);
uint64_t zh_gguf_tensor_count(const zh_gguf *f);
uint64_t zh_gguf_metadata_count(const zh_gguf *f);
uint64_t zh_gguf_data_offset(const zh_gguf *f);    /* tensor_data_offset */
const void *zh_gguf_data(const zh_gguf *f);        /* the mapped file */
uint64_t zh_gguf_file_size(const zh_gguf *f);
/* Tensor i of the table: name (NUL-terminated, owned by f), n_dims, dims[4]
 * (unused dims 1), GGMLType, offset in the data section and sizeBytes
 * (gguf.zig:222-229; ZH_ERR_UNSUPPORTED_QUANT_TYPE for a type without a
 * block size). */
int zh_gguf_tensor_info(const zh_gguf *f, uint64_t i, const char **name, uint32_t *n_dims, uint64_t *dims,
                        uint32_t *type, uint64_t *offset, uint64_t *bytes);
/* findTensor (gguf.zig:305-310): index, or -1. */
int64_t zh_gguf_find_tensor(const zh_gguf *f, const char *name);
/* Metadata lookups with the reference's conversions (MetadataValue.asU32 /
 * asU64 / asF32 / asBool / asString, gguf.zig:143-193); ZH_ERR_NOT_FOUND when
 * the key is absent or the value does not convert (the reference's null). */
int zh_gguf_get_u32(const zh_gguf *f, const char *key, uint32_t *v);
int zh_gguf_get_u64(const zh_gguf *f, const char *key, uint64_t *v);
int zh_gguf_get_f32(const zh_gguf *f, const char *key, float *v);
int zh_gguf_get_bool(const zh_gguf *f, const char *key, int *v);
int zh_gguf_get_string(const zh_gguf *f, const char *key, const char **s, uint64_t *len);
/* Metadata entry i: key, value tag, and for arrays the element tag and count. */
int zh_gguf_metadata_entry(const zh_gguf *f, uint64_t i, const char **key, uint32_t *type, uint32_t *elem_type,
                           uint64_t *count);
/* extractConfig (loader.zig:81-346) for the architectures on the path,
 * qwen3 (dense) and qwen3moe: dimensions, eps, rope base, experts,
 * vocab (metadata, else output.weight / token_embd.weight rows), with the
 * per-class types read from blk.0's tensors (type_more_bits 0: the engine
 * takes each tensor's own type from the file). max_ctx is the caller's KV
 * capacity (rounded up to 16 tokens). Other architectures:
 * ZH_ERR_UNSUPPORTED_ARCHITECTURE. */
int zh_gguf_model_config(const zh_gguf *f, uint32_t max_ctx, zh_model_config *cfg);
/* loader.load + InferenceEngine.init (loader.zig:414-486, forward.zig:1226):
 * an engine whose weights are the file's tensors, each uploaded to the device
 * in its own storage type (a Q4_K_M file's Q6_K attn_v / ffn_down layers
 * included). Missing tensors: ZH_ERR_TENSOR_NOT_FOUND; a tensor whose shape
 * differs from the config: ZH_ERR_INVALID_ARGUMENT; a format the kernels do
 * not take: ZH_ERR_UNSUPPORTED_QUANT_TYPE. Without output.weight the LM head
 * reads token_embd.weight (tied embeddings). */
int zh_engine_create_gguf(zh_ctx *ctx, const zh_gguf *f, uint32_t max_ctx, zh_engine **out);
/* Concurrent sequences (no counterpart in the reference, whose engine decodes
 * one sequence): a second engine on context `ctx` (its own HIP stream) over
 * the weights of `base` -- own KV cache (max_ctx tokens, 0: base's), own
 * activations and step graph. Engines on different contexts decode
 * independent sequences at the same time from different host threads,
 * sharing one copy of the weights. Destroy sharing engines before base. */
int zh_engine_create_shared(zh_ctx *ctx, zh_engine *base, uint32_t max_ctx, zh_engine **out);
/* The storage type of an engine tensor (by stream id, as zh_engine_tensor). */
int zh_engine_tensor_type(zh_engine *eng, uint64_t stream, uint32_t *type);

/* Measurement entries (no counterpart in the reference; the benchmark uses
 * them for per-kernel bandwidth). A launch group is one per-layer stage of
 * the decode step: */
#define ZH_GROUP_QKV 1u      /* attn_norm + Q/K/V projections (one launch when fused) */
#define ZH_GROUP_ATTN 2u     /* q/k norm + RoPE + KV write + split-K attention + merge */
/* ZH_GROUP_QKV | ZH_GROUP_ATTN: both as the step runs them (one launch when
 * zh_engine_set_fused_attn applies) */
#define ZH_GROUP_O 4u        /* O projection + residual */
#define ZH_GROUP_FFN_IN 8u   /* ffn_norm + gate/up + SwiGLU (MoE: + router, top-k) */
#define ZH_GROUP_FFN_OUT 16u /* down projection + residual (MoE: + weighted expert sum) */
/* ZH_GROUP_FFN_IN | ZH_GROUP_FFN_OUT: both as the step runs them (one launch
 * when zh_engine_set_fused_ffn applies) */
#define ZH_GROUP_HEAD 32u    /* output_norm + LM head + argmax (not per layer) */
/* Average duration of one launch of `group`, replayed with the engine's own
 * arguments and state over `iters` launches rotating through the layers, by
 * HIP events on the engine's stream. Leaves the activations changed. */
int zh_engine_time_kernel(zh_engine *eng, uint32_t group, uint32_t iters, float *us_per_launch);
/* The kernels one launch group of layer 0 launches (mangled names, read
 * from the graph its launches capture into; ZH_GROUP_HEAD: the output head), joined with "; " into names. */
int zh_engine_group_kernels(zh_engine *eng, uint32_t group, char *names, size_t len);
/* Algorithmic bytes of one launch of `group` at context length L. */
uint64_t zh_engine_group_bytes(zh_engine *eng, uint32_t group, uint32_t L);

#ifdef __cplusplus
}
#endif
#endif /* ZINC_HIP_H */
