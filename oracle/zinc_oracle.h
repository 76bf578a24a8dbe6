/*
 * zinc_oracle.h — CPU restatement of ZINC's decode-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * backend in zinc_amd/. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product path never calls it and never
 * falls back to it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the zolotukhin/zinc source tree). The reference is Zig 0.15.2; no Zig
 * toolchain exists in this image, so the reference cannot be built and this
 * restatement is pinned by the reference's in-source known-answer tests,
 * closed forms and brute force (tests/test_oracle_*.py).
 */
#ifndef ZINC_ORACLE_H
#define ZINC_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGMLType enum values: src/model/gguf.zig:38-69 */
enum {
    ZO_F32 = 0, ZO_F16 = 1, ZO_Q8_0 = 8, ZO_Q4_K = 12, ZO_Q5_K = 13, ZO_Q6_K = 14, ZO_MXFP4 = 39
};

/* GGMLType.blockSize / bytesPerBlock: src/model/gguf.zig:75-124 */
uint32_t zo_block_size(uint32_t type);
uint32_t zo_bytes_per_block(uint32_t type);
/* TensorInfo.sizeBytes: src/model/gguf.zig:222-229 (row-wise: rows * cols/bs * bpb) */
uint64_t zo_tensor_bytes(uint32_t type, uint64_t rows, uint64_t cols);

/* IEEE binary16 <-> binary32 (round-to-nearest-even), as Zig @floatCast. */
float    zo_f16_to_f32(uint16_t h);
uint16_t zo_f32_to_f16(float f);

/* getScaleMinK4: src/compute/forward.zig:229-238 */
void zo_get_scale_min_k4(uint32_t j, const uint8_t *scales, uint8_t *sc, uint8_t *m);

/* dequantRow: src/compute/forward.zig:242-465 (F32, F16, Q8_0, Q6_K, Q5_K, Q4_K, MXFP4).
 * Returns 0 on success, -1 for an unsupported type (reference logs and zero-fills). */
int zo_dequant_row(const uint8_t *raw, uint32_t row, uint32_t cols, uint32_t type, float *out);

/* dotQ8_0Row: src/compute/forward_metal.zig:6890-6917 (8-lane partials, @reduce) */
float zo_dot_q8_0_row(const uint8_t *raw, uint32_t row, uint32_t cols, const float *x);

/* cpuDmmvFallback: src/compute/forward_metal.zig:6407-6435.
 * y[r] (=, or += when acc_mode==1 as DmmvPushConstants.acc_mode dmmv.zig:21-28)
 * = serial f32 dot(dequantRow(r), x). Rows split over nthreads (<=0: 1). */
int zo_dmmv(const uint8_t *W, uint32_t type, const float *x, float *y,
            uint32_t M, uint32_t K, uint32_t acc_mode, int nthreads);
/* Same, accumulating in f64 (error-bound reference; not in the reference). */
int zo_dmmv_f64(const uint8_t *W, uint32_t type, const float *x, double *y,
                uint32_t M, uint32_t K, int nthreads);
/* Sum over rows of |w_i * x_i| in f64: the magnitude that fp32 rounding of a
 * dot product scales with. */
int zo_dmmv_absdot(const uint8_t *W, uint32_t type, const float *x, double *y,
                   uint32_t M, uint32_t K, int nthreads);

/* cpuRmsNormMul: src/compute/forward.zig:618-626 */
void zo_rms_norm_mul(const float *in, const float *w, uint32_t w_len, float *out,
                     uint32_t n, uint32_t n_groups, float eps);
/* cpuPerHeadRmsNormMul: src/compute/forward_metal.zig:6482-6491 (in place) */
void zo_per_head_rms_norm(float *data, const float *w, uint32_t head_dim,
                          uint32_t n_heads, float eps);
/* RoPE inverse frequencies: src/compute/forward.zig:1495-1500 */
void zo_rope_inv_freq(float *inv_freq, uint32_t rope_dim, float base);
/* cpuRopeWithFreqs: src/compute/forward_metal.zig:6542-6564 (NeoX pairs i, i+rope_dim/2) */
void zo_rope(float *data, uint32_t stride, uint32_t rope_dim, uint32_t n_heads,
             uint32_t position, const float *inv_freq);
/* cpuSwiGLU: src/compute/forward_metal.zig:6567-6572 */
void zo_swiglu(const float *g, const float *u, float *out, uint32_t n);

/* cpuAttention: src/compute/forward_metal.zig:6600-6646, with K/V read from an
 * fp16 cache (the build's cache precision). k/v are logical-token-major:
 * k[t*kv_dim + kv_h*head_dim + d]. attn_scale 0 => 1/sqrt(head_dim). */
void zo_attention_f16(const float *q, const uint16_t *k, const uint16_t *v, float *out,
                      uint32_t head_dim, uint32_t n_heads, uint32_t n_kv_heads,
                      uint32_t seq_len, float attn_scale);

/* topKSoftmax: src/compute/forward.zig:496-537 */
void zo_topk_softmax(const float *logits, uint32_t n, uint32_t k, uint32_t *ids, float *w);
/* sampleGreedy CPU scan: src/compute/forward.zig:10343-10356 (first max wins) */
uint32_t zo_argmax(const float *logits, uint32_t n);
/* SamplingParams.requiresLogitsReadback and sampleFromLogits
 * (src/compute/forward.zig:95-105, 10229-10334), no softcap; u is the
 * caller's random.float(f64) draw. */
int      zo_sampling_requires_readback(float temperature, float top_p, float repetition_penalty);
uint32_t zo_sample_from_logits(const float *logits, uint32_t n, const uint32_t *hist, uint32_t nh,
                               float temperature, float top_p, float rep_pen, uint32_t top_k, double u);
/* kvPageCountForContext / logicalTokenToPhysicalToken: src/compute/forward.zig:677-698.
 * Returns -1 for ContextLengthExceeded. */
int64_t zo_logical_to_physical(const uint32_t *page_ids, uint32_t n_pages, uint32_t logical);
uint32_t zo_kv_page_count(uint32_t context_tokens);

/* ---- Seeded synthetic data (shared spec with the HIP generator) ---- */
uint64_t zo_rand(uint64_t seed, uint64_t stream, uint64_t ctr);
float    zo_normal(uint64_t r);
/* Fill a rows x cols tensor of `type` with BASELINE-distributed random blocks.
 * type | 0x100 (Q4_K / Q5_K): model-init variant, dmin = f16(7.5*d) / f16(15.5*d).
 * type | 0x200 | e << 12 (Q8_0): a router, d = f16(d * 2^-e). */
int  zo_synth_tensor(uint8_t *dst, uint32_t type, uint64_t rows, uint64_t cols,
                     uint64_t seed, uint64_t stream);
/* e of the router flag for a router with K columns: router logits of an
 * RMS-normed input about N(0,1) */
uint32_t zo_router_shift(uint64_t K);
void zo_synth_normal_f32(float *dst, uint64_t n, float scale, uint64_t seed, uint64_t stream);
void zo_synth_normal_f16(uint16_t *dst, uint64_t n, uint64_t seed, uint64_t stream);
void zo_synth_norm_weight(float *dst, uint64_t n, uint64_t seed, uint64_t stream);

/* ---- Whole-model decode step (dense Qwen3 and qwen3moe shapes) ---- */
typedef struct zo_model_config {
    uint32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab;
    uint32_t n_experts, n_experts_used, expert_ffn; /* n_experts==0 => dense */
    uint32_t max_ctx;
    uint32_t type_attn, type_ffn_gate_up, type_ffn_down, type_lm_head, type_embd, type_router;
    float rope_base, eps;
    uint64_t seed;
    /* 0: off. Else the layers llama.cpp's Q4_K_M / Q5_K_M recipe gives more
     * bits (use_more_bits: the first and last eighth of the layers and every
     * third layer between) hold attn_v and ffn_down (dense or expert) in this
     * type; the other layers use type_attn / type_ffn_down. */
    uint32_t type_more_bits, reserved;
} zo_model_config;
/* use_more_bits(i_layer, n_layers) of llama.cpp's quantizer (the rule the
 * Q4_K_M mix of GGUF files follows). */
int zo_more_bits_layer(uint32_t i, uint32_t n);

typedef struct zo_model zo_model;
zo_model *zo_model_create(const zo_model_config *cfg, int nthreads);
void      zo_model_destroy(zo_model *m);
/* Fill KV positions [0, n) of every layer with N(0,1) fp16 values (identity page map). */
void      zo_model_prefill_kv_random(zo_model *m, uint32_t n, uint64_t seed);
/* One decodeStep (src/compute/forward.zig:4299-7865) at position `pos`; writes
 * logits (vocab floats) if non-NULL and returns the greedy token. */
uint32_t  zo_model_decode_step(zo_model *m, uint32_t token, uint32_t pos, float *logits);
/* Raw access for tests: tensor bytes by stream id, hidden state after step. */
const uint8_t *zo_model_tensor(zo_model *m, uint64_t stream, uint64_t *bytes);
/* Storage type of a tensor (0 for the f32 norms), -1 if the model has none. */
int       zo_model_tensor_type(zo_model *m, uint64_t stream);
/* Replace a tensor's data and storage type (a weight loaded from a file):
 * n must be its size in that type; 0 on success, < 0 on a mismatch. */
int       zo_model_set_tensor(zo_model *m, uint64_t stream, uint32_t type, const void *src, uint64_t n);
const float   *zo_model_hidden(zo_model *m);
/* test diagnostic: smallest relative router top-k gap of the last step */
float          zo_model_route_gap(const zo_model *m);
/* test diagnostic: the experts the last decode step selected in `layer`
 * (n_experts_used ids and weights, in topKSoftmax's order) and that layer's
 * router gap as zo_model_route_gap's (INFINITY: no tie, e.g. a selection
 * holding zero-probability experts); -1 for a dense model */
int            zo_model_routing(const zo_model *m, uint32_t layer, uint32_t *ids, float *weights, float *gap);
/* fp16 K (which 0) or V (1) cache row of `token` in `layer`: n_kv_heads*head_dim values. */
const uint16_t *zo_model_kv(zo_model *m, uint32_t layer, uint32_t which, uint32_t token);

#ifdef __cplusplus
}
#endif
#endif
