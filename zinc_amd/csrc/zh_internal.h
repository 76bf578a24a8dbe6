// zh_internal.h — host-side internals shared by the libzinc_hip.so sources.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>
#include <vector>

// Ablation switches for measuring one kernel path against another. Only a
// debug build (-DZH_DEBUG_KNOBS) reads them from the environment; the product
// build compiles every switch to its default.
#ifdef ZH_DEBUG_KNOBS
#include <stdlib.h>
static inline bool zh_knob(const char *name) { return getenv(name) != nullptr; }
static inline int zh_knob_int(const char *name, int dflt) {
    const char *e = getenv(name);
    return e ? atoi(e) : dflt;
}
#else
static inline bool zh_knob(const char *) { return false; }
static inline int zh_knob_int(const char *, int dflt) { return dflt; }
#endif

#include "../../include/zinc_hip.h"

struct zh_buf {
    void *ptr;
    uint64_t size;
};

struct zh_ctx {
    int device = 0;
    int cu_count = 0;
    int xcd_rr = -1;  // zhk_xcd_round_robin: -1 unknown, 0 no, 1 yes
    // Bumped by zh_sync when a bounded wait gave up, after it probed the
    // workgroup placement again (xcd_rr): every engine re-records its step
    // graph before its next step, which takes the per-group launches if the
    // placement the per-XCD launches rely on no longer holds.
    uint32_t place_gen = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev[64] = {};
    std::string err;
    // Stream-ordered scratch for zh_dmmv's activation quantisation.
    void *scratch = nullptr;
    uint64_t scratch_size = 0;
    // Other contexts run kernels on this device at the same time (engines
    // sharing weights): kernels must not wait on workgroups of their own grid
    // that may not be resident (the attention merge then needs no waiting).
    bool concurrent = false;
    // Device control words: err_dev[0] is the error word, which kernels OR
    // ZH_DEVERR_* bits into for input they had to clamp or a bounded wait
    // that gave up (the launch still completes); zh_sync reports and clears
    // it. err_dev[1] is the attention merge's wait limit in ticks of the
    // 100 MHz s_memrealtime clock, read by the kernels at run time so that a
    // captured graph follows zh_set_attn_wait_limit.
    uint32_t *err_dev = nullptr;
    // Device words of the cross-workgroup exchanges (flag and epoch words,
    // epoch-tagged values) of the engines on this context. A bounded wait
    // that gave up leaves them inconsistent (a late workgroup may publish
    // after its launch's epoch was abandoned), so zh_sync zeroes them all
    // when it reports ZH_ERR_WAIT_TIMEOUT: the next launch starts at epoch 1.
    struct XWords { const void *owner; void *p; uint64_t bytes; };
    std::vector<XWords> xwords;
};
enum : uint32_t { ZH_DEVERR_EXPERT_ID = 1u, ZH_DEVERR_ATTN_WAIT = 2u, ZH_DEVERR_STEP_BARRIER = 4u };
// default merge wait: 50 ms
constexpr uint32_t ZH_ATTN_WAIT_TICKS = 5000000u;

int zh_set_err(zh_ctx *ctx, int code, const char *fmt, ...);
#define ZH_HIP(ctx, call)                                                                    \
    do {                                                                                     \
        hipError_t e_ = (call);                                                              \
        if (e_ != hipSuccess)                                                                \
            return zh_set_err((ctx), ZH_ERR_HIP, "%s failed: %s", #call, hipGetErrorString(e_)); \
    } while (0)
#define ZH_LAUNCH_CHECK(ctx) ZH_HIP(ctx, hipGetLastError())

// Scratch (grows; stream ordered, so reuse across sequential calls is safe).
int zh_scratch(zh_ctx *ctx, uint64_t bytes, void **out);

static inline uint32_t zh_block_size(uint32_t t) {
    switch (t) {
    case ZH_Q8_0: case ZH_MXFP4: return 32;
    case ZH_Q4_K: case ZH_Q5_K: case ZH_Q6_K: return 256;
    default: return 1;
    }
}
static inline uint32_t zh_bytes_per_block(uint32_t t) {
    switch (t) {
    case ZH_F32: return 4;
    case ZH_F16: return 2;
    case ZH_Q8_0: return 34;
    case ZH_MXFP4: return 17;
    case ZH_Q4_K: return 144;
    case ZH_Q5_K: return 176;
    case ZH_Q6_K: return 210;
    default: return 0;
    }
}
static inline uint64_t zh_tensor_bytes(uint32_t t, uint64_t rows, uint64_t cols) {
    return rows * (cols / zh_block_size(t)) * zh_bytes_per_block(t);
}
static inline uint64_t zh_xq_bytes_int(uint32_t K) { return (uint64_t)(K / 32) * 108; }

// ---- raw-pointer launchers (stream = ctx->stream); validation done by callers
int zhk_quantize_xq(zh_ctx *ctx, const float *x, void *xq, uint32_t K, uint32_t n_vec,
                    uint32_t x_stride);
int zhk_dmmv(zh_ctx *ctx, uint32_t qtype, const uint8_t *W, const void *xq, float *y, uint32_t M,
             uint32_t K, uint32_t acc, float *ycopy = nullptr);  // ycopy: the outputs also stored there
// Up to three stacked matrices sharing K and x (e.g. Q, K, V) in one launch.
int zhk_dmmv_multi(zh_ctx *ctx, uint32_t qtype, uint32_t nseg, const uint8_t *const *W, float *const *y,
                   const uint32_t *M, const void *xq, uint32_t K);
int zhk_dmmv_gate_up(zh_ctx *ctx, uint32_t qtype, const uint8_t *Wg, const uint8_t *Wu,
                     const void *xq, float *y, uint32_t M, uint32_t K);
// LDS-staged DMMV (MoE router): f32 activation staged per workgroup with an
// optional fused RMSNorm; optional XQ copy of the staged activation and router
// top-k by the last workgroup (cnt zero between launches).
bool zhk_dmmv_lds_supported(uint32_t qtype, uint32_t K);
int zhk_dmmv_lds_plain(zh_ctx *ctx, uint32_t qtype, uint32_t nseg, const uint8_t *const *W, float *const *y,
                       const uint32_t *M, const float *x, const float *norm_w, float eps, uint32_t K,
                       uint32_t acc, void *xq_out, uint32_t topk, uint32_t *routing_out, uint32_t *cnt);
// Expert down projections of n_slots selected experts + routing-weighted sum into y (y += ...);
// XQ inputs, slot stride 108 K/32 bytes.
int zhk_dmmv_lds_down_acc(zh_ctx *ctx, uint32_t qtype, const uint8_t *W, uint64_t expert_stride,
                          const uint32_t *routing, uint32_t n_slots, uint32_t n_experts, const void *xq, float *y,
                          uint32_t M, uint32_t K);
int zhk_dmmv_moe(zh_ctx *ctx, uint32_t qtype, const uint8_t *W, uint64_t expert_stride,
                 const uint32_t *routing, const void *xq, uint64_t xq_slot_stride, float *y,
                 uint32_t M, uint32_t K, uint32_t n_used, int gate_up, const uint8_t *W2, uint32_t n_experts,
                 uint32_t *err = nullptr);
int zhk_dequant_rows(zh_ctx *ctx, uint32_t qtype, const uint8_t *W, uint32_t row0, uint32_t n_rows,
                     uint32_t K, float *out, const uint32_t *row_from_dev, uint32_t clamp_rows, uint32_t gather = 0);
uint32_t zh_router_shift(uint64_t K);  // the router flag's shift of zhk_synth_tensor (zh_runtime.hip)
int zhk_synth_tensor(zh_ctx *ctx, uint8_t *dst, uint32_t qtype, uint64_t rows, uint64_t cols,
                     uint64_t seed, uint64_t stream);
int zhk_synth_vector(zh_ctx *ctx, void *dst, uint32_t kind, uint64_t n, float scale, uint64_t seed,
                     uint64_t stream);
int zhk_rms_norm(zh_ctx *ctx, const float *x, const float *w, uint32_t w_len, float *out, void *xq,
                 uint32_t n, uint32_t n_groups, float eps);
int zhk_swiglu(zh_ctx *ctx, const float *g, const float *u, float *out, uint32_t n);
// y = W x for f32 weights (row-major M x K, K % 4 == 0).
int zhk_matvec_f32(zh_ctx *ctx, const float *W, const float *x, float *y, uint32_t M, uint32_t K);
struct zh_pos_src {  // where a kernel reads the position: host scalar or device word
    uint32_t value;
    const uint32_t *dev;  // if non-null: position = *dev + value
};
int zhk_qk_norm_rope_kv(zh_ctx *ctx, float *q, const float *qw, const float *k, const float *kw,
                        const float *v, const float *inv_freq, uint16_t *kc, uint16_t *vc,
                        const uint32_t *pages, uint32_t n_pages, uint32_t cache_tokens,
                        uint32_t nq, uint32_t nkv, uint32_t hd, zh_pos_src pos, float eps,
                        uint32_t n_tok = 1);  // n_tok rows of q / k / v at positions pos .. pos + n_tok - 1
int zhk_flash_decode(zh_ctx *ctx, const float *q, const uint16_t *kc, const uint16_t *vc,
                     const uint32_t *pages, uint32_t n_pages, uint32_t cache_tokens, float *out,
                     void *xq_out, uint32_t nh, uint32_t nkv, uint32_t hd, zh_pos_src seq_len,
                     uint32_t max_seq, float scale, float *partials);
uint64_t zhk_flash_decode_partials_bytes(uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_seq);
// Fused decode attention: q/k RMSNorm + RoPE, KV write of the new token at
// `pos`, attention over [0, pos], chunk merge. `partials` as above, with its
// trailing counter words zero before the first launch.
// RoPE table cs[pos][64] = (cos, sin) of pos * inv_freq (head_dim 128)
int zhk_rope_table(zh_ctx *ctx, const float *inv_freq, uint32_t n_pos, float *cs);
int zhk_attn_decode_fused(zh_ctx *ctx, const float *q, const float *k, const float *v, const float *qw,
                          const float *kw, const float *rope_cs, uint16_t *kc, uint16_t *vc,
                          const uint32_t *pages, uint32_t n_pages, uint32_t cache_tokens, float *out,
                          void *xq_out, uint32_t nh, uint32_t nkv, zh_pos_src pos, uint32_t max_seq,
                          float scale, float eps, float *partials, bool ident_pages);
int zhk_attn_decode_fused_z(zh_ctx *ctx, uint32_t n, const float *const *q, const float *const *k,
                            const float *const *v, const float *qw, const float *kw, const float *rope_cs,
                            uint16_t *const *kc, uint16_t *const *vc, const uint32_t *pages, uint32_t n_pages,
                            uint32_t cache_tokens, float *const *out, void *const *xq_out, uint32_t nh, uint32_t nkv,
                            const uint32_t *const *pos_dev, uint32_t max_seq, float scale, float eps,
                            float *const *partials);
// Prefill (zh_prefill.hip)
int zhk_gemm(zh_ctx *ctx, uint32_t qtype, const uint8_t *W, const _Float16 *X, uint32_t ldx, float *Y, uint32_t ldy,
             uint32_t M, uint32_t K, uint32_t N, uint32_t acc, const float *x_unscale = nullptr);
// Epilogue of the stacked q | k | v projection (head_dim 128): q/k RMSNorm +
// RoPE, q written back in place, k and v into the KV cache (the work of
// zhk_qk_norm_rope_kv, fused into the split-K sums when K is split).
struct zh_gemm_rope {
    const float *q_norm, *k_norm, *inv_freq;
    uint16_t *kc, *vc;
    const uint32_t *pages;
    uint32_t n_pages, cache_tokens, nq, nkv, pos0;
    float eps;
};
// Up to three stacked matrices sharing X (segment rows multiples of 64).
int zhk_gemm_multi(zh_ctx *ctx, uint32_t qtype, uint32_t nseg, const uint8_t *const *W, const _Float16 *X,
                   uint32_t ldx, float *const *Y, const uint32_t *ldy, const uint32_t *M, uint32_t K, uint32_t N,
                   uint32_t acc, const float *x_unscale = nullptr, const float *norm_w = nullptr,
                   _Float16 *norm_out = nullptr, float eps = 0.f, const zh_gemm_rope *rope = nullptr);
// Y (+)= X W^T (one matrix, Y rows M apart), then norm_out = fp16 RMSNorm of
// Y's rows times norm_w (the next GEMM's input; fused into the split-K
// epilogue when K is split).
int zhk_gemm_norm(zh_ctx *ctx, uint32_t qtype, const uint8_t *W, const _Float16 *X, uint32_t ldx, float *Y,
                  uint32_t M, uint32_t K, uint32_t N, uint32_t acc, const float *x_unscale, const float *norm_w,
                  _Float16 *norm_out, float eps);
int zhk_rms_norm_rows_f16(zh_ctx *ctx, const float *x, const float *w, _Float16 *out, uint32_t n, uint32_t rows,
                          float eps);
int zhk_swiglu_rows_f16(zh_ctx *ctx, const float *g, const float *u, _Float16 *out, float *unscale, uint32_t n,
                        uint32_t rows);
int zhk_attn_prefill(zh_ctx *ctx, const float *q, const uint16_t *kc, const uint16_t *vc, const uint32_t *pages,
                     uint32_t n_pages, uint32_t cache_tokens, uint32_t nq, uint32_t nkv, uint32_t hd, uint32_t pos0,
                     uint32_t N, float scale, _Float16 *out);
int zhk_softmax_topk(zh_ctx *ctx, const float *logits, uint32_t n, uint32_t k, uint32_t *routing);
int zhk_moe_weighted_acc(zh_ctx *ctx, float *a, const float *b, const uint32_t *routing, uint32_t n,
                         uint32_t n_used, uint32_t src_stride);
int zhk_argmax(zh_ctx *ctx, const float *logits, uint32_t n, uint32_t *result, uint32_t *partials,
               uint32_t *token_ring, const uint32_t *ring_index);

// Lane-per-block K-quant DMMV (zh_dmmv_lpb.hip): stages f32 x (optionally
// RMS-normalised with norm_w) into LDS itself. mode 0: plain (up to 3 stacked
// matrices), mode 1: fused gate/up/SwiGLU (Q4_K, W = gate, W2 = up).
// Device sampling (zh_sample.hip).
bool zhk_sampling_requires_readback(const zh_sampling_params *s);
uint32_t zhk_sample_max_vocab();
int zhk_sample(zh_ctx *ctx, const float *logits, uint32_t n, const uint32_t *hist, uint32_t nh,
               const zh_sampling_params *s, double u, uint64_t *keys, uint32_t *out);
int zhk_sample_host(zh_ctx *ctx, const float *logits, uint32_t n, const zh_sampling_params *s,
                    const uint32_t *history, uint32_t nh, double u, uint32_t *token);
bool zhk_lpb_supported(uint32_t qtype, uint32_t K);
int zhk_dmmv_lpb(zh_ctx *ctx, uint32_t qtype, int mode, uint32_t nseg, const uint8_t *const *W, const uint8_t *W2,
                 float *const *y, const uint32_t *M, const float *x, const float *norm_w, float eps,
                 float *normed_out, uint32_t K, uint32_t acc, const void *xq = nullptr,
                 uint8_t *xq_out = nullptr, uint32_t *grp_cnt = nullptr, float *ycopy = nullptr);
// Streaming Q4_K DMMV (zh_dmmv_ring.hip), same arguments as zhk_dmmv_lpb;
// returns -1 (nothing launched) for shapes it does not take.
int zhk_dmmv_ring(zh_ctx *ctx, uint32_t qtype, int mode, uint32_t nseg, const uint8_t *const *W, const uint8_t *W2,
                  float *const *y, const uint32_t *M, const float *x, const float *norm_w, float eps,
                  float *normed_out, uint32_t K, uint32_t acc, const void *xq, uint8_t *xq_out, uint32_t *grp_cnt);
// Batched DMMV: y[s * n_vec + v] (+)= W[s] x_v, x_v = x[v] (f32, optional
// fused RMSNorm) or xq[v] (XQ, x == nullptr); mode 0 plain, 1 gate/up+SwiGLU.
int zhk_dmmv_batched(zh_ctx *ctx, uint32_t qtype, int mode, uint32_t nseg, const uint8_t *const *W, const uint8_t *W2,
                     const uint32_t *M, uint32_t K, uint32_t n_vec, const float *const *x, const void *const *xq,
                     float *const *y, const float *norm_w, float eps, uint32_t acc);

// Persistent decode-layers kernel (zh_step.hip): the layers [l0, l1) of one
// decode step in one launch of one workgroup per CU, the phases (Q/K/V,
// attention, O, gate/up, down) separated by grid barriers.
struct zh_step_layer {  // one layer's weights and cache (a device table of these)
    const uint8_t *wq, *wk, *wv, *wo, *gate, *up, *down;
    const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
    uint16_t *kc, *vc;
};
struct zh_step_args {
    const zh_step_layer *layers;  // device table, [n_layers]
    uint32_t l0, l1;
    uint32_t hidden, n_heads, n_kv_heads, ffn, max_ctx;
    float eps, scale;
    float *x, *q, *k, *v, *attn, *s;  // residual stream and activations
    uint8_t *xq_attn, *xq_s;          // XQ images of the attention and SwiGLU outputs
    uint32_t *grp_cnt;                // SwiGLU XQ group counters (zero between launches)
    const float *rope_cs;
    const uint32_t *pages;
    uint32_t n_pages, ident;
    zh_pos_src pos;                   // position of the token
    float *part;                      // attention partials: n_heads x (CUs / n_kv_heads) x 130 f32
    uint32_t *ctl;                    // zh_step_ctl_bytes() zeroed bytes (barriers, merge counters)
};
uint64_t zh_step_ctl_bytes();
// Q/K/V projection + decode attention in one launch (zh_qkv_attn.hip) on a
// 256-CU device of 8 XCDs, identity page table, the device to itself: 8 kv
// heads (one per XCD), Q4_K Q/K/V with K = 4096; or 4 kv heads of 8 q heads
// (two XCDs each), Q8_0 Q/K/V with K = 2048 (hidden selects the shape);
// contexts up to 65536.
bool zhk_xcd_round_robin(zh_ctx *ctx);
bool zhk_qkv_attn_supported(zh_ctx *ctx, uint32_t hidden, uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_ctx);
uint32_t zhk_qkv_attn_flag_words();  // zeroed u32 words the caller keeps per engine
// The split residual's atomic part: 64-bit fixed point in units of 2^-24
// (zh_xcd.h fix_add / fix_to_f), so that its sums do not depend on the order
// of the atomics.
typedef long long zh_fix;
int zhk_qkv_attn(zh_ctx *ctx, const uint8_t *wq, const uint8_t *wk, const uint8_t *wv, const float *x,
                 const float *norm_w, float *q, float *k, float *v, const float *qw, const float *kw,
                 const float *rope_cs, uint16_t *kc, uint16_t *vc, uint32_t cache_tokens, float *out, void *xq_out,
                 uint32_t nh, zh_pos_src pos, float scale, float eps, float *partials, uint32_t *flags,
                 const uint8_t *wo = nullptr, void *x_acc = nullptr, const zh_fix *xb = nullptr,
                 float *x_out = nullptr, zh_fix *zero = nullptr, uint32_t hidden = 4096, uint64_t *xrows = nullptr);
uint64_t zhk_qkv_attn_xrows_bytes();  // zeroed bytes the caller keeps per engine (xrows: the rows' exchange)
// xb != nullptr (with wo): the input is x + xb, stored into x_out (16 rows
// per workgroup); x_acc starts at zero (it is not x's copy), `zero` (H
// floats) is cleared. Per-XCD FFN (zh_ffn_xcd.hip) with the same split
// residual: xa + xb in, xout = xa + xb, the down projection added into acc,
// `zero` cleared; hidden 4096, FFN 12288, Q4_K gate/up, Q6_K down (read from
// the copy zhk_ffn_pack_down makes, zhk_ffn_pack_bytes per layer); `part`:
// zhk_ffn_part_bytes of scratch.
bool zhk_ffn_xcd_supported(zh_ctx *ctx, uint32_t hidden, uint32_t ffn);
uint32_t zhk_ffn_xcd_flag_words();
uint64_t zhk_ffn_pack_bytes();
uint64_t zhk_ffn_part_bytes();
int zhk_ffn_pack_down(zh_ctx *ctx, const uint8_t *q6k_down, uint8_t *packed);
// Per-XCD MoE FFN (zh_moe_xcd.hip): hidden 2048, 128 experts top-8, expert FFN
// 768, Q8_0 router, Q4_K experts (unmodified); x is a copy of y taken before
// the launch; scratch: zhk_moe_part_bytes (epoch-tagged exchange words).
bool zhk_moe_xcd_supported(zh_ctx *ctx, uint32_t hidden, uint32_t n_experts, uint32_t n_used, uint32_t expert_ffn);
uint32_t zhk_moe_xcd_flag_words();
uint64_t zhk_moe_part_bytes();
int zhk_moe_xcd(zh_ctx *ctx, const float *x, const float *norm_w, float eps, const uint8_t *router,
                const uint8_t *egate, const uint8_t *eup, const uint8_t *edown, void *y, void *scratch,
                uint32_t *routing, uint32_t *flags, const zh_fix *xb = nullptr, float *xout = nullptr,
                zh_fix *zero = nullptr,  // xb: the split residual (x = x + xb, stored into xout; zero cleared;
                                         // y then zh_fix, else f32)
                const uint32_t *force = nullptr);  // test hook: run these 8 expert ids instead of the selection
int zhk_ffn_xcd(zh_ctx *ctx, const float *xa, const zh_fix *xb, const float *norm_w, float eps, const uint8_t *wg,
                const uint8_t *wu, const uint8_t *packed, float *part, float *xout, zh_fix *acc, zh_fix *zero,
                uint32_t *flags);
// wo != nullptr (4 q heads per kv head): also the O projection, added into
// x_acc with device atomics; x must then be a copy of x_acc (x_acc changes
// during the launch).
// The geometry the kernel is built for (hidden 2048 or 4096 = n_heads x 128,
// FFN 12288 or 14336, 4 q heads per kv head, enough CUs); the caller checks
// the layer formats (Q4_K Q/K/V/O/gate/up, Q6_K down, 16-byte aligned) and
// that no other work shares the device. false: use the per-phase kernels.
bool zhk_step_supported(zh_ctx *ctx, const zh_step_args &a);
int zhk_step_layers(zh_ctx *ctx, const zh_step_args &a);
