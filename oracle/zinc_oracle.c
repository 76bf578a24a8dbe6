/*
 * zinc_oracle.c — CPU restatement of ZINC's decode-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker, never the product). Built with
 *   gcc -O3 -march=native -ffp-contract=off -fPIC -shared -pthread
 * so that every f32 multiply and add rounds separately, as Zig does without
 * @mulAdd. Reference citations are relative to the zolotukhin/zinc tree.
 */
#include "zinc_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <pthread.h>

/* ------------------------------------------------------------------ */
/* Block geometry: src/model/gguf.zig:75-124                           */
/* ------------------------------------------------------------------ */
uint32_t zo_block_size(uint32_t t) {
    switch (t) {
    case ZO_F32: case ZO_F16: return 1;
    case ZO_Q8_0: case ZO_MXFP4: return 32;
    case ZO_Q4_K: case ZO_Q5_K: case ZO_Q6_K: return 256;
    default: return 1;
    }
}
uint32_t zo_bytes_per_block(uint32_t t) {
    switch (t) {
    case ZO_F32: return 4;
    case ZO_F16: return 2;
    case ZO_Q8_0: return 34;
    case ZO_MXFP4: return 17;
    case ZO_Q4_K: return 144;
    case ZO_Q5_K: return 176;
    case ZO_Q6_K: return 210;
    default: return 0;
    }
}
uint64_t zo_tensor_bytes(uint32_t t, uint64_t rows, uint64_t cols) {
    uint64_t bs = zo_block_size(t), bpb = zo_bytes_per_block(t);
    return rows * ((cols + bs - 1) / bs) * bpb;
}

/* ------------------------------------------------------------------ */
/* binary16 conversions (exact widen; RNE narrow incl. subnormals)     */
/* ------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float zo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7F800000u | (man << 13));
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t zo_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) /* inf / nan */
        return sign | 0x7C00u | (a > 0x7F800000u ? 0x200u : 0);
    if (a >= 0x477FF000u) return sign | 0x7C00u; /* rounds to >= 65520 -> inf */
    if (a < 0x38800000u) {
        /* result is subnormal (or zero): value / 2^-24, rounded to even */
        if (a < 0x33000000u) return sign; /* < 2^-25: rounds to 0 */
        uint32_t e = a >> 23, man = (a & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e; /* 14..24 */
        uint32_t q = man >> shift, rem = man & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return sign | (uint16_t)q;
    }
    uint32_t q = ((a - 0x38000000u) >> 13); /* rebias 127->15 */
    uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return sign | (uint16_t)q;
}

static inline float rd_f16(const uint8_t *p) { return zo_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* ------------------------------------------------------------------ */
/* getScaleMinK4: src/compute/forward.zig:229-238                       */
/* ------------------------------------------------------------------ */
void zo_get_scale_min_k4(uint32_t j, const uint8_t *s, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* ------------------------------------------------------------------ */
/* dequantRow: src/compute/forward.zig:242-465                          */
/* ------------------------------------------------------------------ */
static const float kMxfp4Lut[16] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f,
                                    -0.f, -.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f};

int zo_dequant_row(const uint8_t *raw, uint32_t row, uint32_t cols, uint32_t type, float *out) {
    switch (type) {
    case ZO_F32: /* forward.zig:244-249 */
        memcpy(out, raw + (size_t)row * cols * 4, (size_t)cols * 4);
        return 0;
    case ZO_F16: /* forward.zig:250-257 */
        for (uint32_t i = 0; i < cols; i++) out[i] = rd_f16(raw + ((size_t)row * cols + i) * 2);
        return 0;
    case ZO_Q8_0: { /* forward.zig:258-275: out = i8 * scale */
        size_t bpr = cols / 32, ro = (size_t)row * bpr * 34;
        for (size_t b = 0; b < bpr; b++) {
            const uint8_t *bo = raw + ro + b * 34;
            float scale = rd_f16(bo);
            for (int j = 0; j < 32; j++) out[b * 32 + j] = (float)(int8_t)bo[2 + j] * scale;
        }
        return 0;
    }
    case ZO_Q6_K: { /* forward.zig:276-325 */
        size_t bpr = cols / 256, ro = (size_t)row * bpr * 210;
        for (size_t b = 0; b < bpr; b++) {
            const uint8_t *bb = raw + ro + b * 210;
            float d = rd_f16(bb + 208);
            const uint8_t *ql = bb, *qh = bb + 128;
            const int8_t *sc = (const int8_t *)(bb + 192);
            float *o = out + b * 256;
            for (int half = 0; half < 2; half++) {
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                    int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    /* Zig evaluates d * s * q left to right: (d*s)*q */
                    o[l + 0] = d * (float)sc[is + 0] * (float)q1;
                    o[l + 32] = d * (float)sc[is + 2] * (float)q2;
                    o[l + 64] = d * (float)sc[is + 4] * (float)q3;
                    o[l + 96] = d * (float)sc[is + 6] * (float)q4;
                }
                ql += 64; qh += 32; sc += 8; o += 128;
            }
        }
        return 0;
    }
    case ZO_Q4_K: { /* forward.zig:370-409 */
        size_t bpr = cols / 256, ro = (size_t)row * bpr * 144;
        for (size_t b = 0; b < bpr; b++) {
            const uint8_t *bb = raw + ro + b * 144;
            float d = rd_f16(bb), dmin = rd_f16(bb + 2);
            const uint8_t *scales = bb + 4, *qs = bb + 16;
            float *o = out + b * 256;
            for (int p = 0; p < 4; p++) {
                uint8_t sc0, m0, sc1, m1;
                zo_get_scale_min_k4(2 * p, scales, &sc0, &m0);
                zo_get_scale_min_k4(2 * p + 1, scales, &sc1, &m1);
                float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
                float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
                for (int l = 0; l < 32; l++) o[64 * p + l] = d1 * (float)(qs[32 * p + l] & 0xF) - mm1;
                for (int l = 0; l < 32; l++) o[64 * p + 32 + l] = d2 * (float)(qs[32 * p + l] >> 4) - mm2;
            }
        }
        return 0;
    }
    case ZO_Q5_K: { /* forward.zig:326-368: the fifth bit of element l of the
                     * 64-group p comes from qh[l] bit 2p (low half) / 2p+1 (high half) */
        size_t bpr = cols / 256, ro = (size_t)row * bpr * 176;
        for (size_t b = 0; b < bpr; b++) {
            const uint8_t *bb = raw + ro + b * 176;
            float d = rd_f16(bb), dmin = rd_f16(bb + 2);
            const uint8_t *scales = bb + 4, *qh = bb + 16, *qs = bb + 48;
            float *o = out + b * 256;
            for (int p = 0; p < 4; p++) {
                uint8_t sc0, m0, sc1, m1;
                zo_get_scale_min_k4(2 * p, scales, &sc0, &m0);
                zo_get_scale_min_k4(2 * p + 1, scales, &sc1, &m1);
                float d1 = d * (float)sc0, mm1 = dmin * (float)m0;
                float d2 = d * (float)sc1, mm2 = dmin * (float)m1;
                for (int l = 0; l < 32; l++) {
                    int lo = (qs[32 * p + l] & 0xF) | (((qh[l] >> (2 * p)) & 1) << 4);
                    int hi = (qs[32 * p + l] >> 4) | (((qh[l] >> (2 * p + 1)) & 1) << 4);
                    o[64 * p + l] = d1 * (float)lo - mm1;
                    o[64 * p + 32 + l] = d2 * (float)hi - mm2;
                }
            }
        }
        return 0;
    }
    case ZO_MXFP4: { /* forward.zig:441-459 */
        size_t bpr = cols / 32, ro = (size_t)row * bpr * 17;
        for (size_t b = 0; b < bpr; b++) {
            const uint8_t *bo = raw + ro + b * 17;
            uint8_t e = bo[0];
            float d = u2f(e == 0 ? 0x00400000u : ((uint32_t)e << 23));
            for (int j = 0; j < 16; j++) {
                out[b * 32 + j] = d * kMxfp4Lut[bo[1 + j] & 0xF];
                out[b * 32 + j + 16] = d * kMxfp4Lut[bo[1 + j] >> 4];
            }
        }
        return 0;
    }
    default: /* forward.zig:460-463: warn and zero-fill */
        memset(out, 0, (size_t)cols * 4);
        return -1;
    }
}

/* dotQ8_0Row: src/compute/forward_metal.zig:6890-6917 */
float zo_dot_q8_0_row(const uint8_t *raw, uint32_t row, uint32_t cols, const float *x) {
    size_t bpr = cols / 32, ro = (size_t)row * bpr * 34;
    float acc[8] = {0};
    for (size_t b = 0; b < bpr; b++) {
        const uint8_t *bo = raw + ro + b * 34;
        float scale = rd_f16(bo);
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 8; l++) {
                float qf = (float)(int8_t)bo[2 + c * 8 + l];
                acc[l] = acc[l] + (qf * scale) * x[b * 32 + c * 8 + l];
            }
    }
    /* @reduce(.Add) over a @Vector(8, f32): LLVM lowers it as a pairwise tree
     * (x86 shuffle reduction): (0+4,1+5,2+6,3+7) then (0+2,1+3) then (0+1). */
    float s4[4], s2[2];
    for (int i = 0; i < 4; i++) s4[i] = acc[i] + acc[i + 4];
    for (int i = 0; i < 2; i++) s2[i] = s4[i] + s4[i + 2];
    return s2[0] + s2[1];
}

/* ------------------------------------------------------------------ */
/* Threaded row loops                                                  */
/* ------------------------------------------------------------------ */
typedef struct {
    const uint8_t *W; uint32_t type; const float *x; float *y; double *yd;
    uint32_t M, K, acc, r0, r1; int mode; /* 0 f32, 1 f64, 2 absdot */
} dmmv_job;

static void *dmmv_worker(void *arg) {
    dmmv_job *j = (dmmv_job *)arg;
    float *row = (float *)malloc((size_t)j->K * sizeof(float));
    for (uint32_t r = j->r0; r < j->r1; r++) {
        if (j->mode == 0 && j->type == ZO_Q8_0) {
            float dot = zo_dot_q8_0_row(j->W, r, j->K, j->x);
            j->y[r] = j->acc ? j->y[r] + dot : dot;
            continue;
        }
        zo_dequant_row(j->W, r, j->K, j->type, row);
        if (j->mode == 0) { /* forward_metal.zig:6429-6433: serial f32 dot */
            float dot = 0.f;
            for (uint32_t d = 0; d < j->K; d++) dot += row[d] * j->x[d];
            j->y[r] = j->acc ? j->y[r] + dot : dot;
        } else if (j->mode == 1) {
            double dot = 0.0;
            for (uint32_t d = 0; d < j->K; d++) dot += (double)row[d] * (double)j->x[d];
            j->yd[r] = dot;
        } else {
            double dot = 0.0;
            for (uint32_t d = 0; d < j->K; d++) dot += fabs((double)row[d] * (double)j->x[d]);
            j->yd[r] = dot;
        }
    }
    free(row);
    return NULL;
}

static int run_dmmv(const uint8_t *W, uint32_t type, const float *x, float *y, double *yd,
                    uint32_t M, uint32_t K, uint32_t acc, int nthreads, int mode) {
    if (zo_bytes_per_block(type) == 0 || K % zo_block_size(type) != 0) return -1;
    if (nthreads < 1) nthreads = 1;
    if ((uint32_t)nthreads > M) nthreads = M ? (int)M : 1;
    pthread_t th[256];
    dmmv_job jobs[256];
    if (nthreads > 256) nthreads = 256;
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = (dmmv_job){W, type, x, y, yd, M, K, acc,
                             (uint32_t)((uint64_t)M * t / nthreads),
                             (uint32_t)((uint64_t)M * (t + 1) / nthreads), mode};
    }
    if (nthreads == 1) { dmmv_worker(&jobs[0]); return 0; }
    for (int t = 0; t < nthreads; t++) pthread_create(&th[t], NULL, dmmv_worker, &jobs[t]);
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    return 0;
}

int zo_dmmv(const uint8_t *W, uint32_t type, const float *x, float *y,
            uint32_t M, uint32_t K, uint32_t acc_mode, int nthreads) {
    return run_dmmv(W, type, x, y, NULL, M, K, acc_mode, nthreads, 0);
}
int zo_dmmv_f64(const uint8_t *W, uint32_t type, const float *x, double *y,
                uint32_t M, uint32_t K, int nthreads) {
    return run_dmmv(W, type, x, NULL, y, M, K, 0, nthreads, 1);
}
int zo_dmmv_absdot(const uint8_t *W, uint32_t type, const float *x, double *y,
                   uint32_t M, uint32_t K, int nthreads) {
    return run_dmmv(W, type, x, NULL, y, M, K, 0, nthreads, 2);
}

/* ------------------------------------------------------------------ */
/* Elementwise restatements                                            */
/* ------------------------------------------------------------------ */
void zo_rms_norm_mul(const float *in, const float *w, uint32_t w_len, float *out,
                     uint32_t n, uint32_t n_groups, float eps) {
    for (uint32_t g = 0; g < n_groups; g++) {
        const float *x = in + (size_t)g * n;
        float sq = 0.f;
        for (uint32_t i = 0; i < n; i++) sq += x[i] * x[i];
        float rms_inv = 1.0f / sqrtf(sq / (float)n + eps);
        for (uint32_t i = 0; i < n; i++) out[(size_t)g * n + i] = w[i % w_len] * (x[i] * rms_inv);
    }
}

void zo_per_head_rms_norm(float *data, const float *w, uint32_t head_dim, uint32_t n_heads, float eps) {
    for (uint32_t h = 0; h < n_heads; h++) {
        float *x = data + (size_t)h * head_dim;
        float sq = 0.f;
        for (uint32_t i = 0; i < head_dim; i++) sq += x[i] * x[i];
        float rms_inv = 1.0f / sqrtf(sq / (float)head_dim + eps);
        for (uint32_t i = 0; i < head_dim; i++) x[i] = x[i] * rms_inv * w[i];
    }
}

void zo_rope_inv_freq(float *inv_freq, uint32_t rope_dim, float base) {
    for (uint32_t k = 0; k < rope_dim / 2; k++) {
        float exponent = (float)(2 * k) / (float)rope_dim;
        inv_freq[k] = 1.0f / powf(base, exponent);
    }
}

void zo_rope(float *data, uint32_t stride, uint32_t rope_dim, uint32_t n_heads,
             uint32_t position, const float *inv_freq) {
    uint32_t half = rope_dim / 2;
    for (uint32_t h = 0; h < n_heads; h++) {
        float *b = data + (size_t)h * stride;
        for (uint32_t i = 0; i < half; i++) {
            float theta = (float)position * inv_freq[i];
            float c = cosf(theta), s = sinf(theta);
            float x0 = b[i], x1 = b[i + half];
            b[i] = x0 * c - x1 * s;
            b[i + half] = x0 * s + x1 * c;
        }
    }
}

void zo_swiglu(const float *g, const float *u, float *out, uint32_t n) {
    for (uint32_t i = 0; i < n; i++) {
        float x = g[i];
        out[i] = (x / (1.0f + expf(-x))) * u[i];
    }
}

void zo_attention_f16(const float *q, const uint16_t *k, const uint16_t *v, float *out,
                      uint32_t head_dim, uint32_t n_heads, uint32_t n_kv_heads,
                      uint32_t seq_len, float attn_scale) {
    uint32_t gqa = n_heads / (n_kv_heads ? n_kv_heads : 1);
    uint32_t kv_dim = n_kv_heads * head_dim;
    float scale = attn_scale != 0.f ? attn_scale : 1.0f / sqrtf((float)head_dim);
    float *scores = (float *)malloc((size_t)seq_len * sizeof(float));
    for (uint32_t h = 0; h < n_heads; h++) {
        uint32_t kvh = h / gqa;
        const float *qh = q + (size_t)h * head_dim;
        float mx = -INFINITY;
        for (uint32_t t = 0; t < seq_len; t++) {
            const uint16_t *kv = k + (size_t)t * kv_dim + (size_t)kvh * head_dim;
            float dot = 0.f;
            for (uint32_t d = 0; d < head_dim; d++) dot += qh[d] * zo_f16_to_f32(kv[d]);
            scores[t] = dot * scale;
            if (scores[t] > mx) mx = scores[t];
        }
        float sum = 0.f;
        for (uint32_t t = 0; t < seq_len; t++) {
            scores[t] = expf(scores[t] - mx);
            sum += scores[t];
        }
        if (sum > 0.f)
            for (uint32_t t = 0; t < seq_len; t++) scores[t] /= sum;
        float *o = out + (size_t)h * head_dim;
        for (uint32_t d = 0; d < head_dim; d++) {
            float val = 0.f;
            for (uint32_t t = 0; t < seq_len; t++)
                val += scores[t] * zo_f16_to_f32(v[(size_t)t * kv_dim + (size_t)kvh * head_dim + d]);
            o[d] = val;
        }
    }
    free(scores);
}

void zo_topk_softmax(const float *logits, uint32_t n, uint32_t k, uint32_t *ids, float *w) {
    float mx = -INFINITY;
    for (uint32_t i = 0; i < n; i++) if (logits[i] > mx) mx = logits[i];
    float probs[256];
    float sum = 0.f;
    for (uint32_t i = 0; i < n; i++) { probs[i] = expf(logits[i] - mx); sum += probs[i]; }
    if (sum > 0.f) for (uint32_t i = 0; i < n; i++) probs[i] /= sum;
    unsigned char used[256] = {0};
    for (uint32_t ki = 0; ki < k; ki++) {
        uint32_t best = 0;
        float bv = -1.0f;
        for (uint32_t i = 0; i < n; i++)
            if (!used[i] && probs[i] > bv) { bv = probs[i]; best = i; }
        ids[ki] = best;
        w[ki] = bv;
        used[best] = 1;
    }
    float ws = 0.f;
    for (uint32_t i = 0; i < k; i++) ws += w[i];
    if (ws > 0.f) for (uint32_t i = 0; i < k; i++) w[i] /= ws;
}

uint32_t zo_argmax(const float *logits, uint32_t n) {
    float mv = logits[0];
    uint32_t mi = 0;
    for (uint32_t i = 1; i < n; i++) if (logits[i] > mv) { mv = logits[i]; mi = i; }
    return mi;
}

/* SamplingParams.requiresLogitsReadback (forward.zig:102-104). */
int zo_sampling_requires_readback(float temperature, float top_p, float repetition_penalty) {
    return temperature > 0.0001f || top_p < 0.9999f || repetition_penalty > 1.0001f;
}

/* adjustedLogit (forward.zig:10241-10245) with tokenSeen's linear scan
 * (:10229-10234); the models on this path have no final-logit softcap. */
static float adjusted_logit(float logit, uint32_t token, const uint32_t *hist, uint32_t nh, float pen) {
    if (pen <= 1.0001f) return logit;
    int seen = 0;
    for (uint32_t i = 0; i < nh && !seen; i++) seen = hist[i] == token;
    if (!seen) return logit;
    return logit >= 0 ? logit / pen : logit * pen;
}

/* argmaxFromLogits (forward.zig:10247-10259): first strict maximum, starting
 * from logits[0] (a NaN there is never replaced). */
static uint32_t argmax_adjusted(const float *logits, uint32_t n, const uint32_t *hist, uint32_t nh, float pen) {
    uint32_t best = 0;
    float bv = adjusted_logit(logits[0], 0, hist, nh, pen);
    for (uint32_t i = 1; i < n; i++) {
        float v = adjusted_logit(logits[i], i, hist, nh, pen);
        if (v > bv) { bv = v; best = i; }
    }
    return best;
}

/* sampleFromLogits (forward.zig:10261-10334) without a softcap. `u` is the
 * value the reference draws with random.float(f64) (consumed only when the
 * choice is random). Candidates: the top_k (1..128) finite adjusted logits,
 * kept by an insertion that places a value after equal ones (earlier token
 * first); weights exp(l/T - l0/T) in f64; top_p keeps the shortest prefix
 * whose cumulative share reaches top_p (at least two candidates once
 * reached past the first); then the first candidate whose cumulative weight
 * reaches u * kept_weight. */
uint32_t zo_sample_from_logits(const float *logits, uint32_t n, const uint32_t *hist, uint32_t nh,
                               float temperature, float top_p, float rep_pen, uint32_t top_k, double u) {
    if (n == 0) return 0;
    if (!zo_sampling_requires_readback(temperature, top_p, rep_pen)) return argmax_adjusted(logits, n, hist, nh, 1.0f);
    if (temperature <= 0.0001f) return argmax_adjusted(logits, n, hist, nh, rep_pen);
    enum { MAXC = 128 };
    uint32_t k = top_k < 1 ? 1 : top_k > MAXC ? MAXC : top_k;
    float tp = top_p < 0.f ? 0.f : top_p > 1.f ? 1.f : top_p;
    float temp = temperature > 0.0001f ? temperature : 0.0001f;
    uint32_t ids[MAXC];
    float lv[MAXC];
    uint32_t cnt = 0;
    for (uint32_t i = 0; i < n; i++) {
        if (!isfinite(logits[i])) continue;
        float v = adjusted_logit(logits[i], i, hist, nh, rep_pen);
        uint32_t at = cnt;
        while (at > 0 && v > lv[at - 1]) at--;
        if (at >= k) continue;
        if (cnt < k) cnt++;
        for (uint32_t j = cnt - 1; j > at; j--) { ids[j] = ids[j - 1]; lv[j] = lv[j - 1]; }
        ids[at] = i;
        lv[at] = v;
    }
    if (cnt == 0) return 0;
    if (cnt == 1) return ids[0];
    double w[MAXC], total = 0.0;
    const double m0 = (double)lv[0] / (double)temp;
    for (uint32_t i = 0; i < cnt; i++) {
        w[i] = exp((double)lv[i] / (double)temp - m0);
        total += w[i];
    }
    if (!(total > 0.0) || !isfinite(total)) return ids[0];
    uint32_t keep = cnt;
    if (tp < 0.9999f) {
        double cum = 0.0;
        for (uint32_t i = 0; i < cnt; i++) {
            cum += w[i] / total;
            keep = i + 1;
            if (cum >= (double)tp && i > 0) break;
        }
    }
    double kept = 0.0;
    for (uint32_t i = 0; i < keep; i++) kept += w[i];
    if (!(kept > 0.0) || !isfinite(kept)) return ids[0];
    const double target = u * kept;
    double cum = 0.0;
    for (uint32_t i = 0; i < keep; i++) {
        cum += w[i];
        if (target <= cum) return ids[i];
    }
    return ids[keep - 1];
}

uint32_t zo_kv_page_count(uint32_t ctx) { return ctx == 0 ? 0 : (ctx + 15) / 16; }
int64_t zo_logical_to_physical(const uint32_t *page_ids, uint32_t n_pages, uint32_t logical) {
    uint32_t slot = logical / 16;
    if (slot >= n_pages) return -1;
    return (int64_t)page_ids[slot] * 16 + (logical % 16);
}

/* ------------------------------------------------------------------ */
/* Seeded synthetic data. The HIP generator implements the same spec:  */
/*   r(seed, stream, ctr) = fmix64(key + (ctr + 1) * G),               */
/*   key = fmix64(seed ^ (stream * 0xD1B54A32D192ED03)),               */
/* with fmix64 the splitmix64 finaliser. normal(r) is Irwin-Hall(4) of */
/* the four 16-bit fields, standardised with one f32 multiply (bounded */
/* to +-3.46; every step is exact or a single correctly rounded op).   */
/* ------------------------------------------------------------------ */
static inline uint64_t fmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
uint64_t zo_rand(uint64_t seed, uint64_t stream, uint64_t ctr) {
    uint64_t key = fmix64(seed ^ (stream * 0xD1B54A32D192ED03ull));
    return fmix64(key + (ctr + 1) * 0x9E3779B97F4A7C15ull);
}
float zo_normal(uint64_t r) {
    int32_t s = (int32_t)(r & 0xFFFF) + (int32_t)((r >> 16) & 0xFFFF) +
                (int32_t)((r >> 32) & 0xFFFF) + (int32_t)((r >> 48) & 0xFFFF) - 131070;
    return (float)s * 2.6429573e-05f;
}
static inline uint16_t scale_f16(uint64_t r) { return zo_f32_to_f16(fabsf(zo_normal(r)) * 0.02f); }

/* the router weights' scale shift: 2^-e with 2^e nearest to 1.466 sqrt(K), 1.466 being the standard
 * deviation of the synthetic Q8_0 weights d * q (d = |N(0, .02)|, q uniform -127..127) */
uint32_t zo_router_shift(uint64_t K) {
    long e = lround(log2(1.466 * sqrt((double)K)));
    return e < 0 ? 0u : e > 15 ? 15u : (uint32_t)e;
}

int zo_synth_tensor(uint8_t *dst, uint32_t type_flags, uint64_t rows, uint64_t cols,
                    uint64_t seed, uint64_t stream) {
    /* type | 0x100: model-init variant of Q4_K / Q5_K with dmin = f16(7.5 * d) / f16(15.5 * d) (zero-mean
     * sub-blocks); the synthetic models use it for every Q4_K tensor. */
    /* type | 0x200 | e << 12: a router (Q8_0): d = f16(d * 2^-e), e = zo_router_shift(cols), so that the
     * router logits of an RMS-normed input are about N(0,1), not the O(sqrt(cols))
     * of the other projections, whose outputs the next RMSNorm rescales. */
    uint32_t type = type_flags & 0xFF;
    int centered = (type_flags & 0x100) != 0;
    uint64_t bs = zo_block_size(type), bpb = zo_bytes_per_block(type);
    if (bpb == 0 || cols % bs) return -1;
    uint64_t nb = rows * (cols / bs);
    for (uint64_t b = 0; b < nb; b++) {
        uint8_t *o = dst + b * bpb;
        switch (type) {
        case ZO_Q4_K: { /* d, dmin = f16(|N(0,.02)|); 12 scale bytes + 128 qs bytes uniform */
            uint16_t d = scale_f16(zo_rand(seed, stream, b * 32 + 0));
            uint16_t dm = centered ? zo_f32_to_f16(zo_f16_to_f32(d) * 7.5f) : scale_f16(zo_rand(seed, stream, b * 32 + 1));
            o[0] = d & 0xFF; o[1] = d >> 8; o[2] = dm & 0xFF; o[3] = dm >> 8;
            for (int i = 0; i < 140; i++) {
                uint64_t r = zo_rand(seed, stream, b * 32 + 2 + i / 8);
                o[4 + i] = (uint8_t)(r >> (8 * (i % 8)));
            }
            break;
        }
        case ZO_Q5_K: { /* as Q4_K (d, dmin, then 172 bytes: scales, qh, qs uniform);
                         * centered: dmin = f16(15.5 * d), the mean 5-bit quant */
            uint16_t d = scale_f16(zo_rand(seed, stream, b * 32 + 0));
            uint16_t dm = centered ? zo_f32_to_f16(zo_f16_to_f32(d) * 15.5f) : scale_f16(zo_rand(seed, stream, b * 32 + 1));
            o[0] = d & 0xFF; o[1] = d >> 8; o[2] = dm & 0xFF; o[3] = dm >> 8;
            for (int i = 0; i < 172; i++) {
                uint64_t r = zo_rand(seed, stream, b * 32 + 2 + i / 8);
                o[4 + i] = (uint8_t)(r >> (8 * (i % 8)));
            }
            break;
        }
        case ZO_Q6_K: { /* ql,qh uniform; int8 scales uniform -32..31; d = f16(|N(0,.02)|) */
            for (int i = 0; i < 192; i++) {
                uint64_t r = zo_rand(seed, stream, b * 32 + 1 + i / 8);
                o[i] = (uint8_t)(r >> (8 * (i % 8)));
            }
            for (int i = 0; i < 16; i++) {
                uint64_t r = zo_rand(seed, stream, b * 32 + 25 + i / 8);
                uint8_t byte = (uint8_t)(r >> (8 * (i % 8)));
                o[192 + i] = (uint8_t)(int8_t)((int)(byte & 63) - 32);
            }
            uint16_t d = scale_f16(zo_rand(seed, stream, b * 32 + 0));
            o[208] = d & 0xFF; o[209] = d >> 8;
            break;
        }
        case ZO_Q8_0: { /* f16 scale |N(0,.02)|; int8 uniform -127..127 */
            uint16_t d = scale_f16(zo_rand(seed, stream, b * 16 + 0));
            if (type_flags & 0x200) /* router: d * 2^-e (e in bits 12..15) */
                d = zo_f32_to_f16(ldexpf(zo_f16_to_f32(d), -(int)((type_flags >> 12) & 15)));
            o[0] = d & 0xFF; o[1] = d >> 8;
            for (int i = 0; i < 32; i++) {
                uint64_t r = zo_rand(seed, stream, b * 16 + 1 + i / 4);
                uint32_t u = (uint32_t)(r >> (16 * (i % 4))) & 0xFFFF;
                o[2 + i] = (uint8_t)(int8_t)((int)(u % 255u) - 127);
            }
            break;
        }
        case ZO_MXFP4: { /* e8m0 uniform 118..130; e2m1 code bytes uniform */
            uint64_t r0 = zo_rand(seed, stream, b * 4 + 0);
            o[0] = (uint8_t)(118 + (r0 % 13));
            for (int i = 0; i < 16; i++) {
                uint64_t r = zo_rand(seed, stream, b * 4 + 1 + i / 8);
                o[1 + i] = (uint8_t)(r >> (8 * (i % 8)));
            }
            break;
        }
        case ZO_F32: {
            float v = zo_normal(zo_rand(seed, stream, b));
            memcpy(o, &v, 4);
            break;
        }
        case ZO_F16: {
            uint16_t h = zo_f32_to_f16(zo_normal(zo_rand(seed, stream, b)));
            o[0] = h & 0xFF; o[1] = h >> 8;
            break;
        }
        default: return -1;
        }
    }
    return 0;
}

void zo_synth_normal_f32(float *dst, uint64_t n, float scale, uint64_t seed, uint64_t stream) {
    for (uint64_t i = 0; i < n; i++) dst[i] = zo_normal(zo_rand(seed, stream, i)) * scale;
}
void zo_synth_normal_f16(uint16_t *dst, uint64_t n, uint64_t seed, uint64_t stream) {
    for (uint64_t i = 0; i < n; i++) dst[i] = zo_f32_to_f16(zo_normal(zo_rand(seed, stream, i)));
}
void zo_synth_norm_weight(float *dst, uint64_t n, uint64_t seed, uint64_t stream) {
    /* 1 + U(-0.01, 0.01) with a 16-bit grid */
    for (uint64_t i = 0; i < n; i++) {
        int32_t s = (int32_t)(zo_rand(seed, stream, i) & 0xFFFF) - 32768;
        dst[i] = 1.0f + (float)s * 3.0517578e-07f;
    }
}

/* ------------------------------------------------------------------ */
/* Whole-model decode step                                             */
/* ------------------------------------------------------------------ */
/* Tensor stream ids (same numbering in the HIP engine). */
#define ZS_TOKEN_EMBD 1
#define ZS_OUTPUT_NORM 2
#define ZS_OUTPUT 3
#define ZS_LAYER(l, kind) ((((uint64_t)(l) + 1) << 8) | (kind))
enum { ZK_ATTN_NORM = 1, ZK_WQ, ZK_WK, ZK_WV, ZK_WO, ZK_Q_NORM, ZK_K_NORM, ZK_FFN_NORM,
       ZK_GATE, ZK_UP, ZK_DOWN, ZK_ROUTER, ZK_EXP_GATE, ZK_EXP_UP, ZK_EXP_DOWN };
#define ZS_KV(l, which) (0x100000ull + 2ull * (l) + (which))

typedef struct {
    uint32_t t[16]; /* storage type of each tensor kind (ZK_*) in this layer */
    uint8_t *wq, *wk, *wv, *wo, *gate, *up, *down, *router, *egate, *eup, *edown;
    float *attn_norm, *q_norm, *k_norm, *ffn_norm;
    uint16_t *kc, *vc; /* [max_ctx][kv_dim] fp16, logical == physical (identity pages) */
} zo_layer;

struct zo_model {
    zo_model_config c;
    int nthreads;
    uint32_t t_embd, t_lm; /* storage types of token_embd and output */
    uint8_t *embd, *lm;
    float *out_norm, *inv_freq;
    zo_layer *L;
    float *hidden, *norm, *q, *k, *v, *attn, *g, *u, *s, *logits, *rl, *eacc;
    /* test diagnostic, not part of the restated algorithm: over the MoE
     * layers of the last decode step, the smallest gap between the k-th
     * selected router logit and the best unselected one, as a fraction of
     * the layer's max |router logit| (a near tie that a sum in another order
     * can flip); layers whose selection includes a zero-probability expert
     * have no such tie */
    float route_gap;
    /* test diagnostic: per MoE layer of the last decode step, the selected
     * expert ids (n_experts_used each) and that layer's gap as above
     * (INFINITY when it has none) */
    uint32_t *sel_ids;
    float *sel_w, *sel_gap;
};

static uint8_t *alloc_tensor(uint32_t type, uint64_t rows, uint64_t cols, uint64_t seed, uint64_t stream) {
    uint8_t *p = (uint8_t *)malloc(zo_tensor_bytes(type, rows, cols));
    zo_synth_tensor(p, type | 0x100, rows, cols, seed, stream);
    return p;
}
static float *alloc_norm(uint64_t n, uint64_t seed, uint64_t stream) {
    float *p = (float *)malloc(n * 4);
    zo_synth_norm_weight(p, n, seed, stream);
    return p;
}

int zo_more_bits_layer(uint32_t i, uint32_t n) {
    return i < n / 8 || i >= 7 * n / 8 || (i - n / 8) % 3 == 2;
}

typedef struct { zo_model *m; uint32_t l0, l1; } build_job;
static void build_layer(zo_model *m, uint32_t l) {
    zo_model_config *c = &m->c;
    uint64_t s = c->seed;
    uint32_t H = c->hidden, qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim;
    zo_layer *y = &m->L[l];
    memset(y, 0, sizeof(*y));
    const int more = c->type_more_bits && zo_more_bits_layer(l, c->n_layers);
    y->t[ZK_WQ] = y->t[ZK_WK] = y->t[ZK_WO] = c->type_attn;
    y->t[ZK_WV] = more ? c->type_more_bits : c->type_attn;
    y->t[ZK_GATE] = y->t[ZK_UP] = y->t[ZK_EXP_GATE] = y->t[ZK_EXP_UP] = c->type_ffn_gate_up;
    y->t[ZK_DOWN] = y->t[ZK_EXP_DOWN] = more ? c->type_more_bits : c->type_ffn_down;
    y->t[ZK_ROUTER] = c->type_router;
    y->attn_norm = alloc_norm(H, s, ZS_LAYER(l, ZK_ATTN_NORM));
    y->wq = alloc_tensor(y->t[ZK_WQ], qd, H, s, ZS_LAYER(l, ZK_WQ));
    y->wk = alloc_tensor(y->t[ZK_WK], kvd, H, s, ZS_LAYER(l, ZK_WK));
    y->wv = alloc_tensor(y->t[ZK_WV], kvd, H, s, ZS_LAYER(l, ZK_WV));
    y->wo = alloc_tensor(y->t[ZK_WO], H, qd, s, ZS_LAYER(l, ZK_WO));
    y->q_norm = alloc_norm(c->head_dim, s, ZS_LAYER(l, ZK_Q_NORM));
    y->k_norm = alloc_norm(c->head_dim, s, ZS_LAYER(l, ZK_K_NORM));
    y->ffn_norm = alloc_norm(H, s, ZS_LAYER(l, ZK_FFN_NORM));
    if (c->n_experts == 0) {
        y->gate = alloc_tensor(y->t[ZK_GATE], c->ffn, H, s, ZS_LAYER(l, ZK_GATE));
        y->up = alloc_tensor(y->t[ZK_UP], c->ffn, H, s, ZS_LAYER(l, ZK_UP));
        y->down = alloc_tensor(y->t[ZK_DOWN], H, c->ffn, s, ZS_LAYER(l, ZK_DOWN));
    } else {
        y->router = (uint8_t *)malloc(zo_tensor_bytes(y->t[ZK_ROUTER], c->n_experts, H));
        zo_synth_tensor(y->router, y->t[ZK_ROUTER] | 0x100 | 0x200 | (zo_router_shift(H) << 12), c->n_experts, H, s,
                        ZS_LAYER(l, ZK_ROUTER));
        y->egate = alloc_tensor(y->t[ZK_EXP_GATE], (uint64_t)c->n_experts * c->expert_ffn, H, s, ZS_LAYER(l, ZK_EXP_GATE));
        y->eup = alloc_tensor(y->t[ZK_EXP_UP], (uint64_t)c->n_experts * c->expert_ffn, H, s, ZS_LAYER(l, ZK_EXP_UP));
        y->edown = alloc_tensor(y->t[ZK_EXP_DOWN], (uint64_t)c->n_experts * H, c->expert_ffn, s, ZS_LAYER(l, ZK_EXP_DOWN));
    }
    y->kc = (uint16_t *)calloc((size_t)c->max_ctx * kvd, 2);
    y->vc = (uint16_t *)calloc((size_t)c->max_ctx * kvd, 2);
}
static void *build_worker(void *a) {
    build_job *j = (build_job *)a;
    for (uint32_t l = j->l0; l < j->l1; l++) build_layer(j->m, l);
    return NULL;
}

zo_model *zo_model_create(const zo_model_config *cfg, int nthreads) {
    zo_model *m = (zo_model *)calloc(1, sizeof(zo_model));
    m->c = *cfg;
    m->nthreads = nthreads < 1 ? 1 : nthreads;
    zo_model_config *c = &m->c;
    uint32_t H = c->hidden;
    m->t_embd = c->type_embd;
    m->t_lm = c->type_lm_head;
    m->embd = alloc_tensor(c->type_embd, c->vocab, H, c->seed, ZS_TOKEN_EMBD);
    m->out_norm = alloc_norm(H, c->seed, ZS_OUTPUT_NORM);
    m->lm = alloc_tensor(c->type_lm_head, c->vocab, H, c->seed, ZS_OUTPUT);
    m->inv_freq = (float *)malloc(c->head_dim / 2 * 4);
    zo_rope_inv_freq(m->inv_freq, c->head_dim, c->rope_base);
    m->L = (zo_layer *)calloc(c->n_layers, sizeof(zo_layer));
    int nt = m->nthreads > (int)c->n_layers ? (int)c->n_layers : m->nthreads;
    pthread_t th[256];
    build_job jobs[256];
    if (nt > 256) nt = 256;
    for (int t = 0; t < nt; t++) {
        jobs[t] = (build_job){m, c->n_layers * t / nt, c->n_layers * (t + 1) / nt};
        pthread_create(&th[t], NULL, build_worker, &jobs[t]);
    }
    for (int t = 0; t < nt; t++) pthread_join(th[t], NULL);
    uint32_t qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim;
    uint32_t fmax = c->ffn > c->expert_ffn ? c->ffn : c->expert_ffn;
    m->hidden = (float *)calloc(H, 4);
    m->norm = (float *)calloc(H > qd ? H : qd, 4);
    m->q = (float *)calloc(qd, 4);
    m->k = (float *)calloc(kvd, 4);
    m->v = (float *)calloc(kvd, 4);
    m->attn = (float *)calloc(qd, 4);
    m->g = (float *)calloc(fmax, 4);
    m->u = (float *)calloc(fmax, 4);
    m->s = (float *)calloc(fmax, 4);
    m->logits = (float *)calloc(c->vocab, 4);
    m->rl = (float *)calloc(c->n_experts ? c->n_experts : 1, 4);
    m->eacc = (float *)calloc(H, 4);
    m->sel_ids = (uint32_t *)calloc((size_t)c->n_layers * 16 + 1, 4);
    m->sel_gap = (float *)calloc((size_t)c->n_layers + 1, 4);
    m->sel_w = (float *)calloc((size_t)c->n_layers * 16 + 1, 4);
    return m;
}

void zo_model_destroy(zo_model *m) {
    if (!m) return;
    for (uint32_t l = 0; l < m->c.n_layers; l++) {
        zo_layer *y = &m->L[l];
        free(y->wq); free(y->wk); free(y->wv); free(y->wo); free(y->gate); free(y->up);
        free(y->down); free(y->router); free(y->egate); free(y->eup); free(y->edown);
        free(y->attn_norm); free(y->q_norm); free(y->k_norm); free(y->ffn_norm);
        free(y->kc); free(y->vc);
    }
    free(m->L); free(m->embd); free(m->lm); free(m->out_norm); free(m->inv_freq);
    free(m->hidden); free(m->norm); free(m->q); free(m->k); free(m->v); free(m->attn);
    free(m->g); free(m->u); free(m->s); free(m->logits); free(m->rl); free(m->eacc); free(m->sel_ids); free(m->sel_w); free(m->sel_gap);
    free(m);
}

void zo_model_prefill_kv_random(zo_model *m, uint32_t n, uint64_t seed) {
    uint32_t kvd = m->c.n_kv_heads * m->c.head_dim;
    for (uint32_t l = 0; l < m->c.n_layers; l++) {
        zo_synth_normal_f16(m->L[l].kc, (uint64_t)n * kvd, seed, ZS_KV(l, 0));
        zo_synth_normal_f16(m->L[l].vc, (uint64_t)n * kvd, seed, ZS_KV(l, 1));
    }
}

/* The storage slot of a tensor: its data pointer, storage type (NULL for
 * the f32 norm weights) and shape. Returns 0 when the model has no such
 * tensor. */
static int tensor_slot(zo_model *m, uint64_t stream, uint8_t ***data, uint32_t **type, uint64_t *rows,
                       uint64_t *cols) {
    zo_model_config *c = &m->c;
    uint64_t H = c->hidden, qd = (uint64_t)c->n_heads * c->head_dim, kvd = (uint64_t)c->n_kv_heads * c->head_dim;
    uint64_t E = c->n_experts, F = c->expert_ffn;
    *type = NULL;
    if (stream == ZS_TOKEN_EMBD) { *data = &m->embd; *type = &m->t_embd; *rows = c->vocab; *cols = H; return 1; }
    if (stream == ZS_OUTPUT) { *data = &m->lm; *type = &m->t_lm; *rows = c->vocab; *cols = H; return 1; }
    if (stream == ZS_OUTPUT_NORM) { *data = (uint8_t **)&m->out_norm; *rows = 1; *cols = H; return 1; }
    uint64_t l = (stream >> 8) - 1, kind = stream & 0xFF;
    if (stream <= 0xFF || l >= c->n_layers || kind == 0 || kind > ZK_EXP_DOWN) return 0;
    zo_layer *y = &m->L[l];
    const int dense = E == 0;
    switch (kind) {
    case ZK_ATTN_NORM: *data = (uint8_t **)&y->attn_norm; *rows = 1; *cols = H; return 1;
    case ZK_FFN_NORM: *data = (uint8_t **)&y->ffn_norm; *rows = 1; *cols = H; return 1;
    case ZK_Q_NORM: *data = (uint8_t **)&y->q_norm; *rows = 1; *cols = c->head_dim; return 1;
    case ZK_K_NORM: *data = (uint8_t **)&y->k_norm; *rows = 1; *cols = c->head_dim; return 1;
    case ZK_WQ: *data = &y->wq; *rows = qd; *cols = H; break;
    case ZK_WK: *data = &y->wk; *rows = kvd; *cols = H; break;
    case ZK_WV: *data = &y->wv; *rows = kvd; *cols = H; break;
    case ZK_WO: *data = &y->wo; *rows = H; *cols = qd; break;
    case ZK_GATE: if (!dense) return 0; *data = &y->gate; *rows = c->ffn; *cols = H; break;
    case ZK_UP: if (!dense) return 0; *data = &y->up; *rows = c->ffn; *cols = H; break;
    case ZK_DOWN: if (!dense) return 0; *data = &y->down; *rows = H; *cols = c->ffn; break;
    case ZK_ROUTER: if (dense) return 0; *data = &y->router; *rows = E; *cols = H; break;
    case ZK_EXP_GATE: if (dense) return 0; *data = &y->egate; *rows = E * F; *cols = H; break;
    case ZK_EXP_UP: if (dense) return 0; *data = &y->eup; *rows = E * F; *cols = H; break;
    case ZK_EXP_DOWN: if (dense) return 0; *data = &y->edown; *rows = E * H; *cols = F; break;
    default: return 0;
    }
    *type = &y->t[kind];
    return 1;
}

const uint8_t *zo_model_tensor(zo_model *m, uint64_t stream, uint64_t *bytes) {
    uint8_t **d;
    uint32_t *t;
    uint64_t rows, cols;
    if (!tensor_slot(m, stream, &d, &t, &rows, &cols)) { *bytes = 0; return NULL; }
    *bytes = t ? zo_tensor_bytes(*t, rows, cols) : rows * cols * 4;
    return *d;
}

int zo_model_tensor_type(zo_model *m, uint64_t stream) {
    uint8_t **d;
    uint32_t *t;
    uint64_t rows, cols;
    if (!tensor_slot(m, stream, &d, &t, &rows, &cols)) return -1;
    return t ? (int)*t : 0;
}

int zo_model_set_tensor(zo_model *m, uint64_t stream, uint32_t type, const void *src, uint64_t n) {
    uint8_t **d;
    uint32_t *t;
    uint64_t rows, cols;
    if (!tensor_slot(m, stream, &d, &t, &rows, &cols)) return -1;
    if (!t && type != 0) return -2; /* norm weights stay f32 */
    const uint64_t want = t ? zo_tensor_bytes(type, rows, cols) : rows * cols * 4;
    if (want == 0 || n != want) return -3;
    uint8_t *p = (uint8_t *)malloc(n);
    if (!p) return -4;
    memcpy(p, src, n);
    free(*d);
    *d = p;
    if (t) *t = type;
    return 0;
}
const float *zo_model_hidden(zo_model *m) { return m->hidden; }
float zo_model_route_gap(const zo_model *m) { return m->route_gap; }
int zo_model_routing(const zo_model *m, uint32_t layer, uint32_t *ids, float *weights, float *gap) {
    if (!m->c.n_experts || layer >= m->c.n_layers) return -1;
    for (uint32_t j = 0; j < m->c.n_experts_used && j < 16; j++) {
        ids[j] = m->sel_ids[(size_t)layer * 16 + j];
        weights[j] = m->sel_w[(size_t)layer * 16 + j];
    }
    *gap = m->sel_gap[layer];
    return 0;
}
const uint16_t *zo_model_kv(zo_model *m, uint32_t layer, uint32_t which, uint32_t token) {
    if (layer >= m->c.n_layers || which > 1 || token >= m->c.max_ctx) return NULL;
    const zo_layer *y = &m->L[layer];
    return (which ? y->vc : y->kc) + (size_t)token * m->c.n_kv_heads * m->c.head_dim;
}

typedef struct { const float *q; const uint16_t *k, *v; float *out; uint32_t hd, nh, nkv, L, h0, h1; } attn_job;
static void *attn_worker(void *a) {
    attn_job *j = (attn_job *)a;
    /* Heads are independent in cpuAttention; run a head range as a sub-problem. */
    uint32_t gqa = j->nh / j->nkv;
    for (uint32_t h = j->h0; h < j->h1; h++) {
        uint32_t kvh = h / gqa;
        /* one-head call: q/out offset by h, k/v viewed with kv_dim stride via n_kv_heads */
        uint32_t kv_dim = j->nkv * j->hd;
        float *scores = (float *)malloc((size_t)j->L * 4);
        const float *qh = j->q + (size_t)h * j->hd;
        float scale = 1.0f / sqrtf((float)j->hd), mx = -INFINITY;
        for (uint32_t t = 0; t < j->L; t++) {
            const uint16_t *kv = j->k + (size_t)t * kv_dim + (size_t)kvh * j->hd;
            float dot = 0.f;
            for (uint32_t d = 0; d < j->hd; d++) dot += qh[d] * zo_f16_to_f32(kv[d]);
            scores[t] = dot * scale;
            if (scores[t] > mx) mx = scores[t];
        }
        float sum = 0.f;
        for (uint32_t t = 0; t < j->L; t++) { scores[t] = expf(scores[t] - mx); sum += scores[t]; }
        if (sum > 0.f) for (uint32_t t = 0; t < j->L; t++) scores[t] /= sum;
        float *o = j->out + (size_t)h * j->hd;
        for (uint32_t d = 0; d < j->hd; d++) {
            float val = 0.f;
            for (uint32_t t = 0; t < j->L; t++)
                val += scores[t] * zo_f16_to_f32(j->v[(size_t)t * kv_dim + (size_t)kvh * j->hd + d]);
            o[d] = val;
        }
        free(scores);
    }
    return NULL;
}

uint32_t zo_model_decode_step(zo_model *m, uint32_t token, uint32_t pos, float *logits_out) {
    zo_model_config *c = &m->c;
    uint32_t H = c->hidden, hd = c->head_dim, qd = c->n_heads * hd, kvd = c->n_kv_heads * hd;
    int nt = m->nthreads;
    if (pos >= c->max_ctx) return UINT32_MAX; /* ContextLengthExceeded, forward.zig:4300 */
    /* embedToken: forward.zig:4255-4290 (safe_id clamp) */
    uint32_t tid = token < c->vocab ? token : c->vocab - 1;
    zo_dequant_row(m->embd, tid, H, m->t_embd, m->hidden);
    m->route_gap = INFINITY;
    for (uint32_t l = 0; l < c->n_layers; l++) {
        zo_layer *y = &m->L[l];
        zo_rms_norm_mul(m->hidden, y->attn_norm, H, m->norm, H, 1, c->eps);
        zo_dmmv(y->wq, y->t[ZK_WQ], m->norm, m->q, qd, H, 0, nt);
        zo_dmmv(y->wk, y->t[ZK_WK], m->norm, m->k, kvd, H, 0, nt);
        zo_dmmv(y->wv, y->t[ZK_WV], m->norm, m->v, kvd, H, 0, nt);
        zo_per_head_rms_norm(m->q, y->q_norm, hd, c->n_heads, c->eps);
        zo_per_head_rms_norm(m->k, y->k_norm, hd, c->n_kv_heads, c->eps);
        zo_rope(m->q, hd, hd, c->n_heads, pos, m->inv_freq);
        zo_rope(m->k, hd, hd, c->n_kv_heads, pos, m->inv_freq);
        for (uint32_t i = 0; i < kvd; i++) {
            y->kc[(size_t)pos * kvd + i] = zo_f32_to_f16(m->k[i]);
            y->vc[(size_t)pos * kvd + i] = zo_f32_to_f16(m->v[i]);
        }
        {
            int ntt = nt > (int)c->n_heads ? (int)c->n_heads : nt;
            pthread_t th[256];
            attn_job jobs[256];
            if (ntt > 256) ntt = 256;
            for (int t = 0; t < ntt; t++) {
                jobs[t] = (attn_job){m->q, y->kc, y->vc, m->attn, hd, c->n_heads, c->n_kv_heads, pos + 1,
                                     c->n_heads * t / ntt, c->n_heads * (t + 1) / ntt};
                pthread_create(&th[t], NULL, attn_worker, &jobs[t]);
            }
            for (int t = 0; t < ntt; t++) pthread_join(th[t], NULL);
        }
        zo_dmmv(y->wo, y->t[ZK_WO], m->attn, m->hidden, H, qd, 1, nt);
        zo_rms_norm_mul(m->hidden, y->ffn_norm, H, m->norm, H, 1, c->eps);
        if (c->n_experts == 0) {
            zo_dmmv(y->gate, y->t[ZK_GATE], m->norm, m->g, c->ffn, H, 0, nt);
            zo_dmmv(y->up, y->t[ZK_UP], m->norm, m->u, c->ffn, H, 0, nt);
            zo_swiglu(m->g, m->u, m->s, c->ffn);
            zo_dmmv(y->down, y->t[ZK_DOWN], m->s, m->hidden, H, c->ffn, 1, nt);
        } else {
            /* MoE FFN: forward.zig:5958-6500 (router -> topKSoftmax -> experts -> weighted acc) */
            uint32_t ids[64];
            float w[64];
            uint32_t F = c->expert_ffn;
            zo_dmmv(y->router, y->t[ZK_ROUTER], m->norm, m->rl, c->n_experts, H, 0, nt);
            zo_topk_softmax(m->rl, c->n_experts, c->n_experts_used, ids, w);
            {
                /* selection is by softmax probability; when a selected expert
                 * has probability 0 (underflow), every expert with a positive
                 * probability is selected and no order between selected and
                 * unselected ones matters for the output */
                float kth = INFINITY, rest = -INFINITY, amax = 0.f;
                int zero = 0;
                for (uint32_t j = 0; j < c->n_experts_used; j++) {
                    kth = fminf(kth, m->rl[ids[j]]);
                    zero |= w[j] == 0.f;
                }
                for (uint32_t i = 0; i < c->n_experts; i++) {
                    int sel = 0;
                    for (uint32_t j = 0; j < c->n_experts_used; j++) sel |= ids[j] == i;
                    if (!sel) rest = fmaxf(rest, m->rl[i]);
                    amax = fmaxf(amax, fabsf(m->rl[i]));
                }
                const float lg = amax > 0.f && !zero ? (kth - rest) / amax : INFINITY;
                m->route_gap = fminf(m->route_gap, lg);
                m->sel_gap[l] = lg;
                for (uint32_t j = 0; j < c->n_experts_used && j < 16; j++) {
                    m->sel_ids[(size_t)l * 16 + j] = ids[j];
                    m->sel_w[(size_t)l * 16 + j] = w[j];
                }
            }
            uint64_t gstride = zo_tensor_bytes(y->t[ZK_EXP_GATE], F, H), ustride = zo_tensor_bytes(y->t[ZK_EXP_UP], F, H);
            uint64_t dstride = zo_tensor_bytes(y->t[ZK_EXP_DOWN], H, F);
            float *dout = (float *)malloc((size_t)c->n_experts_used * H * 4);
            for (uint32_t j = 0; j < c->n_experts_used; j++) {
                zo_dmmv(y->egate + ids[j] * gstride, y->t[ZK_EXP_GATE], m->norm, m->g, F, H, 0, nt);
                zo_dmmv(y->eup + ids[j] * ustride, y->t[ZK_EXP_UP], m->norm, m->u, F, H, 0, nt);
                zo_swiglu(m->g, m->u, m->s, F);
                zo_dmmv(y->edown + ids[j] * dstride, y->t[ZK_EXP_DOWN], m->s, dout + (size_t)j * H, H, F, 0, nt);
            }
            /* moe_weighted_acc.comp:23-33: sum_j w_j*b_j then a += sum */
            for (uint32_t i = 0; i < H; i++) {
                float sum = 0.f;
                for (uint32_t j = 0; j < c->n_experts_used; j++) sum += w[j] * dout[(size_t)j * H + i];
                m->hidden[i] += sum;
            }
            free(dout);
        }
    }
    zo_rms_norm_mul(m->hidden, m->out_norm, H, m->norm, H, 1, c->eps);
    zo_dmmv(m->lm, m->t_lm, m->norm, m->logits, c->vocab, H, 0, nt);
    if (logits_out) memcpy(logits_out, m->logits, (size_t)c->vocab * 4);
    return zo_argmax(m->logits, c->vocab);
}
