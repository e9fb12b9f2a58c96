/*
 * CPU oracle for the packed-batch EmbeddingGemma encoder forward.
 * TEST INFRASTRUCTURE ONLY: the parity checker and the timed CPU baseline.
 * See oracle.h for the pinning status of every function. Reference paths
 * are relative to vendor/embeddinggemma.c/src/.
 *
 * Build with -ffp-contract=off and without -ffast-math: every float
 * expression below is evaluated in the order written, each operation
 * rounded once, exactly as the x86-64 SSE2 build of the reference does.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- fp16 */

/* quants.c:13-37. Round-half-up on the dropped mantissa bits (not RNE);
 * values >= 2^16 with a nonzero mantissa become NaN, exactly as there. */
uint16_t or_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mant = x & 0x007FFFFFu;
    int32_t e = (int32_t)((x >> 23) & 0xFFu) - 127 + 15;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x00800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t h = sign | (mant >> shift);
        if ((mant >> (shift - 1u)) & 1u) h++;
        return (uint16_t)h;
    }
    if (e >= 31) {
        if (mant == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7C00u | (mant >> 13) | 1u);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13);
    if (mant & 0x00001000u) h++;
    return (uint16_t)h;
}

/* common.h:17-40: exact IEEE half -> float (subnormals, inf, nan). */
float or_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int sh = 0;
            uint32_t m = man;
            while (!(m & 0x400u)) {
                m <<= 1;
                sh++;
            }
            /* value = man * 2^-24 = 1.f * 2^(-14 - sh) */
            bits = sign | ((uint32_t)(127 - 14 - sh) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((e - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* ---------------------------------------------------------------- Q8_0 */

/* quants.c:97-177, scalar branch (:122-127, :128-133, :169-174):
 * amax = max|x|; d = amax/127 (fp32); stored d = fp16(d); amax == 0 -> zeros;
 * id = 1/d (fp32 d, not the stored half); q = roundf(x*id) clamped. */
void or_quantize_row_q8_0(const float *x, or_block_q8_0 *out, int32_t n) {
    int32_t nb = n / OR_QK;
    for (int32_t b = 0; b < nb; b++) {
        const float *xb = x + b * OR_QK;
        float amax = 0.0f;
        for (int j = 0; j < OR_QK; j++) {
            float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f;
        out[b].d = or_fp32_to_fp16(d);
        if (amax == 0.0f) {
            memset(out[b].qs, 0, sizeof out[b].qs);
            continue;
        }
        float id = 1.0f / d;
        for (int j = 0; j < OR_QK; j++) {
            int q = (int)roundf(xb[j] * id);
            if (q < -128) q = -128;
            if (q > 127) q = 127;
            out[b].qs[j] = (int8_t)q;
        }
    }
}

/* quants.c:55-91, scalar branch (:86-88): d = fp16(d) * scale; out = d * q. */
void or_dequantize_row_q8_0_scaled(const or_block_q8_0 *row, int32_t n, float scale,
                                   float *out) {
    for (int32_t b = 0; b < n / OR_QK; b++) {
        float d = or_fp16_to_fp32(row[b].d) * scale;
        for (int j = 0; j < OR_QK; j++) out[b * OR_QK + j] = d * (float)row[b].qs[j];
    }
}

/* ---------------------------------------------------------------- rows */

/* kernels.c:82-94 (SSE2): two 4-lane accumulators over 8-element strides,
 * then hsum ((v0+v2)+(v1+v3)) of their sum (kernels.c:35-39), then the tail. */
float or_sum_squares(const float *x, int32_t n) {
    float s0[4] = {0.0f, 0.0f, 0.0f, 0.0f}, s1[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int32_t i = 0;
    for (; i + 7 < n; i += 8) {
        for (int j = 0; j < 4; j++) {
            float p = x[i + j] * x[i + j];
            s0[j] = s0[j] + p;
        }
        for (int j = 0; j < 4; j++) {
            float p = x[i + 4 + j] * x[i + 4 + j];
            s1[j] = s1[j] + p;
        }
    }
    float v[4];
    for (int j = 0; j < 4; j++) v[j] = s0[j] + s1[j];
    float sum = (v[0] + v[2]) + (v[1] + v[3]);
    for (; i < n; i++) sum += x[i] * x[i];
    return sum;
}

/* kernels.c:289-295 (SSE2): one 4-lane accumulator, hsum, scalar tail. */
float or_dot_f32(const float *a, const float *b, int32_t n) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int32_t i = 0;
    for (; i + 3 < n; i += 4)
        for (int j = 0; j < 4; j++) {
            float p = a[i + j] * b[i + j];
            s[j] = s[j] + p;
        }
    float sum = (s[0] + s[2]) + (s[1] + s[3]);
    for (; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* kernels.c:124-133 (SSE2): (x*w)*scale over 8-wide chunks, x*scale*w tail. */
static void norm_scale(const float *x, const float *w, int32_t n, float scale, float *out) {
    int32_t i = 0;
    for (; i + 7 < n; i += 8)
        for (int j = 0; j < 8; j++) {
            float p = x[i + j] * w[i + j];
            out[i + j] = p * scale;
        }
    for (; i < n; i++) out[i] = x[i] * scale * w[i];
}

static float rms_inv(const float *x, int32_t n, float eps) {
    return 1.0f / sqrtf(or_sum_squares(x, n) / (float)n + eps);
}

/* kernels.c:153-156 */
void or_rms_norm(const float *x, const float *w, int32_t n, float eps, float *out) {
    norm_scale(x, w, n, rms_inv(x, n, eps), out);
}

/* kernels.c:139-151: one inverse RMS for the row, then per 32-block
 * normalise + quantize. */
void or_rms_norm_quantize_q8_0(const float *x, const float *w, int32_t n, float eps,
                               or_block_q8_0 *out) {
    float inv = rms_inv(x, n, eps);
    for (int32_t b = 0; b < n / OR_QK; b++) {
        float normalized[OR_QK];
        norm_scale(x + b * OR_QK, w + b * OR_QK, OR_QK, inv, normalized);
        or_quantize_row_q8_0(normalized, out + b, OR_QK);
    }
}

/* kernels.c:163-188; the SSE2 build takes the scalar branch (:186):
 * residual += (x*scale)*w. */
void or_rms_norm_residual_inplace(float *residual, const float *x, const float *w, int32_t n,
                                  float eps) {
    float scale = rms_inv(x, n, eps);
    for (int32_t i = 0; i < n; i++) residual[i] += x[i] * scale * w[i];
}

/* kernels.c:245-249: theta = pos * powf(base, -2*dim/256); glibc cosf/sinf. */
void or_rope_cos_sin(int32_t pos, float base, float *cos_out, float *sin_out) {
    for (int32_t dim = 0; dim < OR_HEAD_DIM / 2; dim++) {
        float theta = (float)pos * powf(base, -2.0f * (float)dim / (float)OR_HEAD_DIM);
        cos_out[dim] = cosf(theta);
        sin_out[dim] = sinf(theta);
    }
}

/* kernels.c:233-264: per-head RMS (weights applied before the inverse),
 * NeoX pairs (d, d+128), Q scaled by 0.0625 after rotation, K unscaled. */
void or_qk_norm_rope_qk_inplace(float *q, float *k, const float *q_weight, const float *k_weight,
                                int32_t pos, float base, float eps) {
    float q_inv[OR_N_HEAD];
    for (int32_t h = 0; h < OR_N_HEAD; h++)
        q_inv[h] = 1.0f / sqrtf(or_sum_squares(q + h * OR_HEAD_DIM, OR_HEAD_DIM) /
                                    (float)OR_HEAD_DIM + eps);
    float k_inv = 1.0f / sqrtf(or_sum_squares(k, OR_HEAD_DIM) / (float)OR_HEAD_DIM + eps);
    const int32_t half = OR_HEAD_DIM / 2;
    for (int32_t dim = 0; dim < half; dim++) {
        float theta = (float)pos * powf(base, -2.0f * (float)dim / (float)OR_HEAD_DIM);
        float c = cosf(theta);
        float s = sinf(theta);
        for (int32_t h = 0; h < OR_N_HEAD; h++) {
            float *r = q + h * OR_HEAD_DIM;
            float x0 = r[dim] * q_weight[dim] * q_inv[h];
            float x1 = r[dim + half] * q_weight[dim + half] * q_inv[h];
            r[dim] = (x0 * c - x1 * s) * 0.0625f;
            r[dim + half] = (x0 * s + x1 * c) * 0.0625f;
        }
        float x0 = k[dim] * k_weight[dim] * k_inv;
        float x1 = k[dim + half] * k_weight[dim + half] * k_inv;
        k[dim] = x0 * c - x1 * s;
        k[dim + half] = x0 * s + x1 * c;
    }
}

/* kernels.c:324-360. Q rows are [768] (3 heads), K/V rows [256] (one KV
 * head shared by all query heads). window > 0 limits keys to
 * |qt - kt| <= window/2 inside the sequence. ctx rows are zeroed first. */
void or_attention_range(const float *q, const float *k, const float *v, int32_t n_tokens,
                        int32_t window, int32_t query_begin, int32_t query_end, float *ctx,
                        float *scores) {
    memset(ctx + (size_t)query_begin * OR_N_EMBD, 0,
           sizeof(float) * (size_t)(query_end - query_begin) * OR_N_EMBD);
    const int32_t half_window = window > 0 ? window / 2 : 0;
    for (int32_t qt = query_begin; qt < query_end; qt++) {
        const int32_t first = window > 0 ? (qt - half_window > 0 ? qt - half_window : 0) : 0;
        const int32_t last = window > 0 ? (qt + half_window + 1 < n_tokens ? qt + half_window + 1
                                                                             : n_tokens)
                                        : n_tokens;
        for (int32_t h = 0; h < OR_N_HEAD; h++) {
            const float *qv = q + (size_t)qt * OR_N_EMBD + h * OR_HEAD_DIM;
            float max_score = -INFINITY;
            for (int32_t kt = first; kt < last; kt++) {
                float score = or_dot_f32(qv, k + (size_t)kt * OR_HEAD_DIM, OR_HEAD_DIM);
                scores[kt] = score;
                if (score > max_score) max_score = score;
            }
            float sum = 0.0f;
            for (int32_t kt = first; kt < last; kt++) {
                float p = expf(scores[kt] - max_score);
                scores[kt] = p;
                sum += p;
            }
            const float inv_sum = 1.0f / sum;
            float *out = ctx + (size_t)qt * OR_N_EMBD + h * OR_HEAD_DIM;
            for (int32_t kt = first; kt < last; kt++) {
                /* ei_axpy scalar branch (kernels.c:320): dst += scale*src. */
                const float scale = scores[kt] * inv_sum;
                const float *src = v + (size_t)kt * OR_HEAD_DIM;
                for (int32_t z = 0; z < OR_HEAD_DIM; z++) out[z] += scale * src[z];
            }
        }
    }
}

/* kernels.c:367-371 */
float or_gelu_tanh(float x) {
    const float a = 0.044715f;
    const float s = 0.79788456080286535587989211986876f;
    return 0.5f * x * (1.0f + tanhf(s * x * (1.0f + a * x * x)));
}

/* kernels.c:377-391 (and, identically, kernels.c:373-375 then quantize). */
void or_gelu_mul_quantize_q8_0(const float *gate, const float *up, int32_t n, or_block_q8_0 *out) {
    for (int32_t b = 0; b < n / OR_QK; b++) {
        float act[OR_QK];
        for (int32_t i = 0; i < OR_QK; i++)
            act[i] = or_gelu_tanh(gate[b * OR_QK + i]) * up[b * OR_QK + i];
        or_quantize_row_q8_0(act, out + b, OR_QK);
    }
}

/* kernels.c:393-396 with ei_vec_scale_inplace's scalar branch (:220). */
void or_l2_normalize(float *x, int32_t n) {
    const float ss = or_sum_squares(x, n);
    if (ss != 0.0f) {
        const float scale = 1.0f / sqrtf(ss);
        for (int32_t i = 0; i < n; i++) x[i] *= scale;
    }
}

/* kernels.c:398-407 */
int or_normalize_prefix(float *embedding, int32_t dimensions) {
    if (!(dimensions == 128 || dimensions == 256 || dimensions == 512 ||
          dimensions == OR_N_EMBD))
        return 0;
    if (dimensions < OR_N_EMBD) or_l2_normalize(embedding, dimensions);
    return 1;
}

/* kernels.c:417-425: per-token RMS (in place), token-ordered sum, times
 * 1/n -- the mean pool without the L2 of :426. */
void or_mean_pool_rms(float *x, int32_t n_tokens, const float *w, float eps, float *out) {
    memset(out, 0, sizeof(float) * OR_N_EMBD);
    for (int32_t t = 0; t < n_tokens; t++) {
        float *row = x + (size_t)t * OR_N_EMBD;
        or_rms_norm(row, w, OR_N_EMBD, eps, row);
        for (int32_t i = 0; i < OR_N_EMBD; i++) out[i] += 1.0f * row[i];
    }
    const float scale = 1.0f / (float)n_tokens;
    for (int32_t i = 0; i < OR_N_EMBD; i++) out[i] *= scale;
}

/* kernels.c:417-427: the mean pool above, then L2. */
void or_mean_pool_rms_l2(float *x, int32_t n_tokens, const float *w, float eps, float *out) {
    or_mean_pool_rms(x, n_tokens, w, eps, out);
    or_l2_normalize(out, OR_N_EMBD);
}

/* ---------------------------------------------------------------- threads */

typedef void (*or_task)(void *ctx, int32_t begin, int32_t end);
typedef struct {
    or_task fn;
    void *ctx;
    int32_t begin, end;
} or_job;

static void *or_run_job(void *p) {
    or_job *j = p;
    if (j->begin < j->end) j->fn(j->ctx, j->begin, j->end);
    return NULL;
}

/* Static split of [0,count) over `threads` workers. Every item is computed
 * independently, so the split never changes a result. */
static void or_parallel_for(int32_t count, int32_t threads, or_task fn, void *ctx) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if (threads == 1 || count < 2) {
        fn(ctx, 0, count);
        return;
    }
    if (threads > count) threads = count;
    pthread_t tid[256];
    or_job jobs[256];
    int started[256];
    for (int32_t i = 0; i < threads; i++) {
        jobs[i].fn = fn;
        jobs[i].ctx = ctx;
        jobs[i].begin = (int32_t)((int64_t)count * i / threads);
        jobs[i].end = (int32_t)((int64_t)count * (i + 1) / threads);
        started[i] = i > 0 && pthread_create(&tid[i], NULL, or_run_job, &jobs[i]) == 0;
    }
    or_run_job(&jobs[0]);
    for (int32_t i = 1; i < threads; i++) {
        if (started[i])
            pthread_join(tid[i], NULL);
        else
            or_run_job(&jobs[i]);
    }
}

/* ---------------------------------------------------------------- GEMM */

typedef struct {
    const or_block_q8_0 *w, *xq;
    int32_t n, k, m;
    float *y;
} gemm_ctx;

/* gemma2.c:120-141: per output, a sequential fp32 sum over K blocks of
 * ((float)int_dot * d_w) * d_x. */
static void gemm_rows(void *opaque, int32_t begin, int32_t end) {
    gemm_ctx *c = opaque;
    const int32_t nb = c->k / OR_QK;
    for (int32_t t = begin; t < end; t++) {
        const or_block_q8_0 *b = c->xq + (size_t)t * nb;
        float dx[256];
        for (int32_t p = 0; p < nb; p++) dx[p] = or_fp16_to_fp32(b[p].d);
        for (int32_t r = 0; r < c->m; r++) {
            const or_block_q8_0 *a = c->w + (size_t)r * nb;
            float sum = 0.0f;
            for (int32_t p = 0; p < nb; p++) {
                int32_t dot = 0;
                for (int z = 0; z < OR_QK; z++) dot += (int32_t)a[p].qs[z] * (int32_t)b[p].qs[z];
                float term = (float)dot * or_fp16_to_fp32(a[p].d);
                term = term * dx[p];
                sum = sum + term;
            }
            c->y[(size_t)t * c->m + r] = sum;
        }
    }
}

void or_gemm_q8_0(const or_block_q8_0 *w, const or_block_q8_0 *xq, int32_t n, int32_t k,
                  int32_t m, float *y, int32_t threads) {
    gemm_ctx c = {w, xq, n, k, m, y};
    or_parallel_for(n, threads, gemm_rows, &c);
}

/* ---------------------------------------------------------------- layer */

typedef struct {
    const float *in;
    const float *w;
    or_block_q8_0 *out;
    int32_t width;
    float eps;
} norm_quant_ctx;

static void norm_quant_rows(void *opaque, int32_t begin, int32_t end) {
    norm_quant_ctx *c = opaque;
    for (int32_t t = begin; t < end; t++)
        or_rms_norm_quantize_q8_0(c->in + (size_t)t * c->width, c->w, c->width, c->eps,
                                  c->out + (size_t)t * (c->width / OR_QK));
}

typedef struct {
    float *q, *k;
    const float *qw, *kw;
    const int32_t *positions;
    float base, eps;
} qk_ctx;

static void qk_rows(void *opaque, int32_t begin, int32_t end) {
    qk_ctx *c = opaque;
    for (int32_t t = begin; t < end; t++)
        or_qk_norm_rope_qk_inplace(c->q + (size_t)t * OR_N_EMBD, c->k + (size_t)t * OR_HEAD_DIM,
                                   c->qw, c->kw, c->positions[t], c->base, c->eps);
}

typedef struct {
    const float *q, *k, *v;
    float *ctx;
    const size_t *offsets;
    size_t batch;
    int32_t window;
} attn_ctx;

/* engine.c:850-873: split a token range at sequence boundaries. */
static void attn_rows(void *opaque, int32_t begin, int32_t end) {
    attn_ctx *c = opaque;
    float *scores = malloc(sizeof(float) * (OR_N_CTX > 65536 ? OR_N_CTX : 65536));
    size_t s = 0;
    while (s + 1 < c->batch && c->offsets[s + 1] <= (size_t)begin) s++;
    while (begin < end) {
        size_t start = c->offsets[s], stop = c->offsets[s + 1];
        int32_t seg_end = end < (int32_t)stop ? end : (int32_t)stop;
        or_attention_range(c->q + start * OR_N_EMBD, c->k + start * OR_HEAD_DIM,
                           c->v + start * OR_HEAD_DIM, (int32_t)(stop - start), c->window,
                           begin - (int32_t)start, seg_end - (int32_t)start,
                           c->ctx + start * OR_N_EMBD, scores);
        begin = seg_end;
        s++;
    }
    free(scores);
}

typedef struct {
    const float *in;
    or_block_q8_0 *out;
    int32_t width;
} quant_ctx;

static void quant_rows(void *opaque, int32_t begin, int32_t end) {
    quant_ctx *c = opaque;
    for (int32_t t = begin; t < end; t++)
        or_quantize_row_q8_0(c->in + (size_t)t * c->width, c->out + (size_t)t * (c->width / OR_QK),
                             c->width);
}

typedef struct {
    float *x;
    const float *h;
    const float *w;
    float eps;
} resid_ctx;

static void resid_rows(void *opaque, int32_t begin, int32_t end) {
    resid_ctx *c = opaque;
    for (int32_t t = begin; t < end; t++)
        or_rms_norm_residual_inplace(c->x + (size_t)t * OR_N_EMBD, c->h + (size_t)t * OR_N_EMBD,
                                     c->w, OR_N_EMBD, c->eps);
}

typedef struct {
    const float *gate, *up;
    or_block_q8_0 *out;
} gelu_ctx;

static void gelu_rows(void *opaque, int32_t begin, int32_t end) {
    gelu_ctx *c = opaque;
    for (int32_t t = begin; t < end; t++)
        or_gelu_mul_quantize_q8_0(c->gate + (size_t)t * OR_N_FF, c->up + (size_t)t * OR_N_FF,
                                  OR_N_FF, c->out + (size_t)t * (OR_N_FF / OR_QK));
}

/* The multirow packed layer of engine.c: build_qkv_multirow (:488-508),
 * batch_attention_rows (:850-873), apply_attention_output_multirow
 * (:640-656), apply_ffn_multirow (:746-779) with gelu-then-quantize
 * (:758-771). The per-token paths of engine.c compute the same values. */
void or_layer_forward(const or_layer *L, float eps, float *x, const int32_t *positions,
                      const size_t *offsets, size_t batch, int32_t threads) {
    const int32_t T = (int32_t)offsets[batch];
    or_block_q8_0 *xq = malloc(sizeof(or_block_q8_0) * (size_t)T * (OR_N_FF / OR_QK));
    float *q = malloc(sizeof(float) * (size_t)T * OR_N_EMBD);
    float *k = malloc(sizeof(float) * (size_t)T * OR_HEAD_DIM);
    float *v = malloc(sizeof(float) * (size_t)T * OR_HEAD_DIM);
    float *ctx = malloc(sizeof(float) * (size_t)T * OR_N_EMBD);
    float *h = malloc(sizeof(float) * (size_t)T * OR_N_EMBD);
    float *up = malloc(sizeof(float) * (size_t)T * OR_N_FF);
    float *gate = malloc(sizeof(float) * (size_t)T * OR_N_FF);

    norm_quant_ctx nq = {x, L->attn_norm, xq, OR_N_EMBD, eps};
    or_parallel_for(T, threads, norm_quant_rows, &nq);
    or_gemm_q8_0(L->attn_q, xq, T, OR_N_EMBD, OR_N_EMBD, q, threads);
    or_gemm_q8_0(L->attn_k, xq, T, OR_N_EMBD, OR_HEAD_DIM, k, threads);
    or_gemm_q8_0(L->attn_v, xq, T, OR_N_EMBD, OR_HEAD_DIM, v, threads);
    qk_ctx qk = {q, k, L->attn_q_norm, L->attn_k_norm, positions, L->rope_base, eps};
    or_parallel_for(T, threads, qk_rows, &qk);

    attn_ctx ac = {q, k, v, ctx, offsets, batch, L->window};
    or_parallel_for(T, threads, attn_rows, &ac);

    quant_ctx qc = {ctx, xq, OR_N_EMBD};
    or_parallel_for(T, threads, quant_rows, &qc);
    or_gemm_q8_0(L->attn_output, xq, T, OR_N_EMBD, OR_N_EMBD, h, threads);
    resid_ctx r1 = {x, h, L->post_attention_norm, eps};
    or_parallel_for(T, threads, resid_rows, &r1);

    norm_quant_ctx nf = {x, L->ffn_norm, xq, OR_N_EMBD, eps};
    or_parallel_for(T, threads, norm_quant_rows, &nf);
    or_gemm_q8_0(L->ffn_up, xq, T, OR_N_EMBD, OR_N_FF, up, threads);
    or_gemm_q8_0(L->ffn_gate, xq, T, OR_N_EMBD, OR_N_FF, gate, threads);
    gelu_ctx gc = {gate, up, xq};
    or_parallel_for(T, threads, gelu_rows, &gc);
    or_gemm_q8_0(L->ffn_down, xq, T, OR_N_FF, OR_N_EMBD, h, threads);
    resid_ctx r2 = {x, h, L->post_ffw_norm, eps};
    or_parallel_for(T, threads, resid_rows, &r2);

    free(gate);
    free(up);
    free(h);
    free(ctx);
    free(v);
    free(k);
    free(q);
    free(xq);
}

/* engine.c:288-295 */
void or_input_embeddings(const or_model *m, const int32_t *ids, int32_t n_tokens, float *x) {
    const float scale = sqrtf((float)OR_N_EMBD);
    for (int32_t t = 0; t < n_tokens; t++)
        or_dequantize_row_q8_0_scaled(m->token_embd + (size_t)ids[t] * (OR_N_EMBD / OR_QK),
                                      OR_N_EMBD, scale, x + (size_t)t * OR_N_EMBD);
}

/* engine.c:1021-1138 (validation :1024-1041, positions :1099-1104, layers
 * :1115-1127, pooling :1129-1135). The dense head has no reference
 * implementation; EXTRACTION.md:178-181 places it after the mean pool and
 * before normalisation: dense_2 then dense_3, no biases, no activation. It
 * is the pinned Q8_0 GEMM applied twice to the (un-normalised) mean, each
 * input Q8_0-quantized like every other projection input, then the L2 of
 * kernels.c:393-396. Without the head the pool is kernels.c:417-427 as is. */
int or_forward(const or_model *m, const int32_t *ids, const size_t *offsets, size_t batch,
               float *out, int32_t threads) {
    if (!ids || !offsets || !out || batch == 0 || offsets[0] != 0) return -1;
    for (size_t s = 0; s < batch; s++)
        if (offsets[s + 1] <= offsets[s]) return -1;
    const size_t total = offsets[batch];
    if (total > OR_N_CTX) return -1;
    for (size_t i = 0; i < total; i++)
        if (ids[i] < 0 || ids[i] >= OR_VOCAB) return -1;
    const int32_t T = (int32_t)total;
    int32_t *positions = malloc(sizeof(int32_t) * (size_t)T);
    float *x = malloc(sizeof(float) * (size_t)T * OR_N_EMBD);
    for (size_t s = 0; s < batch; s++)
        for (size_t t = offsets[s]; t < offsets[s + 1]; t++)
            positions[t] = (int32_t)(t - offsets[s]);
    or_input_embeddings(m, ids, T, x);
    for (int32_t il = 0; il < m->n_layer; il++)
        or_layer_forward(&m->layers[il], m->eps, x, positions, offsets, batch, threads);
    const int dense = m->dense_2 && m->dense_3;
    for (size_t s = 0; s < batch; s++) {
        float *xs = x + offsets[s] * OR_N_EMBD;
        const int32_t n = (int32_t)(offsets[s + 1] - offsets[s]);
        if (dense)
            or_mean_pool_rms(xs, n, m->output_norm, m->eps, out + s * OR_N_EMBD);
        else
            or_mean_pool_rms_l2(xs, n, m->output_norm, m->eps, out + s * OR_N_EMBD);
    }
    if (dense) {
        const int32_t B = (int32_t)batch;
        or_block_q8_0 *pq = malloc(sizeof(or_block_q8_0) * (size_t)B * (OR_DENSE_FF / OR_QK));
        float *mid = malloc(sizeof(float) * (size_t)B * OR_DENSE_FF);
        for (int32_t s = 0; s < B; s++)
            or_quantize_row_q8_0(out + (size_t)s * OR_N_EMBD, pq + (size_t)s * (OR_N_EMBD / OR_QK),
                                 OR_N_EMBD);
        or_gemm_q8_0(m->dense_2, pq, B, OR_N_EMBD, OR_DENSE_FF, mid, threads);
        for (int32_t s = 0; s < B; s++)
            or_quantize_row_q8_0(mid + (size_t)s * OR_DENSE_FF,
                                 pq + (size_t)s * (OR_DENSE_FF / OR_QK), OR_DENSE_FF);
        or_gemm_q8_0(m->dense_3, pq, B, OR_DENSE_FF, OR_N_EMBD, out, threads);
        for (int32_t s = 0; s < B; s++) or_l2_normalize(out + (size_t)s * OR_N_EMBD, OR_N_EMBD);
        free(mid);
        free(pq);
    }
    free(x);
    free(positions);
    return 0;
}

/* The host libm's expf and tanhf over an array (the functions the
 * reference calls at kernels.c:348 and :370), for comparing a device
 * restatement with them. */
void or_libm_eval(const float *x, size_t n, float *expf_out, float *tanhf_out) {
    for (size_t i = 0; i < n; i++) {
        expf_out[i] = expf(x[i]);
        tanhf_out[i] = tanhf(x[i]);
    }
}
