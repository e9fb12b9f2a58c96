/*
 * CPU oracle for the packed-batch EmbeddingGemma encoder forward.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker and the
 * timed CPU baseline. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it. The HIP product path never
 * links, loads or calls it.
 *
 * It restates, in plain C, the arithmetic of the reference CPU path as it is
 * compiled by the vendored Makefile (`cc -std=c11 -O2` on x86-64: SSE2 paths
 * in kernels.c, the scalar `roundf` path in quants.c). Every function cites
 * the reference file:line it follows; paths are relative to
 * vendor/embeddinggemma.c/src/ unless stated otherwise.
 *
 * Pinning status (what checks each function; see tests/):
 *   fp16 <-> fp32, Q8_0 quantize/dequantize, sum_squares, rms_norm,
 *   rms_norm_quantize, rms_norm_residual, qk_norm_rope, dot, attention,
 *   gelu_tanh, gelu_mul_quantize, l2_normalize, normalize_prefix,
 *   mean_pool_rms_l2, Q8_0 x Q8_0 GEMM:
 *       golden fixtures written by the compiled reference
 *       (tests/golden/), bit-for-bit; plus closed forms / brute force.
 *   or_layer_forward / or_forward: composition of the pinned functions in
 *       the order of engine.c:488-821, 1098-1135; pinned through a
 *       double-precision brute-force layer on tiny inputs (tolerance).
 *   Dense head (dense_2, dense_3 on the mean pool, then L2): the reference
 *       describes it (EXTRACTION.md:178-181) but never implements it; its
 *       composition is pinned by a float64 brute force on tiny models that
 *       rejects planted mistakes (L2 before the head, the middle activation
 *       not re-quantized, an activation between the layers, a transposed
 *       weight), including a scale case where normalising first changes
 *       the quantized input (tests/test_oracle_math.py).
 */
#ifndef EG_ORACLE_H
#define EG_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Model constants of the 300M profile (model.h:8-15). */
#define OR_N_EMBD 768
#define OR_N_FF 1152
#define OR_N_HEAD 3
#define OR_HEAD_DIM 256
#define OR_N_CTX 2048
#define OR_VOCAB 262144
#define OR_QK 32
#define OR_DENSE_FF 3072

/* GGUF Q8_0 block: little-endian fp16 scale, then 32 int8 (quants.h:13-19). */
typedef struct {
    uint16_t d;
    int8_t qs[32];
} or_block_q8_0;

uint16_t or_fp32_to_fp16(float f);
float or_fp16_to_fp32(uint16_t h);
void or_quantize_row_q8_0(const float *x, or_block_q8_0 *out, int32_t n);
void or_dequantize_row_q8_0_scaled(const or_block_q8_0 *row, int32_t n, float scale, float *out);

float or_sum_squares(const float *x, int32_t n);
float or_dot_f32(const float *a, const float *b, int32_t n);
void or_rms_norm(const float *x, const float *w, int32_t n, float eps, float *out);
void or_rms_norm_quantize_q8_0(const float *x, const float *w, int32_t n, float eps,
                               or_block_q8_0 *out);
void or_rms_norm_residual_inplace(float *residual, const float *x, const float *w, int32_t n,
                                  float eps);
void or_rope_cos_sin(int32_t pos, float base, float *cos_out, float *sin_out);
void or_qk_norm_rope_qk_inplace(float *q, float *k, const float *q_weight, const float *k_weight,
                                int32_t pos, float base, float eps);
void or_attention_range(const float *q, const float *k, const float *v, int32_t n_tokens,
                        int32_t window, int32_t query_begin, int32_t query_end, float *ctx,
                        float *scores);
float or_gelu_tanh(float x);
void or_gelu_mul_quantize_q8_0(const float *gate, const float *up, int32_t n, or_block_q8_0 *out);
void or_l2_normalize(float *x, int32_t n);
int or_normalize_prefix(float *embedding, int32_t dimensions);
void or_mean_pool_rms(float *x, int32_t n_tokens, const float *w, float eps, float *out);
void or_mean_pool_rms_l2(float *x, int32_t n_tokens, const float *w, float eps, float *out);

/* y[t*m + r] = sum_p float(dot_p) * d_w * d_x over the K/32 blocks, in block
 * order (gemma2.c:120-141). w: m rows of k/32 blocks; xq: n rows of k/32. */
void or_gemm_q8_0(const or_block_q8_0 *w, const or_block_q8_0 *xq, int32_t n, int32_t k,
                  int32_t m, float *y, int32_t threads);

typedef struct {
    const or_block_q8_0 *attn_q, *attn_k, *attn_v, *attn_output;
    const or_block_q8_0 *ffn_up, *ffn_gate, *ffn_down;
    const float *attn_norm, *attn_q_norm, *attn_k_norm;
    const float *post_attention_norm, *ffn_norm, *post_ffw_norm;
    float rope_base;
    int32_t window; /* 0 = full attention inside the segment */
} or_layer;

typedef struct {
    const or_block_q8_0 *token_embd; /* [OR_VOCAB][768/32] */
    const float *output_norm;
    const or_block_q8_0 *dense_2; /* optional [3072][768/32] (NULL = absent) */
    const or_block_q8_0 *dense_3; /* optional [768][3072/32] */
    int32_t n_layer;
    float eps;
    or_layer layers[64];
} or_model;

/* One encoder layer over a packed wave, in place on x [T][768]
 * (engine.c:1115-1127 body: build_qkv_batch, batch attention,
 * apply_attention_output, apply_ffn). */
void or_layer_forward(const or_layer *layer, float eps, float *x, const int32_t *positions,
                      const size_t *offsets, size_t batch, int32_t threads);

/* Embedding lookup (engine.c:288-295). */
void or_input_embeddings(const or_model *m, const int32_t *ids, int32_t n_tokens, float *x);

/* Whole packed-wave forward: ids [offsets[batch]], out [batch][768] L2-normalised
 * (engine.c:1098-1135), then the optional dense head + L2.
 * Returns 0 on success, -1 on invalid input. */
int or_forward(const or_model *m, const int32_t *ids, const size_t *offsets, size_t batch,
               float *out, int32_t threads);

/* Host libm expf / tanhf over n floats. */
void or_libm_eval(const float *x, size_t n, float *expf_out, float *tanhf_out);

#ifdef __cplusplus
}
#endif
#endif
