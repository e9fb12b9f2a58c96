/*
 * Operator-level C ABI of the gfx950 kernels behind the executor, plus the
 * host helpers the executor and its tests share.
 *
 * Device entry points take device pointers, unsigned sizes and a HIP stream
 * (hipStream_t passed as void*, NULL = the null stream). They enqueue work
 * and return 0 or a hipError_t code (eg2_hip_error_string names it); they
 * never synchronise. Q8_0 activations and weights use a split layout: the
 * int8 values in "row tiles" and one float per 32-block holding the value
 * of the block's fp16 scale, stored transposed as [k/32][ld] (the order
 * the projection GEMM reads them in). Row tiles are int8
 * [ceil(rows/32)][k/32][2][32][16]: value e of row r is at byte
 * ((((r / 32) * (k/32) + e / 32) * 2 + (e / 16) % 2) * 512 + (r % 32) * 16
 * + e % 16, so each 32 x 32 block is 1 KB in the register order of the int8
 * MFMA operand (eg2_q8_tile_bytes gives the size; eg2_q8_pack_rows and
 * eg2_q8_unpack_rows convert from and to row-major int8). The attention
 * operands are the fp32 rows [q0 q1 q2 | k | v] of the fused projection.
 *
 * Each entry names the reference function whose semantics it implements
 * (paths relative to vendor/embeddinggemma.c/src/ unless they start with
 * src/ or kernels/).
 */
#ifndef EG2_HIP_H
#define EG2_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#include "gguf.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ device ops */

/* engine.c:288-295 input_embeddings (x = fp16(d)*sqrt(768)*q from the raw
 * GGUF Q8_0 table) fused with kernels.c:139-151 ei_rms_norm_quantize_q8_0
 * (layer-0 attn_norm) into xq/xd. Replaces kernels/eg2.c:36-39 eg2_gather. */
int eg2_hip_embed_norm_quant(const void *table_q8, const int32_t *ids, unsigned rows, float embed_scale,
                             const float *norm_w, float eps, float *x, int8_t *xq, float *xd, void *stream);

/* kernels.c:163-188 ei_rms_norm_residual_inplace (x += rms(h)*post_w) then,
 * when next_w != NULL, kernels.c:139-151 on the updated x. Replaces
 * kernels/eg2.c:192-202 eg2_norm_residual + the following eg2_norm. */
int eg2_hip_residual_norm_quant(float *x, const float *h, const float *post_w, const float *next_w, float eps,
                                int8_t *xq, float *xd, unsigned rows, void *stream);

/* kernels.c:233-264 ei_qk_norm_rope_qk_inplace on rows of the fused
 * projection [q0 q1 q2 | k | v] (1280 fp32 per token): each q head and k
 * normalised and rotated with rope_table[pos[t]] ([0..127] = cos, [128..255]
 * = sin; eg2_rope_table), q scaled by 0.0625 after rotation, v unchanged;
 * the results, bit-identical to the reference, in the same layout in out,
 * which may be qkv itself. Replaces kernels/eg2.c:204-217 eg2_norm_rope. */
int eg2_hip_qk_norm_rope(const float *qkv, const float *q_w, const float *k_w, const float *rope_table,
                         const int32_t *pos, float eps, float *out, unsigned rows, void *stream);

/* kernels.c:324-360 ei_attention_mha_range over packed sequences
 * (engine.c:850-873), bit-identical to the reference: each token attends to
 * the keys of its own sequence, limited to |t - s| <= window/2 when window >
 * 0; 3 query heads share one KV head, head_dim 256; scores in the
 * reference's dot order (the SSE2 ei_dot_f32), expf as the host libm
 * computes it, the sequential sum and context accumulation in key order
 * (products on fp32 MFMA, each rounded once as a multiply); the context
 * row is then quantized to Q8_0 (quants.c:97-177) into cq (row tiles, k =
 * 768) and cd [24][rows]. qkv: rows of [q0 q1 q2 | k | v] as
 * eg2_hip_qk_norm_rope leaves them. items / tok: the plan of
 * eg2_attention_plan on the device; item_count: 2 uint32 on the device,
 * the score items (first in `items`) and the context items after them;
 * `grid` workgroups stride over each list; tok holds one record for each
 * of the `rows` rows, so every row must belong to a planned sequence, e.g.
 * a padding one. scores: scratch of at least the plan's score floats
 * (counts[1]). rows % 4 == 0. longest: the longest sequence of the
 * packing, a hint (at most rows) that picks one of four equivalent
 * softmax kernel forms (<= 128, <= 256, <= 512, and any length for a
 * longer or unknown (0) longest); a wrong hint costs time, never bits. A sequence's result does not depend on its place
 * in the wave. Replaces kernels/eg2.c:145-170 eg2_attention256. */
int eg2_hip_attention(const float *qkv, const uint32_t *items, const uint32_t *item_count, unsigned grid,
                      const uint32_t *tok, unsigned window, unsigned rows, unsigned longest, float *scores, int8_t *cq,
                      float *cd, void *stream);

/* eg2_hip_attention's three stages, launched one at a time (same
 * arguments and checks; run in this order they are eg2_hip_attention):
 * the scores of every planned (token, head, key) into `scores`; the
 * softmax of each score row in place (p values) with 1/sum at the head of
 * `scores`; the context,
 * quantized to Q8_0 into cq / cd. For per-kernel timing (the reference
 * times each dispatch, src/gemma2_kfd.cpp:173-186). Replace, together,
 * kernels/eg2.c:145-170 eg2_attention256. */
int eg2_hip_attention_scores(const float *qkv, const uint32_t *items, const uint32_t *item_count, unsigned grid,
                             unsigned window, unsigned rows, float *scores, void *stream);
int eg2_hip_attention_softmax(const uint32_t *tok, unsigned window, unsigned rows, unsigned longest, float *scores,
                              void *stream);
int eg2_hip_attention_context(const float *qkv, const uint32_t *items, const uint32_t *item_count, unsigned grid,
                              unsigned window, unsigned rows, const float *scores, int8_t *cq, float *cd,
                              void *stream);

/* eg2_hip_attention without allocation. It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops and harnesses that forbid
 * hipMalloc). The work plan is built on the device from the device
 * sequence bounds offsets[0..batch] (uint32; offsets[0] is read as 0 and
 * offsets[batch] as rows, every row must belong to a sequence, e.g. a
 * padding one), and the plan and scores live in a static array of this
 * library, one per GPU, of 48.6 MiB, held until the process ends. The
 * call allocates nothing; it rejects (hipErrorInvalidValue, nothing
 * launched) rows above EG2_ATTENTION_STATIC_ROWS, batch above
 * EG2_ATTENTION_STATIC_BATCH or rows % 4 != 0. The stream must belong to
 * the current device. Calls overlapping on one GPU share its array and
 * race; calls in one stream are ordered. Results are bit-identical to
 * eg2_hip_attention's. */
#define EG2_ATTENTION_STATIC_ROWS 2048u
#define EG2_ATTENTION_STATIC_BATCH 2048u
int eg2_hip_attention_static(const float *qkv, const uint32_t *offsets, unsigned batch, unsigned window,
                             unsigned rows, int8_t *cq, float *cd, void *stream);

/* Host: the plan of eg2_hip_attention for the sequences [offsets[s],
 * offsets[s+1]) (rows = offsets[batch]): the score items of every
 * sequence (per sequence of n tokens, ceil(n/32) key blocks x ceil(3n/32)
 * pair blocks), then its context items (ceil(3n/32) pair blocks; their
 * sixth word is 1 when the context kernel should take its units in
 * per-XCD contiguous eighths, which the plan decides from the packing's
 * balance, else 0), 8 uint32 each as eg2_hip_attention reads them, and
 * one token record per
 * token (4 uint32: sequence start, end, first score index, 0) at tok[4 t].
 * counts[0] = items of both kinds, counts[1] = score floats (ceil4(3 rows)
 * for the 1/sum values, then 3 n ceil4(n) per sequence), counts[2] = score
 * items. Writes the lists and returns 0 when they fit items_cap items and
 * scores_cap score floats; otherwise writes nothing and returns -1 (counts
 * still report the need). */
int eg2_attention_plan(const size_t *offsets, size_t batch, size_t items_cap, size_t scores_cap, uint32_t *items,
                       uint32_t *tok, size_t *counts);

/* Host: counts[0..1] = the most items and score floats eg2_attention_plan
 * can need for any packing of `tokens` tokens into at most `batch`
 * sequences (the sizes the executor allocates for a 2048-token wave plus
 * its padding sequence). */
void eg2_attention_capacity(size_t tokens, size_t batch, size_t *counts);

/* The host libm functions the reference path calls (glibc's expf for the
 * softmax, kernels.c:348, and tanhf for the GELU, kernels.c:370) as this
 * library restates them on the device: expf_out[i] = expf(x[i]),
 * tanhf_out[i] = tanhf(x[i]) for n floats, bit-identical to the host's for
 * every input. For tests that compare the two. */
int eg2_hip_libm_eval(const float *x, unsigned n, float *expf_out, float *tanhf_out, void *stream);

/* The GeGLU kernels evaluate the exact tanhf only where a Q8_0 result depends
 * on it, and an approximation (hardware exp2 and reciprocal) with a proven
 * error bound elsewhere. This sweeps every finite float x on the device and
 * leaves in *out (a device uint32 that must start at 0) the bits of
 * max |approximation(x) - tanhf(x)|, which the kernels assume is at most
 * 2^-21. For the test that asserts it. */
int eg2_hip_tanh_approx_error(uint32_t *out, void *stream);

/* kernels.c:367-391 ei_gelu_mul_quantize_q8_0 on rows [gate 1152 | up 1152].
 * Replaces kernels/eg2.c:173-179 eg2_element mode 1. */
int eg2_hip_gelu_quant(const float *gate_up, int8_t *gq, float *gd, unsigned rows, void *stream);

/* quants.c:97-177 ei_quantize_row_q8_0 on rows of width k (k % 64 == 0). */
int eg2_hip_quantize_rows(const float *x, unsigned k, int8_t *q, float *d, unsigned rows, void *stream);

/* kernels.c:158-161 ei_rms_norm_inplace on rows of width 768. */
int eg2_hip_rms_norm_rows(float *x, const float *w, float eps, unsigned rows, void *stream);

/* kernels.c:417-427 ei_mean_pool_rms_l2 after the per-token RMS
 * (eg2_hip_rms_norm_rows): mean over [offsets[s], offsets[s+1]) then L2.
 * Replaces kernels/eg2.c:181-188 eg2_pool + the host L2 of
 * src/gemma2_kfd.cpp:337-343. */
int eg2_hip_pool_l2(const float *x, const uint32_t *offsets, float *out, unsigned batch, void *stream);

/* The mean of eg2_hip_pool_l2 alone (out = [batch][768], the same
 * token-order sums), spread over 12 workgroups per sequence so that a long
 * sequence is read by 12 CUs; eg2_hip_l2_prefix(out, 768, 768, batch) then
 * completes eg2_hip_pool_l2 bit for bit. The executor takes this form for
 * waves holding a sequence longer than 256 tokens. batch <= 65535. */
int eg2_hip_pool_mean(const float *x, const uint32_t *offsets, float *out, unsigned batch, void *stream);

/* kernels.c:393-407 ei_l2_normalize / ei_embedding_normalize_prefix on the
 * first `dims` entries of rows of width `width` (dims % 8 == 0). */
int eg2_hip_l2_prefix(float *x, unsigned width, unsigned dims, unsigned rows, void *stream);

/* y[n][m] (row stride ldy) = Q8_0 activations [n][k] . Q8_0 weights [m][k]^T
 * with the reference's arithmetic (gemma2.c:120-141): exact integer block
 * dots on int8 MFMA, each scaled ((float)dot * d_w) * d_x and summed in
 * block order in fp32 -- bit-identical to the CPU path. xq/wq are row
 * tiles; xd holds the activation block scales [k/32][ldx] (ldx >= n), wd
 * the weight block scales [k/32][ldw] (ldw >= m; eg2_q8_weight_tiles writes
 * both weight arrays). Replaces kernels/eg2.c:41-119 eg2_mm*. k % 32 == 0;
 * n, m, k and the strides at most 2^24, and each scale array ((k/32) rows
 * of ldx or ldw floats) below 4 GiB (the same for the two fused forms). */
int eg2_hip_gemm_q8(const int8_t *xq, const float *xd, unsigned ldx, const int8_t *wq, const float *wd, unsigned ldw,
                    float *y, unsigned n, unsigned m, unsigned k, unsigned ldy, void *stream);

/* The fused Q|K|V projection with its QK-norm / RoPE in one kernel: for
 * n rows of Q8_0 activations xq/xd [n][k] and the [q 768 | k 256 | v 256]
 * weights (eg2_q8_weight_tiles of the concatenated matrices, ldw >= 1280),
 * the projection exactly as eg2_hip_gemm_q8 computes it, then exactly what
 * eg2_hip_qk_norm_rope does with it (same q_w, k_w, rope_table, pos, eps),
 * into out [n][1280] -- bit-identical to the two calls, without the
 * unnormalised projection in memory. Replaces the Q/K/V eg2_mm* calls and
 * eg2_norm_rope of kernels/eg2.c (:41-119, :204-217). k % 32 == 0. */
int eg2_hip_gemm_q8_qkv_rope(const int8_t *xq, const float *xd, unsigned ldx, const int8_t *wq, const float *wd,
                             unsigned ldw, unsigned n, unsigned k, const float *q_w, const float *k_w,
                             const float *rope_table, const int32_t *pos, float eps, float *out, void *stream);

/* The gate and up projections and the GeGLU with its Q8_0 quantization in
 * one kernel: for rows of Q8_0 activations xq/xd [n][k] and the gate and up
 * weights interleaved in 32-row groups (eg2_q8_geglu_weight_tiles: ldw >=
 * 2 ff), computes gate and up exactly as eg2_hip_gemm_q8 does, then
 * gelu_tanh(gate) * up (kernels.c:367-371) and its Q8_0 blocks
 * (quants.c:97-177) into gq (row tiles, ff / 32 blocks per row) and gd
 * [ff/32][ldg] (ldg >= n) -- bit-identical to eg2_hip_gemm_q8 on
 * [gate | up] followed by eg2_hip_gelu_quant. Replaces the gate and up
 * eg2_mm* calls and eg2_element mode 1 of kernels/eg2.c (:41-119,
 * :173-179). ff % 32 == 0, k % 32 == 0; sizes and strides at most 2^24. */
int eg2_hip_gemm_q8_geglu(const int8_t *xq, const float *xd, unsigned ldx, const int8_t *wq, const float *wd,
                          unsigned ldw, int8_t *gq, float *gd, unsigned ldg, unsigned n, unsigned ff, unsigned k,
                          void *stream);

/* ------------------------------------------------------------ executor phases
 * A context has several lanes (EG2_HIP_LANES, 1..8, 4 by default): each
 * lane is a stream on a hardware queue of its own (the stream carries a
 * CU mask of every CU, which the HIP runtime serves from a dedicated queue
 * whatever GPU_MAX_HW_QUEUES says) with its own 2048-token workspace, pinned staging and
 * hipGraphs, over the context's one copy of the weights, so waves on
 * different lanes run on the device at the same time. ei_gemma2_kfd_batch
 * (gemma2_kfd.h) takes any free lane and runs stage + launch(1) + collect
 * on it; concurrent calls use separate lanes. The phases below have no
 * counterpart in the reference; they let a benchmark time the
 * device-resident forward apart from the host transfers, and a caller keep
 * several waves in flight. Same validation, poisoning (a device failure on
 * any lane fails the whole context) and "HIP: ..." error contract as the
 * batch call; each call holds its lane for its duration. */

/* Number of lanes of ctx (0 for NULL). */
unsigned eg2_kfd_lanes(void *ctx);
/* Takes a lane from the context's pool of free lanes (blocking until one is
 * free; ei_gemma2_kfd_batch uses the same pool) and returns its index (-1
 * for NULL); eg2_kfd_release_lane returns it. A caller that keeps waves in
 * flight on several lanes holds them this way, so that no concurrent batch
 * call stages over its pending waves. */
int eg2_kfd_acquire_lane(void *ctx);
/* Takes a free lane from the pool without waiting: its index, or -1 when
 * every lane is taken (or ctx is NULL). A caller that already holds a lane
 * takes more this way, never by eg2_kfd_acquire_lane: two callers that
 * each hold lanes and wait for more would wait for each other forever. */
int eg2_kfd_try_acquire_lane(void *ctx);
void eg2_kfd_release_lane(void *ctx, unsigned lane);
/* Validates one wave, waits until the lane's previous wave is done with its
 * staging buffers, uploads the ids and packing metadata, and builds (once
 * per lane and padded wave size) its hipGraph. */
bool eg2_kfd_stage_lane(void *ctx, unsigned lane, const int32_t *ids, const size_t *offsets, size_t batch, char *err,
                        size_t len);
/* Enqueues the staged wave's forward `repeats` times (no host copies, no wait). */
bool eg2_kfd_launch_lane(void *ctx, unsigned lane, unsigned repeats, char *err, size_t len);
/* Waits for the lane's wave and copies its [batch][768] embeddings to out. */
bool eg2_kfd_collect_lane(void *ctx, unsigned lane, float *out, char *err, size_t len);
/* No counterpart in the reference; for a caller holding several lanes (the
 * stream driver) that collects whichever wave finishes first: 1 when the
 * lane's enqueued work is done (eg2_kfd_collect_lane then returns without
 * waiting), 0 while it runs, -1 on an error (message in err; collect
 * reports it too). Never waits. */
int eg2_kfd_lane_ready(void *ctx, unsigned lane, char *err, size_t len);
/* The same on lane 0, which eg2_kfd_stage takes from the pool (waiting
 * while a batch call holds it) and keeps until eg2_kfd_collect hands it
 * back; launch and collect without a staged wave fail. */
bool eg2_kfd_stage(void *ctx, const int32_t *ids, const size_t *offsets, size_t batch, char *err, size_t len);
bool eg2_kfd_launch_staged(void *ctx, unsigned repeats, char *err, size_t len);
bool eg2_kfd_collect(void *ctx, float *out, char *err, size_t len);

/* Test hook with no reference counterpart: the context's next device wait
 * (every batch, stage and collect waits on its lane's stream) reports a
 * failure exactly as a failing HIP call does -- the call returns false with
 * "HIP: ... injected HIP failure" and the context is poisoned, so every
 * later call fails with "restart process" (src/gemma2_kfd.cpp:190-191,
 * 214-215, 270). Raised on the host: no device fault is involved. */
void eg2_kfd_inject_failure(void *ctx);

/* The model checks of ei_gemma2_kfd_create alone, on the host with no
 * device call: the gemma-embedding architecture and hyper-parameters
 * (model.c:61-77), and every tensor the executor reads with its type, its
 * [ne0, ne1, 1, 1] shape and exactly the byte count that shape takes
 * (model.c:79-105, Q8_0 matrices; optional dense_2 / dense_3). create runs
 * the same checks before its first device call. Returns false and
 * "HIP: <what>" in err for a model it would reject. */
bool eg2_kfd_validate_gguf(const ei_gguf *g, char *err, size_t len);

/* ------------------------------------------------------------ host helpers */

/* Name of a code returned by the device ops. */
const char *eg2_hip_error_string(int code);

/* 0 when the current HIP device is a gfx950; otherwise -1 and a reason. */
int eg2_hip_device_check(char *err, size_t len);

/* Bytes of a row-tile buffer for `rows` rows of k values (rows rounded up
 * to 32). */
size_t eg2_q8_tile_bytes(size_t rows, unsigned k);

/* Row-major int8 q[rows][k] -> row tiles (padding rows zero), and back. */
void eg2_q8_pack_rows(const int8_t *q, size_t rows, unsigned k, int8_t *tiles);
void eg2_q8_unpack_rows(const int8_t *tiles, size_t rows, unsigned k, int8_t *q);

/* GGUF Q8_0 rows [rows][k] (34-byte blocks) -> the projection GEMM's weight
 * operands: wq, the int8 values as row tiles (eg2_q8_tile_bytes(rows, k)
 * bytes; padding rows zero), and wd [k/32][ldw], ldw = rows rounded up to
 * 32, the exact float value of each block's fp16 scale (common.h:17-40). */
void eg2_q8_weight_tiles(const void *blocks, size_t rows, unsigned k, int8_t *wq, float *wd);

/* GGUF Q8_0 gate and up matrices [ff][k] -> the weight operands of
 * eg2_hip_gemm_q8_geglu: rows interleaved in 32-row groups (gate rows
 * 32j..32j+31, then up rows 32j..32j+31, for j = 0 .. ff/32 - 1), then
 * laid out as eg2_q8_weight_tiles does (2 ff rows, ldw = 2 ff). Returns 0,
 * or -1 when ff % 32 != 0 or k % 32 != 0 (nothing written). */
int eg2_q8_geglu_weight_tiles(const void *gate, const void *up, size_t ff, unsigned k, int8_t *wq, float *wd);

/* RoPE table for positions 0..n_pos-1: row p = [cos(theta_0..127) |
 * sin(theta_0..127)], theta_i = p * powf(base, -2i/256), computed with the
 * host libm exactly as kernels.c:245-249 does per call. */
void eg2_rope_table(float base, unsigned n_pos, float *table);

/* ------------------------------------------------------------ GGUF files */

/* Parses a GGUF v3 file into the engine's ei_gguf layout (gguf.c:119-196:
 * same KV normalisation, alignment rules and tensor validation). The file is
 * mapped read-only. Returns 0, or -1 with a reason in err. */
int eg2_gguf_open(const char *path, ei_gguf *g, char *err, size_t len);
void eg2_gguf_close(ei_gguf *g);

/* Synthetic `gemma-embedding` model with the 300M tensor names and shapes
 * (model.c:61-105) and Q8_0 matrices, for tests and benchmarks (no weights
 * are available offline). Values come from a counter-based generator
 * (splitmix64 + Box-Muller, seeded per tensor row) so they do not depend on
 * the thread count: matrices ~N(0, weight_std) and the embedding table
 * ~N(0, embed_std), both quantized to Q8_0 with the reference quantizer
 * rules; norm weights 1 + norm_std*N(0,1). dense_head adds dense_2 {768,
 * 3072} and dense_3 {3072, 768} (Q8_0). */
typedef struct {
    uint64_t seed;
    unsigned n_layer;
    unsigned dense_head;
    float weight_std;
    float embed_std;
    float norm_std;
    float rope_base_full;
    float rope_base_swa;
    unsigned sliding_window;
    unsigned sliding_window_pattern;
    unsigned threads;
} eg2_synth_config;

int eg2_synth_write_gguf(const char *path, const eg2_synth_config *cfg, char *err, size_t len);

#ifdef __cplusplus
}
#endif
#endif
