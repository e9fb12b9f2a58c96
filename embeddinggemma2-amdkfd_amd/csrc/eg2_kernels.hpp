// Launchers of the gfx950 kernels (host side). All pointers are device
// pointers; row counts are token rows of the packed wave. Q8_0 activations
// are int8 row tiles (q8_tile_offset; buffers hold the rows rounded up to
// 32) plus one float scale per 32-block stored transposed, [k/32][rows];
// attention reads fp32 rows [q0 q1 q2 | k | v].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eg2 {

hipError_t launch_embed_norm_quant(const uint8_t* table, const int32_t* ids, int rows, float embed_scale,
                                   const float* norm_w, float eps, float* x, int8_t* xq, float* xd,
                                   hipStream_t st);
hipError_t launch_residual_norm_quant(float* x, const float* h, const float* post_w, const float* next_w,
                                      float eps, int8_t* xq, float* xd, int rows, hipStream_t st);
// QK-norm / RoPE on rows of the fused projection [q0 q1 q2 | k | v]
// (kQKVCols fp32 each): q heads and k normalised and rotated, q scaled by
// 1/16, v copied; in place when out == qkv.
hipError_t launch_qk_norm_rope(const float* qkv, const float* q_w, const float* k_w, const float* rope,
                               const int32_t* pos, float eps, float* out, int rows, hipStream_t st);
hipError_t launch_libm_eval(const float* x, unsigned n, float* e, float* t, hipStream_t st);
// *out (a zeroed uint32) := the bits of max |tanh_approx(x) - tanhf(x)| over
// every finite float x (an exhaustive sweep of the 2^32 bit patterns).
hipError_t launch_tanh_approx_error(uint32_t* out, hipStream_t st);
hipError_t launch_gelu_quant(const float* gu, int8_t* gq, float* gd, int rows, hipStream_t st);
hipError_t launch_quantize_rows(const float* x, int k, int8_t* q, float* d, int rows, hipStream_t st);
hipError_t launch_rms_norm_rows(float* x, const float* w, float eps, int rows, hipStream_t st);
hipError_t launch_pool_l2(const float* x, const uint32_t* offsets, float* out, int batch, hipStream_t st);
hipError_t launch_pool_mean(const float* x, const uint32_t* offsets, float* out, int batch, hipStream_t st);
hipError_t launch_l2_prefix(float* x, int width, int dims, int rows, hipStream_t st);
// xq/wq: int8 row tiles of the activations [n][k] and weights [m][k];
// xd/wd: their block scales transposed, [k/32][ldx] and [k/32][ldw].
hipError_t launch_gemm_q8(const int8_t* xq, const float* xd, int ldx, const int8_t* wq, const float* wd, int ldw,
                          float* y, int n, int m, int k, int ldy, hipStream_t st);
hipError_t launch_gemm_q8_qkv_rope(const int8_t* xq, const float* xd, int ldx, const int8_t* wq, const float* wd,
                                   int ldw, int n, int k, const float* q_w, const float* k_w, const float* rope,
                                   const int32_t* pos, float eps, float* out, hipStream_t st);
hipError_t launch_gemm_q8_geglu(const int8_t* xq, const float* xd, int ldx, const int8_t* wq, const float* wd, int ldw,
                                int8_t* gq, float* gd, int ldg, int n, int ff, int k, hipStream_t st);

// Attention over the rows [q0 q1 q2 | k | v] of a packed wave, bit-exact
// with the reference (see kernels_attn.hip). `items` holds item_count[0]
// score items (8 uint32: sequence start, end, first key of a 32-key
// block, first pair, end of the pairs, the sequence's first score index,
// 0, 0) followed by item_count[1] context items (sequence start, end,
// first pair of a 32-pair block, end of the pairs, first score index, the
// context kernel's unit order (1: XCD-contiguous eighths, 0: plain stride;
// the same in every context item), 0, 0); a pair is 3 (token - start) +
// head. tok: one record per row (4
// uint32: sequence start, end, first score index, 0). `grid` workgroups
// stride over each item list. scores: the plan's score floats (the 1/sum
// of each (token, head) at [3 t + h], then a row of ceil4(n) scores per
// pair of each sequence of n tokens). The context is quantized to Q8_0
// into cq (row tiles, k = 768) and cd [24][rows]. rows % 4 == 0. longest:
// the longest sequence of the packing, which picks the softmax's kernel
// form (0 = not known: the form for any length); the results are the same.
// The forms change at these lengths: up to kSoftmaxLanes16 tokens 16 lanes
// per (token, head) pair, up to kSoftmaxLanes32 32 lanes, up to
// kSoftmaxWave a wave per pair, any length beyond (a caller that keeps one
// graph per form can round its longest up to the next of them).
constexpr int kSoftmaxLanes16 = 128, kSoftmaxLanes32 = 256, kSoftmaxWave = 512;
hipError_t launch_attention(const float* qkv, const uint32_t* items, const uint32_t* item_count, int grid,
                            const uint32_t* tok, int window, int rows, int longest, float* scores, int8_t* cq,
                            float* cd, hipStream_t st);
// launch_attention's three stages, in that order (one kernel each), for
// callers that time them one by one.
hipError_t launch_attention_scores(const float* qkv, const uint32_t* items, const uint32_t* item_count, int grid,
                                   int window, int rows, float* scores, hipStream_t st);
hipError_t launch_attention_softmax(const uint32_t* tok, int window, int rows, int longest, float* scores,
                                    hipStream_t st);
hipError_t launch_attention_context(const float* qkv, const uint32_t* items, const uint32_t* item_count, int grid,
                                    int window, int rows, const float* scores, int8_t* cq, float* cd,
                                    hipStream_t st);

// The plan of launch_attention for the sequences [offsets[s], offsets[s+1])
// (rows = offsets[batch]): a sequence of n tokens has ceil(n/32) key
// blocks times ceil(3n/32) pair blocks of score items, ceil(3n/32)
// context items and 3 n ceil4(n) score floats, after the 1/sum area of
// ceil4(3 rows). attention_counts gives the counts of a packing
// (items = both kinds); build_attention_plan writes the lists when they
// fit `cap` (else returns false having written nothing) and reports the
// counts in *used; attention_capacity bounds the counts of any packing of
// `tokens` tokens into at most `batch` sequences.
struct AttentionCounts {
  size_t items, score_floats, score_items;
};
AttentionCounts attention_counts(const size_t* offsets, size_t batch);
bool build_attention_plan(const size_t* offsets, size_t batch, const AttentionCounts& cap, uint32_t* items,
                          uint32_t* tok, AttentionCounts* used);
AttentionCounts attention_capacity(size_t tokens, size_t batch);

// Workgroups of the scores and context kernels (four per CU), striding
// over their items.
constexpr int kAttentionGrid = 1024;

// launch_attention with the plan built on the device from the device
// sequence bounds offsets[0..batch] (offsets[0] read as 0, offsets[batch]
// as rows, the rest clamped into a non-decreasing list) and the plan and
// scores kept in a static per-device array: no allocation. rows <= 2048,
// rows % 4 == 0, batch <= 2048. Calls overlapping on one device race.
hipError_t launch_attention_static(const float* qkv, const uint32_t* offsets, int batch, int window, int rows,
                                   int8_t* cq, float* cd, hipStream_t st);

}  // namespace eg2
