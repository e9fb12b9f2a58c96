// Launchers of the gfx950 kernels (host side). All pointers are device
// pointers; row counts are token rows of the packed wave. Q8_0 activations
// are int8 row tiles (q8_tile_offset; buffers hold the rows rounded up to
// 32) plus one float scale per 32-block stored transposed, [k/32][rows];
// attention operands are split fp16 rows [hi | lo].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eg2 {

hipError_t launch_embed_norm_quant(const uint8_t* table, const int32_t* ids, int rows, float embed_scale,
                                   const float* norm_w, float eps, float* x, int8_t* xq, float* xd,
                                   hipStream_t st);
hipError_t launch_residual_norm_quant(float* x, const float* h, const float* post_w, const float* next_w,
                                      float eps, int8_t* xq, float* xd, int rows, hipStream_t st);
hipError_t launch_qk_norm_rope(const float* qkv, const float* q_w, const float* k_w, const float* rope,
                               const int32_t* pos, const int32_t* vcol, float eps, _Float16* qs, _Float16* ks,
                               _Float16* vt, int ldv, int rows, hipStream_t st);
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
                                   const int32_t* pos, const int32_t* vcol, float eps, _Float16* qs, _Float16* ks,
                                   _Float16* vt, int ldv, hipStream_t st);
hipError_t launch_gemm_q8_geglu(const int8_t* xq, const float* xd, int ldx, const int8_t* wq, const float* wd, int ldw,
                                int8_t* gq, float* gd, int ldg, int n, int ff, int k, hipStream_t st);
hipError_t launch_attention(const _Float16* qs, const _Float16* ks, const _Float16* vt, int ldv, const uint32_t* items,
                            const uint32_t* item_count, int grid, int window, int rows, int8_t* cq, float* cd,
                            float* partials, hipStream_t st);
hipError_t launch_attention_merge(const uint32_t* merges, const uint32_t* merge_count, int grid, const float* partials,
                                  int rows, int8_t* cq, float* cd, hipStream_t st);

// Work lists of launch_attention / launch_attention_merge for the
// sequences [offsets[s], offsets[s+1]): per query tile of up to 16 tokens
// of one sequence, one item (8 uint32: first query, end, sequence start,
// sequence end, key chunk start, key chunk end, partial slot or
// 0xFFFFFFFF, 0) per key chunk -- a sequence of n > 256 tokens splits its
// keys into min(ceil(n / 256), 4) chunks of equal size rounded up to 32,
// whose partial results go to consecutive slots -- and, for split tiles,
// one merge record (first query, end, first slot, parts). attention_capacity bounds the counts for a wave of
// `tokens` tokens in at most `batch` sequences.
struct AttentionCounts {
  unsigned items, merges, slots;
};
AttentionCounts build_attention_items(const size_t* offsets, size_t batch, uint32_t* items, uint32_t* merges);
AttentionCounts attention_capacity(size_t tokens, size_t batch);
constexpr size_t kAttentionPartialFloats = 2 * 3 * (16 * 64 * 4 + 64 * 2);  // per slot: 2 query blocks x 3 heads

// V^T column of every token: each sequence starts at a multiple of 32,
// consecutive tokens take consecutive columns. Returns the column count
// used (sequences rounded up to 32 tokens each).
size_t build_vt_columns(const size_t* offsets, size_t batch, int32_t* vcol);

}  // namespace eg2
