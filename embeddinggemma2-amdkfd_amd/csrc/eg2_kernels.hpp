// Launchers of the gfx950 kernels (host side). All pointers are device
// pointers; row counts are token rows of the packed wave.
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
                               const int32_t* pos, float eps, _Float16* qh, _Float16* kh, _Float16* vh,
                               int rows, hipStream_t st);
hipError_t launch_gelu_quant(const float* gu, int8_t* gq, float* gd, int rows, hipStream_t st);
hipError_t launch_quantize_rows(const float* x, int k, int8_t* q, float* d, int rows, hipStream_t st);
hipError_t launch_rms_norm_rows(float* x, const float* w, float eps, int rows, hipStream_t st);
hipError_t launch_pool_l2(const float* x, const uint32_t* offsets, float* out, int batch, hipStream_t st);
hipError_t launch_l2_prefix(float* x, int width, int dims, int rows, hipStream_t st);
hipError_t launch_gemm_q8(const int8_t* xq, const float* xd, const int8_t* wq, const float* wd, float* y, int n,
                          int m, int k, int ldy, hipStream_t st);
hipError_t launch_attention(const _Float16* qh, const _Float16* kh, const _Float16* vh, const uint32_t* seg_lo,
                            const uint32_t* seg_hi, int window, int rows, int8_t* cq, float* cd, hipStream_t st);

}  // namespace eg2
