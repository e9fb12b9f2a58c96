// Row kernels of the packed encoder forward: one 64-lane workgroup per token
// row. They are HBM-bound; each one fuses the element-wise work between two
// GEMMs so a token row is read and written once. Each reproduces the
// reference's operation order, so its results are bit-identical to the CPU
// path for identical inputs (tanhf in the GeGLU kernel is the one libm
// function evaluated on the device).
#include "eg2_device.hpp"
#include "eg2_kernels.hpp"

namespace eg2 {

// Normalises the LDS row `row` (kEmbd floats) with weight w and inverse rms
// `inv` as (x*w)*inv (kernels.c:124-133, SSE2 branch), then quantizes it to
// Q8_0 blocks (quants.c:97-177) written as fp16 integers plus one float
// scale per block. Lane l owns elements l + 64r: its half-wave holds block
// 2r + l/32.
__device__ __forceinline__ void norm_quantize_row(const float* row, const float* __restrict__ w,
                                                  float inv, _Float16* __restrict__ qs,
                                                  float* __restrict__ qd, int k) {
  const int lane = threadIdx.x & 63;
  for (int r = 0; r < k / 64; ++r) {
    const int e = lane + 64 * r;
    const float p = row[e] * w[e];
    const float v = p * inv;
    const Q8Lane q = q8_quantize_lane(v);
    qs[e] = (_Float16)q.q;
    if ((lane & 31) == 0) qd[e / kQK] = q.d;
  }
}

// engine.c:288-295 + kernels.c:139-151 (the next projection's input):
// x = (fp16(d) * sqrt(768)) * q from the raw GGUF Q8_0 row of token_embd,
// then the layer-0 attn_norm RMSNorm quantized to Q8_0.
__global__ void __launch_bounds__(64)
embed_norm_quant_kernel(const uint8_t* __restrict__ table, const int32_t* __restrict__ ids,
                        float embed_scale, const float* __restrict__ norm_w, float eps,
                        float* __restrict__ x, _Float16* __restrict__ xq, float* __restrict__ xd) {
  __shared__ __align__(16) uint8_t raw[kEmbd / kQK * 34];
  __shared__ float row[kEmbd];
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  const uint8_t* src = table + (size_t)ids[t] * (kEmbd / kQK * 34);
  // 816 bytes per row = 51 16-byte chunks; GGUF rows of this tensor are
  // 16-byte aligned because 816 = 16 * 51 and tensor data is 32-aligned.
  if (lane < 51) reinterpret_cast<uint4*>(raw)[lane] = reinterpret_cast<const uint4*>(src)[lane];
  __syncthreads();
  for (int r = 0; r < kEmbd / 64; ++r) {
    const int e = lane + 64 * r;
    const uint8_t* blk = raw + (e / kQK) * 34;
    const uint32_t hbits = (uint32_t)blk[0] | ((uint32_t)blk[1] << 8);
    const float d = fp16_bits_to_fp32(hbits) * embed_scale;  // quants.c:67
    const float v = d * (float)(int8_t)blk[2 + e % kQK];      // quants.c:87
    row[e] = v;
    x[(size_t)t * kEmbd + e] = v;
  }
  __syncthreads();
  const float inv = rms_inverse(sum_squares_sse2(row, kEmbd), kEmbd, eps);
  norm_quantize_row(row, norm_w, inv, xq + (size_t)t * kEmbd, xd + (size_t)t * (kEmbd / kQK), kEmbd);
}

// kernels.c:163-188 (SSE2 build: scalar branch, residual += (h*inv)*w), then
// kernels.c:139-151 with the next norm weight on the updated residual. With
// next_w == nullptr only the residual update runs.
__global__ void __launch_bounds__(64)
residual_norm_quant_kernel(float* __restrict__ x, const float* __restrict__ h,
                           const float* __restrict__ post_w, const float* __restrict__ next_w,
                           float eps, _Float16* __restrict__ xq, float* __restrict__ xd) {
  __shared__ float hrow[kEmbd];
  __shared__ float xrow[kEmbd];
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  for (int r = 0; r < kEmbd / 64; ++r) hrow[lane + 64 * r] = h[(size_t)t * kEmbd + lane + 64 * r];
  __syncthreads();
  const float inv_h = rms_inverse(sum_squares_sse2(hrow, kEmbd), kEmbd, eps);
  for (int r = 0; r < kEmbd / 64; ++r) {
    const int e = lane + 64 * r;
    const float a = hrow[e] * inv_h;
    const float b = a * post_w[e];
    const float v = x[(size_t)t * kEmbd + e] + b;
    xrow[e] = v;
    x[(size_t)t * kEmbd + e] = v;
  }
  if (!next_w) return;
  __syncthreads();
  const float inv = rms_inverse(sum_squares_sse2(xrow, kEmbd), kEmbd, eps);
  norm_quantize_row(xrow, next_w, inv, xq + (size_t)t * kEmbd, xd + (size_t)t * (kEmbd / kQK), kEmbd);
}

// Writes x as the fp16 pair (hi, lo) = (fp16(x), fp16(x - hi)); x - hi is
// exact in fp32, so hi + lo carries 22 of the 24 significand bits.
__device__ __forceinline__ void store_split(_Float16* row, int width, int i, float x) {
  const _Float16 h = (_Float16)x;
  row[i] = h;
  row[width + i] = (_Float16)(x - (float)h);
}

// kernels.c:233-264 on one token of the fused QKV projection output
// [q0 q1 q2 | k | v] (fp32, kQKVCols wide): per-head RMS with the weight
// applied before the inverse, NeoX rotation of pairs (d, d+128) with the
// host-built cos/sin row of this token's position, Q scaled by 0.0625 after
// rotation. The fp32 results (bit-identical to the reference) are written as
// split fp16 pairs for the attention kernel, rows [hi | lo]; q is stored
// times 16 (exact) to keep its low half clear of fp16 subnormals.
__global__ void __launch_bounds__(64)
qk_norm_rope_kernel(const float* __restrict__ qkv, const float* __restrict__ q_w,
                    const float* __restrict__ k_w, const float* __restrict__ rope,
                    const int32_t* __restrict__ pos, float eps, _Float16* __restrict__ qs,
                    _Float16* __restrict__ ks, _Float16* __restrict__ vs) {
  __shared__ float rows[4][kHeadDim];
  __shared__ float inv[4];
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  const float* src = qkv + (size_t)t * kQKVCols;
  for (int i = lane; i < 4 * kHeadDim; i += 64) rows[i / kHeadDim][i % kHeadDim] = src[i];
  for (int i = lane; i < kHeadDim; i += 64) store_split(vs + (size_t)t * 2 * kHeadDim, kHeadDim, i, src[4 * kHeadDim + i]);
  __syncthreads();
  for (int hd = 0; hd < 4; ++hd) {
    const float ss = sum_squares_sse2(rows[hd], kHeadDim);
    if (lane == 0) inv[hd] = rms_inverse(ss, kHeadDim, eps);
  }
  __syncthreads();
  const float* cs = rope + (size_t)pos[t] * kHeadDim;  // [cos 0..127 | sin 0..127]
  constexpr int half = kHeadDim / 2;
  for (int i = lane; i < 4 * half; i += 64) {
    const int hd = i / half, d = i % half;
    const float* w = hd < kHeads ? q_w : k_w;
    const float c = cs[d], s = cs[half + d];
    const float x0 = rows[hd][d] * w[d] * inv[hd];
    const float x1 = rows[hd][d + half] * w[d + half] * inv[hd];
    const float a0 = x0 * c, a1 = x1 * s;
    const float b0 = x0 * s, b1 = x1 * c;
    float lo = a0 - a1, hi = b0 + b1;
    if (hd < kHeads) {
      lo = lo * 0.0625f;
      hi = hi * 0.0625f;
      _Float16* row = qs + (size_t)t * 2 * kEmbd;
      store_split(row, kEmbd, hd * kHeadDim + d, lo * 16.0f);
      store_split(row, kEmbd, hd * kHeadDim + d + half, hi * 16.0f);
    } else {
      _Float16* row = ks + (size_t)t * 2 * kHeadDim;
      store_split(row, kHeadDim, d, lo);
      store_split(row, kHeadDim, d + half, hi);
    }
  }
}

// kernels.c:367-371 and :373-391: gelu_tanh(gate) * up, quantized to Q8_0.
// gu rows hold [gate 0..1151 | up 0..1151].
__global__ void __launch_bounds__(64)
gelu_quant_kernel(const float* __restrict__ gu, _Float16* __restrict__ gq, float* __restrict__ gd) {
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  const float* g = gu + (size_t)t * (2 * kFF);
  const float* u = g + kFF;
  const float a = 0.044715f;
  const float s = 0.79788456080286535587989211986876f;
  for (int r = 0; r < kFF / 64; ++r) {
    const int e = lane + 64 * r;
    const float x = g[e];
    const float inner = s * x * (1.0f + a * x * x);
    const float gelu = 0.5f * x * (1.0f + tanhf(inner));
    const float v = gelu * u[e];
    const Q8Lane q = q8_quantize_lane(v);
    gq[(size_t)t * kFF + e] = (_Float16)q.q;
    if ((lane & 31) == 0) gd[(size_t)t * (kFF / kQK) + e / kQK] = q.d;
  }
}

// quants.c:97-177 on rows of width k (k % 64 == 0).
__global__ void __launch_bounds__(64)
quantize_rows_kernel(const float* __restrict__ x, int k, _Float16* __restrict__ q,
                     float* __restrict__ d) {
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  for (int e = lane; e < k; e += 64) {
    const Q8Lane r = q8_quantize_lane(x[(size_t)t * k + e]);
    q[(size_t)t * k + e] = (_Float16)r.q;
    if ((lane & 31) == 0) d[(size_t)t * (k / kQK) + e / kQK] = r.d;
  }
}

// kernels.c:153-161 in place on a token row: x = (x*w)*inv.
__global__ void __launch_bounds__(64)
rms_norm_rows_kernel(float* __restrict__ x, const float* __restrict__ w, float eps) {
  __shared__ float row[kEmbd];
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  for (int r = 0; r < kEmbd / 64; ++r) row[lane + 64 * r] = x[(size_t)t * kEmbd + lane + 64 * r];
  __syncthreads();
  const float inv = rms_inverse(sum_squares_sse2(row, kEmbd), kEmbd, eps);
  for (int r = 0; r < kEmbd / 64; ++r) {
    const int e = lane + 64 * r;
    const float p = row[e] * w[e];
    x[(size_t)t * kEmbd + e] = p * inv;
  }
}

// kernels.c:417-427 after the per-token RMS (rms_norm_rows_kernel): one
// workgroup per sequence sums its normalised rows in token order, scales by
// 1/n, then L2-normalises in the SSE2 order (kernels.c:393-396).
__global__ void __launch_bounds__(256)
pool_l2_kernel(const float* __restrict__ x, const uint32_t* __restrict__ offsets,
               float* __restrict__ out) {
  __shared__ float acc[kEmbd];
  const int s = blockIdx.x;
  const uint32_t lo = offsets[s], hi = offsets[s + 1];
  for (int e = threadIdx.x; e < kEmbd; e += 256) {
    float sum = 0.0f;
    for (uint32_t t = lo; t < hi; ++t) sum = sum + x[(size_t)t * kEmbd + e];
    const float scale = 1.0f / (float)(hi - lo);
    acc[e] = sum * scale;
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const float ss = sum_squares_sse2(acc, kEmbd);
    const float scale = ss != 0.0f ? 1.0f / __builtin_sqrtf(ss) : 1.0f;
    for (int e = threadIdx.x; e < kEmbd; e += 64) out[(size_t)s * kEmbd + e] = ss != 0.0f ? acc[e] * scale : acc[e];
  }
}

// kernels.c:393-396 on the first `dims` elements of rows of width `width`
// (dims % 8 == 0): the Matryoshka prefix normalisation of kernels.c:398-407
// when dims < width, the plain L2 when dims == width.
__global__ void __launch_bounds__(64)
l2_prefix_kernel(float* __restrict__ x, int width, int dims) {
  extern __shared__ float buf[];
  const int t = blockIdx.x;
  const int lane = threadIdx.x;
  float* row = x + (size_t)t * width;
  for (int e = lane; e < dims; e += 64) buf[e] = row[e];
  __syncthreads();
  const float ss = sum_squares_sse2(buf, dims);
  if (ss == 0.0f) return;
  const float scale = 1.0f / __builtin_sqrtf(ss);
  for (int e = lane; e < dims; e += 64) row[e] = buf[e] * scale;
}

// ---------------------------------------------------------------- launchers

hipError_t launch_embed_norm_quant(const uint8_t* table, const int32_t* ids, int rows, float embed_scale,
                                   const float* norm_w, float eps, float* x, _Float16* xq, float* xd,
                                   hipStream_t st) {
  hipLaunchKernelGGL(embed_norm_quant_kernel, dim3(rows), dim3(64), 0, st, table, ids, embed_scale, norm_w,
                     eps, x, xq, xd);
  return hipGetLastError();
}

hipError_t launch_residual_norm_quant(float* x, const float* h, const float* post_w, const float* next_w,
                                      float eps, _Float16* xq, float* xd, int rows, hipStream_t st) {
  hipLaunchKernelGGL(residual_norm_quant_kernel, dim3(rows), dim3(64), 0, st, x, h, post_w, next_w, eps, xq,
                     xd);
  return hipGetLastError();
}

hipError_t launch_qk_norm_rope(const float* qkv, const float* q_w, const float* k_w, const float* rope,
                               const int32_t* pos, float eps, _Float16* qs, _Float16* ks, _Float16* vs,
                               int rows, hipStream_t st) {
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(rows), dim3(64), 0, st, qkv, q_w, k_w, rope, pos, eps, qs, ks,
                     vs);
  return hipGetLastError();
}

hipError_t launch_gelu_quant(const float* gu, _Float16* gq, float* gd, int rows, hipStream_t st) {
  hipLaunchKernelGGL(gelu_quant_kernel, dim3(rows), dim3(64), 0, st, gu, gq, gd);
  return hipGetLastError();
}

hipError_t launch_quantize_rows(const float* x, int k, _Float16* q, float* d, int rows, hipStream_t st) {
  hipLaunchKernelGGL(quantize_rows_kernel, dim3(rows), dim3(64), 0, st, x, k, q, d);
  return hipGetLastError();
}

hipError_t launch_rms_norm_rows(float* x, const float* w, float eps, int rows, hipStream_t st) {
  hipLaunchKernelGGL(rms_norm_rows_kernel, dim3(rows), dim3(64), 0, st, x, w, eps);
  return hipGetLastError();
}

hipError_t launch_pool_l2(const float* x, const uint32_t* offsets, float* out, int batch, hipStream_t st) {
  hipLaunchKernelGGL(pool_l2_kernel, dim3(batch), dim3(256), 0, st, x, offsets, out);
  return hipGetLastError();
}

hipError_t launch_l2_prefix(float* x, int width, int dims, int rows, hipStream_t st) {
  hipLaunchKernelGGL(l2_prefix_kernel, dim3(rows), dim3(64), (size_t)dims * sizeof(float), st, x, width, dims);
  return hipGetLastError();
}

}  // namespace eg2
