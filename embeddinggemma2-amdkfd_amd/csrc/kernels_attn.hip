// Packed variable-length bidirectional GQA attention (3 query heads, 1 KV
// head, head_dim 256) on MFMA, for a wave of sequences packed back to back.
//
// Reference semantics (kernels.c:324-360 per segment, engine.c:850-873): a
// query token attends to every key of its own sequence (window == 0) or to
// keys with |q - k| <= window/2 inside it; softmax(q.k) with q already
// scaled by 1/16; the context row is then quantized to Q8_0 for the output
// projection (engine.c:644-648), which this kernel does in its epilogue.
//
// Layout: one workgroup per 32 consecutive query tokens, one wave per query
// head; the three waves share each 32-key K tile and transposed V tile in
// LDS. Scores are computed transposed, S^T = K . Q^T, so each lane owns one
// query (lane & 31) and 16 of the tile's keys and the online-softmax
// reductions stay in the lane plus one exchange with lane ^ 32. Operands are
// fp16, accumulation and softmax fp32.
#include "eg2_device.hpp"
#include "eg2_kernels.hpp"

namespace eg2 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kKvTile = 32;
constexpr int kKStride = kHeadDim + 8;  // fp16 per K row in LDS
constexpr int kVStride = kKvTile + 8;   // fp16 per transposed-V row in LDS

__global__ void __launch_bounds__(192)
attention_kernel(const _Float16* __restrict__ qh, const _Float16* __restrict__ kh,
                 const _Float16* __restrict__ vh, const uint32_t* __restrict__ seg_lo,
                 const uint32_t* __restrict__ seg_hi, int window, int rows, int8_t* __restrict__ cq,
                 float* __restrict__ cd) {
  __shared__ __align__(16) _Float16 Ks[kKvTile * kKStride];
  __shared__ __align__(16) _Float16 Vt[kHeadDim * kVStride];

  const int tid = threadIdx.x, lane = tid & 63, head = tid >> 6;
  const int g = lane >> 5, j = lane & 31;
  const int t = blockIdx.x * 32 + j;

  // Key range of this lane's query (kernels.c:330-336 in packed coordinates).
  // Bounds are clamped to the wave so a malformed range can never address
  // outside the K/V rows (an empty range yields a non-finite row instead).
  uint32_t hi = min(seg_hi[t], (uint32_t)rows);
  uint32_t lo = min(seg_lo[t], hi);
  if (window > 0) {
    const uint32_t half = (uint32_t)(window / 2);
    if ((uint32_t)t > half && (uint32_t)t - half > lo) lo = (uint32_t)t - half;
    if ((uint32_t)t + half + 1 < hi) hi = (uint32_t)t + half + 1;
  }
  uint32_t kv_lo = lo, kv_hi = hi;
#pragma unroll
  for (int mk = 16; mk >= 1; mk >>= 1) {
    kv_lo = min(kv_lo, (uint32_t)__shfl_xor((int)kv_lo, mk, 64));
    kv_hi = max(kv_hi, (uint32_t)__shfl_xor((int)kv_hi, mk, 64));
  }

  // Q^T operand: lane holds query j, dims 16s + 8g .. +7 for s = 0..15.
  half8 qf[16];
  const _Float16* qrow = qh + (size_t)t * kEmbd + head * kHeadDim;
#pragma unroll
  for (int s = 0; s < 16; ++s) qf[s] = *reinterpret_cast<const half8*>(qrow + 16 * s + 8 * g);

  floatx16 acc[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = floatx16{};
  float m_run = -INFINITY, l_run = 0.0f;

  for (uint32_t k0 = kv_lo & ~31u; k0 < kv_hi; k0 += kKvTile) {
    __syncthreads();
    for (int c = tid; c < kKvTile * 32; c += 192) {
      const int row = c >> 5, col = (c & 31) * 8;
      *reinterpret_cast<half8*>(&Ks[row * kKStride + col]) =
          *reinterpret_cast<const half8*>(kh + (size_t)(k0 + row) * kHeadDim + col);
    }
    for (int c = tid; c < kKvTile * 32; c += 192) {
      const int key = c & 31, d0 = (c >> 5) * 8;
      const half8 v = *reinterpret_cast<const half8*>(vh + (size_t)(k0 + key) * kHeadDim + d0);
#pragma unroll
      for (int i = 0; i < 8; ++i) Vt[(d0 + i) * kVStride + key] = v[i];
    }
    __syncthreads();

    floatx16 s = floatx16{};
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      const half8 kf = *reinterpret_cast<const half8*>(&Ks[j * kKStride + 16 * st + 8 * g]);
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf, qf[st], s, 0, 0, 0);
    }
    // s[v] is the score of key k0 + 8*(v/4) + 4*g + (v%4) for query j.
    float mt = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const uint32_t key = k0 + 8 * (v >> 2) + 4 * g + (v & 3);
      const bool valid = key >= lo && key < hi;
      s[v] = valid ? s[v] : -INFINITY;
      mt = fmaxf(mt, s[v]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float m_new = fmaxf(m_run, mt);
    const float alpha = m_run == -INFINITY ? 0.0f : expf(m_run - m_new);
    float psum = 0.0f;
    half8 pb0, pb1;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const float p = s[v] == -INFINITY ? 0.0f : expf(s[v] - m_new);
      psum += p;
      if (v < 8)
        pb0[v] = (_Float16)p;
      else
        pb1[v - 8] = (_Float16)p;
    }
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;

    // O^T += V^T . P^T. The k-slots of lane group g map to keys
    // {4g..4g+3, 8+4g..8+4g+3} (first MFMA) and {16+4g.., 24+4g..} (second),
    // matching the keys this lane holds probabilities for.
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const _Float16* vrow = &Vt[(dt * 32 + j) * kVStride];
      const half4 a0 = *reinterpret_cast<const half4*>(vrow + 4 * g);
      const half4 a1 = *reinterpret_cast<const half4*>(vrow + 8 + 4 * g);
      const half4 a2 = *reinterpret_cast<const half4*>(vrow + 16 + 4 * g);
      const half4 a3 = *reinterpret_cast<const half4*>(vrow + 24 + 4 * g);
      const half8 va0 = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
      const half8 va1 = {a2[0], a2[1], a2[2], a2[3], a3[0], a3[1], a3[2], a3[3]};
      acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va0, pb0, acc[dt], 0, 0, 0);
      acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va1, pb1, acc[dt], 0, 0, 0);
    }
  }

  // Epilogue: context = acc / l, then Q8_0 per 32 dims (one d-tile = one
  // block). acc[dt][v] is dim dt*32 + 8*(v/4) + 4*g + (v%4) of query j.
  const float inv_l = 1.0f / l_run;
  int8_t* qrow_out = cq + (size_t)t * kEmbd + head * kHeadDim;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    float vals[16];
    float amax = 0.0f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      vals[v] = acc[dt][v] * inv_l;
      amax = fmaxf(amax, fabsf(vals[v]));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    const float d = amax / 127.0f;
    const float dq = fp16_bits_to_fp32(fp32_to_fp16_bits(d));
    const float id = amax == 0.0f ? 0.0f : 1.0f / d;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      uint32_t packed = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int32_t q = amax == 0.0f ? 0 : q8_round(vals[4 * a + c] * id);
        packed |= ((uint32_t)(q & 0xFF)) << (8 * c);
      }
      *reinterpret_cast<uint32_t*>(qrow_out + dt * 32 + 8 * a + 4 * g) = packed;
    }
    if (g == 0) cd[(size_t)t * (kEmbd / kQK) + head * (kHeadDim / kQK) + dt] = dq;
  }
}

hipError_t launch_attention(const _Float16* qh, const _Float16* kh, const _Float16* vh, const uint32_t* seg_lo,
                            const uint32_t* seg_hi, int window, int rows, int8_t* cq, float* cd, hipStream_t st) {
  if (rows <= 0 || rows % 32 != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_kernel, dim3(rows / 32), dim3(192), 0, st, qh, kh, vh, seg_lo, seg_hi, window, rows,
                     cq, cd);
  return hipGetLastError();
}

}  // namespace eg2
