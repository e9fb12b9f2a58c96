// Packed variable-length bidirectional GQA attention (3 query heads, 1 KV
// head, head_dim 256) on MFMA, for a wave of sequences packed back to back.
//
// Reference semantics (kernels.c:324-360 per segment, engine.c:850-873): a
// query token attends to every key of its own sequence (window == 0) or to
// keys with |q - k| <= window/2 inside it; softmax(q.k) with q already
// scaled by 1/16; the context row is then quantized to Q8_0 for the output
// projection (engine.c:644-648), which this kernel does in its epilogue.
//
// Precision: q, k, v arrive as fp32 values split into fp16 pairs
// (hi = fp16(x), lo = fp16(x - hi); q pre-multiplied by 16 to stay clear of
// fp16 subnormals), and the probabilities are split the same way, so every
// product is formed as hi*hi + hi*lo + lo*hi on v_mfma_f32_32x32x16_f16 with
// fp32 accumulation: about 2^-21 relative error per product, i.e. fp32-level
// attention. Softmax runs in fp32 (online, one pass over 32-key tiles).
//
// Layout: work is cut into query tiles of up to 32 tokens of ONE sequence
// (host-built list: first query, end, sequence start, sequence end); the
// key tiles of a query tile start at its sequence's first token. A query's
// arithmetic therefore depends only on its own sequence, never on where the
// sequence sits in the packed wave, so packed and single-sequence calls give
// bit-identical results. One workgroup (one wave per query head; the three
// waves share each 32-key K tile and transposed V tile in LDS) loops over
// the tile list with a grid stride. Scores are computed transposed,
// S^T = K . Q^T, so each lane owns one query (lane & 31) and 16 of the
// tile's keys, and the softmax reductions stay in the lane plus one
// exchange with lane ^ 32.
#include "eg2_device.hpp"
#include "eg2_kernels.hpp"

namespace eg2 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kKvTile = 32;
constexpr int kKStride = kHeadDim + 8;  // fp16 per K row in LDS
constexpr int kVStride = kKvTile + 8;   // fp16 per transposed-V row in LDS

__device__ __forceinline__ floatx16 mfma(const half8& a, const half8& b, const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__global__ void __launch_bounds__(192)
attention_kernel(const _Float16* __restrict__ qs, const _Float16* __restrict__ ks,
                 const _Float16* __restrict__ vs, const uint4* __restrict__ tiles,
                 const uint32_t* __restrict__ tile_count, int window, int rows, _Float16* __restrict__ cq,
                 float* __restrict__ cd) {
  __shared__ __align__(16) _Float16 Kh[kKvTile * kKStride];
  __shared__ __align__(16) _Float16 Kl[kKvTile * kKStride];
  __shared__ __align__(16) _Float16 Vh[kHeadDim * kVStride];
  __shared__ __align__(16) _Float16 Vl[kHeadDim * kVStride];

  const int tid = threadIdx.x, lane = tid & 63, head = tid >> 6;
  const int g = lane >> 5, j = lane & 31;
  const uint32_t count = *tile_count;
  for (uint32_t tile = blockIdx.x; tile < count; tile += gridDim.x) {
    // Tile fields are clamped to the wave so a malformed list can never
    // address outside the rows (an empty key range yields a non-finite row).
    const uint4 tl = tiles[tile];
    const uint32_t seg_hi = min(tl.w, (uint32_t)rows);
    const uint32_t seg_lo = min(tl.z, seg_hi);
    const uint32_t q_end = min(tl.y, (uint32_t)rows);
    const uint32_t q0 = tl.x;
    const bool active = q0 + j < q_end;
    const uint32_t t = active ? q0 + j : (q_end > 0 ? q_end - 1 : 0);

    // Key range of this lane's query (kernels.c:330-336 in packed coordinates).
    uint32_t lo = seg_lo, hi = seg_hi;
    if (window > 0) {
      const uint32_t half = (uint32_t)(window / 2);
      if (t > half && t - half > lo) lo = t - half;
      if (t + half + 1 < hi) hi = t + half + 1;
    }
    uint32_t kv_lo = active ? lo : 0xFFFFFFFFu, kv_hi = active ? hi : 0u;
#pragma unroll
    for (int mk = 16; mk >= 1; mk >>= 1) {
      kv_lo = min(kv_lo, (uint32_t)__shfl_xor((int)kv_lo, mk, 64));
      kv_hi = max(kv_hi, (uint32_t)__shfl_xor((int)kv_hi, mk, 64));
    }
    // Key tiles are aligned to the sequence start.
    const uint32_t k_first = kv_lo >= kv_hi ? kv_hi : seg_lo + ((kv_lo - seg_lo) & ~31u);

    // Q^T operand: lane holds query t, dims 16s + 8g .. +7 for s = 0..15.
    // Rows of qs are [hi 768 | lo 768].
    half8 qh[16], ql[16];
    const _Float16* qrow = qs + (size_t)t * (2 * kEmbd) + head * kHeadDim;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      qh[s] = *reinterpret_cast<const half8*>(qrow + 16 * s + 8 * g);
      ql[s] = *reinterpret_cast<const half8*>(qrow + kEmbd + 16 * s + 8 * g);
    }

    floatx16 acc[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[dt] = floatx16{};
    float m_run = -INFINITY, l_run = 0.0f;

    for (uint32_t k0 = k_first; k0 < kv_hi; k0 += kKvTile) {
      __syncthreads();
      // Rows past the wave (last tile of the last sequence) are read from the
      // final row and masked below.
      for (int c = tid; c < kKvTile * 32; c += 192) {
        const int row = c >> 5, col = (c & 31) * 8;
        const _Float16* src = ks + (size_t)min(k0 + row, (uint32_t)rows - 1) * (2 * kHeadDim) + col;
        *reinterpret_cast<half8*>(&Kh[row * kKStride + col]) = *reinterpret_cast<const half8*>(src);
        *reinterpret_cast<half8*>(&Kl[row * kKStride + col]) = *reinterpret_cast<const half8*>(src + kHeadDim);
      }
      for (int c = tid; c < kKvTile * 32; c += 192) {
        const int key = c & 31, d0 = (c >> 5) * 8;
        const _Float16* src = vs + (size_t)min(k0 + key, (uint32_t)rows - 1) * (2 * kHeadDim) + d0;
        const half8 a = *reinterpret_cast<const half8*>(src);
        const half8 b = *reinterpret_cast<const half8*>(src + kHeadDim);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          Vh[(d0 + i) * kVStride + key] = a[i];
          Vl[(d0 + i) * kVStride + key] = b[i];
        }
      }
      __syncthreads();

      floatx16 s = floatx16{};
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const half8 kh = *reinterpret_cast<const half8*>(&Kh[j * kKStride + 16 * st + 8 * g]);
        const half8 kl = *reinterpret_cast<const half8*>(&Kl[j * kKStride + 16 * st + 8 * g]);
        s = mfma(kh, qh[st], s);
        s = mfma(kh, ql[st], s);
        s = mfma(kl, qh[st], s);
      }
      // s[v] is 16x the score of key k0 + 8*(v/4) + 4*g + (v%4) for query t.
      float mt = -INFINITY;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const uint32_t key = k0 + 8 * (v >> 2) + 4 * g + (v & 3);
        const bool valid = key >= lo && key < hi;
        s[v] = valid ? s[v] * 0.0625f : -INFINITY;
        mt = fmaxf(mt, s[v]);
      }
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      const float m_new = fmaxf(m_run, mt);
      const float alpha = m_run == -INFINITY ? 0.0f : expf(m_run - m_new);
      float psum = 0.0f;
      half8 ph0, ph1, pl0, pl1;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p = s[v] == -INFINITY ? 0.0f : expf(s[v] - m_new);
        psum += p;
        const _Float16 h = (_Float16)p;
        const _Float16 l = (_Float16)(p - (float)h);
        if (v < 8) {
          ph0[v] = h;
          pl0[v] = l;
        } else {
          ph1[v - 8] = h;
          pl1[v - 8] = l;
        }
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
        const int r = (dt * 32 + j) * kVStride;
        const half4 a0 = *reinterpret_cast<const half4*>(&Vh[r + 4 * g]);
        const half4 a1 = *reinterpret_cast<const half4*>(&Vh[r + 8 + 4 * g]);
        const half4 a2 = *reinterpret_cast<const half4*>(&Vh[r + 16 + 4 * g]);
        const half4 a3 = *reinterpret_cast<const half4*>(&Vh[r + 24 + 4 * g]);
        const half4 b0 = *reinterpret_cast<const half4*>(&Vl[r + 4 * g]);
        const half4 b1 = *reinterpret_cast<const half4*>(&Vl[r + 8 + 4 * g]);
        const half4 b2 = *reinterpret_cast<const half4*>(&Vl[r + 16 + 4 * g]);
        const half4 b3 = *reinterpret_cast<const half4*>(&Vl[r + 24 + 4 * g]);
        const half8 vh0 = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        const half8 vh1 = {a2[0], a2[1], a2[2], a2[3], a3[0], a3[1], a3[2], a3[3]};
        const half8 vl0 = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
        const half8 vl1 = {b2[0], b2[1], b2[2], b2[3], b3[0], b3[1], b3[2], b3[3]};
        acc[dt] = mfma(vh0, ph0, acc[dt]);
        acc[dt] = mfma(vh0, pl0, acc[dt]);
        acc[dt] = mfma(vl0, ph0, acc[dt]);
        acc[dt] = mfma(vh1, ph1, acc[dt]);
        acc[dt] = mfma(vh1, pl1, acc[dt]);
        acc[dt] = mfma(vl1, ph1, acc[dt]);
      }
    }

    // Epilogue: context = acc / l, then Q8_0 per 32 dims (one d-tile = one
    // block; quants.c:97-177). acc[dt][v] is dim dt*32 + 8*(v/4) + 4*g + (v%4)
    // of query t. Values are stored as fp16 integers with a float scale, the
    // scales transposed ([block][row]) for the projection GEMM.
    const float inv_l = 1.0f / l_run;
    _Float16* out = cq + (size_t)t * kEmbd + head * kHeadDim;
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
      if (!active) continue;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        half4 q4;
#pragma unroll
        for (int c = 0; c < 4; ++c) q4[c] = (_Float16)(amax == 0.0f ? 0 : q8_round(vals[4 * a + c] * id));
        *reinterpret_cast<half4*>(out + dt * 32 + 8 * a + 4 * g) = q4;
      }
      if (g == 0) cd[(size_t)(head * (kHeadDim / kQK) + dt) * rows + t] = dq;
    }
  }
}

unsigned build_attention_tiles(const size_t* offsets, size_t batch, uint32_t* tiles) {
  unsigned n = 0;
  for (size_t s = 0; s < batch; ++s)
    for (size_t q = offsets[s]; q < offsets[s + 1]; q += 32) {
      const size_t e = q + 32 < offsets[s + 1] ? q + 32 : offsets[s + 1];
      tiles[4 * n + 0] = (uint32_t)q;
      tiles[4 * n + 1] = (uint32_t)e;
      tiles[4 * n + 2] = (uint32_t)offsets[s];
      tiles[4 * n + 3] = (uint32_t)offsets[s + 1];
      ++n;
    }
  return n;
}

hipError_t launch_attention(const _Float16* qs, const _Float16* ks, const _Float16* vs, const uint32_t* tiles,
                            const uint32_t* tile_count, int grid, int window, int rows, _Float16* cq, float* cd,
                            hipStream_t st) {
  if (rows <= 0 || grid <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_kernel, dim3(grid), dim3(192), 0, st, qs, ks, vs,
                     reinterpret_cast<const uint4*>(tiles), tile_count, window, rows, cq, cd);
  return hipGetLastError();
}

}  // namespace eg2
