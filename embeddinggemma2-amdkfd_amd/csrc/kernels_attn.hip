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
// Work: query tiles of up to 32 tokens of ONE sequence (host-built list:
// first query, end, sequence start, sequence end); the key tiles of a query
// tile start at its sequence's first token, so a query's arithmetic depends
// only on its own sequence and packed and single-sequence calls give
// bit-identical results. One workgroup per query tile, one wave per query
// head; the three waves share each 32-key tile of K and V^T in LDS.
//
// Data movement: K rows ([hi 256 | lo 256] fp16 per token) and V^T rows
// (V transposed by the QK-norm/RoPE kernel into [hi|lo][256 dims][column],
// each sequence starting at a 32-aligned column, so a key tile is 64
// contiguous bytes per dimension) go from global memory straight into a
// double-buffered LDS ring by DMA (global_load_lds_dwordx4), the next tile
// in flight while the current one is used. 16-byte chunks are XOR-swizzled
// so the MFMA fragment reads hit distinct banks.
//
// Scores are computed transposed, S^T = K . Q^T, so each lane owns one
// query (lane & 31) and 16 of the tile's keys and the softmax reductions
// stay in the lane plus one exchange with lane ^ 32. The K rows are fed to
// the score MFMA in a permuted order chosen so that lane group g ends up
// holding the probabilities of keys 8g..8g+7 and 16+8g..16+8g+7: exactly
// the k-slots it supplies to the two P.V MFMAs, whose V^T operand is then
// one aligned 16-byte chunk per lane.
#include "eg2_device.hpp"
#include "eg2_kernels.hpp"

namespace eg2 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kKvTile = 32;
constexpr int kKStage = kKvTile * 2 * kHeadDim * 2;  // [key][hi|lo][256] fp16 = 32 KB
constexpr int kVStage = 2 * kHeadDim * kKvTile * 2;  // [hi|lo][dim][32 keys] fp16 = 32 KB
constexpr int kStage = kKStage + kVStage;
constexpr int kDmaPerStage = kStage / 1024;          // 1 KB DMA instructions per tile

__device__ __forceinline__ floatx16 mfma(const half8& a, const half8& b, const floatx16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// Key fed to row r of the score MFMA (see the header comment): r holds
// register v = 4 * (r / 8) + r % 4 of lane group g = (r / 4) % 2, which is
// to carry key 8g + v (v < 8) or 16 + 8g + (v - 8) (v >= 8).
__device__ __forceinline__ int score_row_key(int r) {
  const int v = 4 * (r >> 3) + (r & 3), g = (r >> 2) & 1;
  return v < 8 ? 8 * g + v : 16 + 8 * g + (v - 8);
}
// Chunk swizzles: K rows hold 32 chunks of 16 bytes per half (key-XOR);
// V^T rows hold 4 chunks (the GEMM's pattern).
__device__ __forceinline__ int vswz(int d) { return ((d >> 1) ^ (d >> 3)) & 3; }

__global__ void __launch_bounds__(192)
attention_kernel(const _Float16* __restrict__ qs, const _Float16* __restrict__ ks, const _Float16* __restrict__ vt,
                 int ldv, const int32_t* __restrict__ vcol, const uint4* __restrict__ tiles,
                 const uint32_t* __restrict__ tile_count, int window, int rows, _Float16* __restrict__ cq,
                 float* __restrict__ cd) {
  __shared__ __align__(16) unsigned char lds[2 * kStage];

  const int tid = threadIdx.x, lane = tid & 63, head = __builtin_amdgcn_readfirstlane(tid >> 6);
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
    kv_lo = __builtin_amdgcn_readfirstlane(kv_lo);
    kv_hi = __builtin_amdgcn_readfirstlane(kv_hi);
    // Key tiles are aligned to the sequence start; so are the V^T columns.
    const uint32_t k_first = kv_lo >= kv_hi ? kv_hi : seg_lo + ((kv_lo - seg_lo) & ~31u);
    const int col_base = __builtin_amdgcn_readfirstlane(vcol[min(seg_lo, (uint32_t)rows - 1)]) - (int)seg_lo;

    // DMA of key tile k0 into stage s: instructions q = head, head + 3, ...
    // q < 32: K row of key q; lane L takes half L/32, stored chunk L%32 =
    // global chunk (L%32) ^ q. q >= 32: V^T rows 16(q-32)..+15 of half
    // (q-32)/16; lane L takes dim row L/4, stored chunk L%4 = global chunk
    // (L%4) ^ vswz(row).
    auto issue = [&](uint32_t k0, int s) {
      unsigned char* base = lds + s * kStage;
      for (int q = head; q < kDmaPerStage; q += 3) {
        const _Float16* src;
        if (q < kKvTile) {
          const uint32_t key = min(k0 + q, (uint32_t)rows - 1);
          src = ks + (size_t)key * (2 * kHeadDim) + (lane >> 5) * kHeadDim + 8 * ((lane & 31) ^ q);
        } else {
          const int vq = q - kKvTile, hl = vq >> 4, d = 16 * (vq & 15) + (lane >> 2);
          const int c = (lane & 3) ^ vswz(d);
          src = vt + ((size_t)hl * kHeadDim + d) * ldv + (col_base + (int)k0) + 8 * c;
        }
        dma16(src, base + q * 1024);
      }
    };

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

    // Every wave has finished with both stages (previous tile of the grid
    // stride) before the first DMA overwrites them.
    __syncthreads();
    if (k_first < kv_hi) issue(k_first, 0);
    const int kkey = score_row_key(j);  // key row this lane feeds to the score MFMA
    int stage = 0;
    for (uint32_t k0 = k_first; k0 < kv_hi; k0 += kKvTile, stage ^= 1) {
      // This tile's DMA has landed for every wave, and every wave is done
      // with the other stage, which the next tile's DMA now refills.
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      if (k0 + kKvTile < kv_hi) issue(k0 + kKvTile, stage ^ 1);
      const unsigned char* kst = lds + stage * kStage;
      const unsigned char* vst = kst + kKStage;

      floatx16 s = floatx16{};
      const unsigned char* krow = kst + kkey * 1024;
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const int c = (2 * st + g) ^ kkey;
        const half8 kh = *reinterpret_cast<const half8*>(krow + 16 * c);
        const half8 kl = *reinterpret_cast<const half8*>(krow + 512 + 16 * c);
        s = mfma(kh, qh[st], s);
        s = mfma(kh, ql[st], s);
        s = mfma(kl, qh[st], s);
      }
      // s[v] is 16x the score of key k0 + (v < 8 ? 8g + v : 16 + 8g + v - 8).
      float mt = -INFINITY;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const uint32_t key = k0 + (v < 8 ? 8 * g + v : 16 + 8 * g + (v - 8));
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

      // O^T += V^T . P^T: lane group g supplies keys 8g..8g+7 (first MFMA)
      // and 16+8g..16+8g+7 (second), i.e. V^T chunks g and 2 + g.
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const int d = dt * 32 + j, f = vswz(d);
        const unsigned char* vh = vst + d * 64;
        const unsigned char* vl = vst + (kHeadDim + d) * 64;
        const half8 vh0 = *reinterpret_cast<const half8*>(vh + 16 * (g ^ f));
        const half8 vh1 = *reinterpret_cast<const half8*>(vh + 16 * ((2 + g) ^ f));
        const half8 vl0 = *reinterpret_cast<const half8*>(vl + 16 * (g ^ f));
        const half8 vl1 = *reinterpret_cast<const half8*>(vl + 16 * ((2 + g) ^ f));
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
  // The last tile's prefetch never runs past the key range, but a wave may
  // still have DMA in flight if the loop ran no tile; drain before exit.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
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

size_t build_vt_columns(const size_t* offsets, size_t batch, int32_t* vcol) {
  size_t base = 0;
  for (size_t s = 0; s < batch; ++s) {
    for (size_t t = offsets[s]; t < offsets[s + 1]; ++t) vcol[t] = (int32_t)(base + (t - offsets[s]));
    base += (offsets[s + 1] - offsets[s] + 31) / 32 * 32;
  }
  return base;
}

hipError_t launch_attention(const _Float16* qs, const _Float16* ks, const _Float16* vt, int ldv, const int32_t* vcol,
                            const uint32_t* tiles, const uint32_t* tile_count, int grid, int window, int rows,
                            _Float16* cq, float* cd, hipStream_t st) {
  if (rows <= 0 || grid <= 0 || ldv <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_kernel, dim3(grid), dim3(192), 0, st, qs, ks, vt, ldv, vcol,
                     reinterpret_cast<const uint4*>(tiles), tile_count, window, rows, cq, cd);
  return hipGetLastError();
}

}  // namespace eg2
