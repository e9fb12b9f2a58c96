// Packed variable-length bidirectional GQA attention (3 query heads, 1 KV
// head, head_dim 256) for a wave of sequences packed back to back, with the
// reference's arithmetic: the context is bit-identical to the CPU path.
//
// Reference (kernels.c:324-360 per sequence, engine.c:850-873): for query
// token t and head h, over the keys kt of t's sequence (limited to
// |t - kt| <= window/2 when window > 0), in key order:
//   score[kt] = dot(q[t,h], k[kt])       four interleaved fp32 chains of 64
//                                         products, then (s0+s2)+(s1+s3)
//                                         (ei_dot_f32's SSE2 branch,
//                                         kernels.c:289-294, and its
//                                         horizontal sum, kernels.c:34-39)
//   m = max score;  p[kt] = expf(score[kt] - m);  sum = p[first] + ... (sequential)
//   out = 0;  out += (p[kt] * (1/sum)) * v[kt]   (sequential over kt)
// then the context row is quantized to Q8_0 for the output projection
// (engine.c:644-648). Every multiply and add is one rounded fp32 operation
// in that order; expf is the host libm's own algorithm (eg2_libm.hpp).
// A last-bit difference here would become a different Q8_0 quantum, and
// through the 24 quantized layers a different embedding, so the kernels
// reproduce the order exactly: on the VALU, since no matrix instruction
// rounds each product before adding it.
//
// Operands: the rows [q0 q1 q2 | k | v] (1280 fp32) that QK-norm/RoPE
// leaves, one per token (q already scaled by 1/16).
//
// Two kernels:
//  - attention_scores_kernel: work items of (sequence, 64 keys, a chunk of
//    its queries). The workgroup stages the 64 K rows in LDS (one per lane,
//    rows 260 floats apart so the lanes' 16-byte reads fall in distinct
//    banks); each wave takes 4 (token, head) pairs at a time, whose q values
//    are wave-uniform scalar loads, and runs the 4 chains of each of the 4
//    dot products per lane: 32 multiplies and adds per 4 dimensions. The
//    scores go to a scratch buffer, one row of the sequence's length per
//    (token, head).
//  - attention_context_kernel: one wave per token, its 3 heads. The row
//    maxima; then per 64-key chunk every lane's expf of its key (for all 3
//    heads) into LDS, and lanes 0-2 add their head's chunk to its sum in key
//    order; 1/sum; then the chunk's scales p * (1/sum) into LDS and, key by
//    key, the lanes' 4 dimensions of each head's context (12 multiplies and
//    adds per key and lane, the V row read once for the 3 heads). The Q8_0
//    epilogue quantizes 32-dimension blocks over 8 lanes.
// A sequence's keys, scores and context depend only on its own tokens, so
// packing never changes a bit.
#include <algorithm>
#include <mutex>

#include "eg2_device.hpp"
#include "eg2_kernels.hpp"
#include "eg2_libm.hpp"

namespace eg2 {

constexpr int kKeyBlock = 64;          // keys of a scores work item, one per lane
constexpr int kKPitch = kHeadDim + 4;  // floats per LDS K row: 4 banks apart, so 8 lanes' b128 reads cover all 32
constexpr int kPairs = 2;              // (token, head) pairs per pass of a scores wave
constexpr int kLd = kQKVCols;          // floats per operand row [q0 q1 q2 | k | v]
constexpr int kKOff = kHeads * kHeadDim, kVOff = kKOff + kHeadDim;

// Query tokens per scores work item: longer sequences take more queries per
// staged K block (fewer restagings); shorter ones fewer (more items to
// spread over the CUs). A function of the length alone.
__host__ __device__ inline size_t query_chunk(size_t len) { return len <= 128 ? 8 : (len <= 512 ? 16 : 32); }

// Key range of query token t in its sequence [lo, hi) (kernels.c:330-336
// in packed coordinates): the sequence, or |t - kt| <= window/2.
__host__ __device__ inline void key_range(uint32_t t, uint32_t lo, uint32_t hi, int window, uint32_t& first,
                                          uint32_t& last) {
  const uint32_t half = window > 0 ? (uint32_t)(window / 2) : 0u;
  first = window > 0 && t - lo > half ? t - half : lo;
  last = window > 0 && t + half + 1 < hi ? t + half + 1 : hi;
}

__global__ void __launch_bounds__(256)
attention_scores_kernel(const float* __restrict__ qkv, const uint4* __restrict__ items,
                        const uint32_t* __restrict__ item_count, int window, int rows,
                        float* __restrict__ scores) {
  __shared__ __align__(16) float kblk[kKeyBlock * kKPitch];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t count = *item_count;
  for (uint32_t item = blockIdx.x; item < count; item += gridDim.x) {
    // Item fields clamped to the wave, so a malformed list cannot address
    // outside the rows.
    const uint4 a = items[2 * item], b = items[2 * item + 1];
    const uint32_t hi = min(a.y, (uint32_t)rows), lo = min(a.x, hi);
    const uint32_t key0 = a.z, q1 = min(b.x, hi), q0 = max(min(a.w, q1), lo);
    const uint32_t len = hi - lo;
    const size_t sbase = b.y;
    if (len == 0 || key0 < lo || key0 >= hi) continue;  // uniform over the workgroup
    __syncthreads();  // the previous item's K rows are no longer read
    // K rows key0 .. key0 + 63 (clamped to the sequence's last), 16 float4
    // per thread, 64 threads per row.
#pragma unroll
    for (int j = 0; j < kKeyBlock * kHeadDim / 4 / 256; ++j) {
      const int idx = tid + 256 * j, r = idx >> 6, c4 = idx & 63;
      const uint32_t key = min(key0 + (uint32_t)r, hi - 1);
      *reinterpret_cast<float4*>(kblk + r * kKPitch + 4 * c4) =
          *reinterpret_cast<const float4*>(qkv + (size_t)key * kLd + kKOff + 4 * c4);
    }
    __syncthreads();
    const float* krow = kblk + lane * kKPitch;
    const uint32_t key = key0 + lane;
    const uint32_t pairs = 3 * (q1 - q0);
    for (uint32_t g = (uint32_t)w; kPairs * g < pairs; g += 4) {
      uint32_t t[kPairs], h[kPairs];
      bool in[kPairs];
      bool any = false;
#pragma unroll
      for (int i = 0; i < kPairs; ++i) {
        const uint32_t c = min(kPairs * g + i, pairs - 1);  // past the end: repeats the last pair, not stored
        t[i] = q0 + c / 3;
        h[i] = c % 3;
        uint32_t first, last;
        key_range(t[i], lo, hi, window, first, last);
        in[i] = kPairs * g + i < pairs && key >= first && key < last;
        any |= in[i];
      }
      if (!__builtin_amdgcn_ballot_w64(any)) continue;  // no key of the block in range for these pairs
      const float* qrow[kPairs];
#pragma unroll
      for (int i = 0; i < kPairs; ++i) qrow[i] = qkv + (size_t)t[i] * kLd + h[i] * kHeadDim;
      // kernels.c:289-294: chain j accumulates q[4s + j] * k[4s + j], s = 0..63.
      float acc[kPairs][4];
#pragma unroll
      for (int i = 0; i < kPairs; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
      // q in chunks of 2 steps (8 floats per pair), wave-uniform scalar
      // loads, two chunks in registers: chunk c + 1 is requested after
      // chunk c has arrived and before chunk c is used, so its latency
      // overlaps chunk c's arithmetic. (Scalar loads return out of order:
      // any wait for one is a wait for all, hence the explicit order.)
      constexpr int kQ = 8, kChunks = kHeadDim / kQ;
      float qa[kPairs][kQ], qb[kPairs][kQ];
      auto load_q = [&](float (&dst)[kPairs][kQ], int c) {
#pragma unroll
        for (int i = 0; i < kPairs; ++i)
#pragma unroll
          for (int e = 0; e < kQ; e += 4) {
            const float4 v = *reinterpret_cast<const float4*>(qrow[i] + kQ * c + e);
            dst[i][e] = v.x;
            dst[i][e + 1] = v.y;
            dst[i][e + 2] = v.z;
            dst[i][e + 3] = v.w;
          }
      };
      auto chunk = [&](const float (&q)[kPairs][kQ], int c) {
#pragma unroll
        for (int s = 0; s < kQ / 4; ++s) {
          const float4 k4 = *reinterpret_cast<const float4*>(krow + kQ * c + 4 * s);
#pragma unroll
          for (int i = 0; i < kPairs; ++i) {
            const float p0 = q[i][4 * s] * k4.x, p1 = q[i][4 * s + 1] * k4.y;
            const float p2 = q[i][4 * s + 2] * k4.z, p3 = q[i][4 * s + 3] * k4.w;
            acc[i][0] = acc[i][0] + p0;
            acc[i][1] = acc[i][1] + p1;
            acc[i][2] = acc[i][2] + p2;
            acc[i][3] = acc[i][3] + p3;
          }
        }
      };
      load_q(qa, 0);
      for (int c = 0; c < kChunks; c += 2) {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): chunk c (and earlier LDS reads) have arrived
        __builtin_amdgcn_sched_barrier(0);
        load_q(qb, c + 1);
        __builtin_amdgcn_sched_barrier(0);
        chunk(qa, c);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // chunk c + 1
        __builtin_amdgcn_sched_barrier(0);
        if (c + 2 < kChunks) load_q(qa, c + 2);
        __builtin_amdgcn_sched_barrier(0);
        chunk(qb, c + 1);
      }
#pragma unroll
      for (int i = 0; i < kPairs; ++i) {
        const float score = (acc[i][0] + acc[i][2]) + (acc[i][1] + acc[i][3]);
        if (in[i]) scores[sbase + ((size_t)3 * (t[i] - lo) + h[i]) * len + (key - lo)] = score;
      }
    }
  }
}

// Lanes l ^ 1, l ^ 2, l ^ 4 combined with l: the maximum over each 8-lane group.
__device__ __forceinline__ float group8_max(float v) {
#pragma unroll
  for (int m = 1; m < 8; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// LDS writes of this wave are visible to its other lanes' later reads.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ void __launch_bounds__(256)
attention_context_kernel(const float* __restrict__ qkv, const float* __restrict__ scores,
                         const uint4* __restrict__ tok, int window, int rows, int8_t* __restrict__ cq,
                         float* __restrict__ cd) {
  __shared__ uint64_t tab[32];
  __shared__ __align__(16) float pbuf[4][kHeads][64];  // per wave: a chunk's p values, per head
  __shared__ __align__(16) float sbuf[4][64][4];       // per wave: a chunk's scales, [key][head]
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (tid < 32) tab[tid] = libm::kExp2Tab.t[tid];
  __syncthreads();
  const uint32_t t = 4 * blockIdx.x + w;
  if (t >= (uint32_t)rows) return;
  const uint4 meta = tok[t];
  const uint32_t hi = min(meta.y, (uint32_t)rows), lo = min(meta.x, hi);
  if (t < lo || t >= hi) return;  // a malformed entry: nothing is written for this token
  const uint32_t len = hi - lo;
  uint32_t first, last;
  key_range(t, lo, hi, window, first, last);
  // Score rows of (t, h); key kt is at srow[h][kt - lo].
  const float* srow[kHeads];
#pragma unroll
  for (int h = 0; h < kHeads; ++h) srow[h] = scores + meta.z + ((size_t)3 * (t - lo) + h) * len;

  // The row maxima (order-free).
  float m[kHeads];
#pragma unroll
  for (int h = 0; h < kHeads; ++h) m[h] = -__builtin_inff();
  for (uint32_t kt = first + lane; kt < last; kt += 64)
#pragma unroll
    for (int h = 0; h < kHeads; ++h) m[h] = fmaxf(m[h], srow[h][kt - lo]);
#pragma unroll
  for (int h = 0; h < kHeads; ++h) m[h] = wave_max(m[h]);

  // sum = p[first] + p[first + 1] + ... in key order: each chunk's p values
  // are computed by all lanes, then lane h adds its head's in order.
  float sum = 0.0f;
  for (uint32_t c0 = first; c0 < last; c0 += 64) {
    const uint32_t kt = c0 + lane;
#pragma unroll
    for (int h = 0; h < kHeads; ++h)
      pbuf[w][h][lane] = kt < last ? libm::expf_tab(srow[h][kt - lo] - m[h], tab) : 0.0f;
    wave_lds_sync();
    if (lane < kHeads) {
      const int n = (int)min(64u, last - c0);
      const float* pr = pbuf[w][lane];
      int j = 0;
      for (; j + 4 <= n; j += 4) {
        const float4 p4 = *reinterpret_cast<const float4*>(pr + j);
        sum = sum + p4.x;
        sum = sum + p4.y;
        sum = sum + p4.z;
        sum = sum + p4.w;
      }
      for (; j < n; ++j) sum = sum + pr[j];
    }
    wave_lds_sync();
  }
  const float inv_lane = 1.0f / sum;
  float inv[kHeads];
#pragma unroll
  for (int h = 0; h < kHeads; ++h) inv[h] = __shfl(inv_lane, h, 64);

  // out = sum over kt in order of (p[kt] * inv) * v[kt]; lane l owns
  // dimensions 4l .. 4l + 3 of each head.
  float acc[kHeads][4];
#pragma unroll
  for (int h = 0; h < kHeads; ++h)
#pragma unroll
    for (int d = 0; d < 4; ++d) acc[h][d] = 0.0f;
  const float* vcol = qkv + kVOff + 4 * lane;
  for (uint32_t c0 = first; c0 < last; c0 += 64) {
    const uint32_t kt = c0 + lane;
    float sc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int h = 0; h < kHeads; ++h) {
      const float p = kt < last ? libm::expf_tab(srow[h][kt - lo] - m[h], tab) : 0.0f;
      sc[h] = p * inv[h];
    }
    *reinterpret_cast<float4*>(sbuf[w][lane]) = make_float4(sc[0], sc[1], sc[2], sc[3]);
    wave_lds_sync();
    const int n = (int)min(64u, last - c0);
    const float* vrow = vcol + (size_t)c0 * kLd;
    // The V rows of 8 keys are in flight while the previous 8 are used
    // (rows past the chunk's end repeat its last one and are not used).
    constexpr int kAhead = 8;
    float4 vq[kAhead];
#pragma unroll
    for (int j = 0; j < kAhead; ++j) vq[j] = *reinterpret_cast<const float4*>(vrow + (size_t)min(j, n - 1) * kLd);
    for (int j0 = 0; j0 < n; j0 += kAhead) {
      float4 vn[kAhead];
#pragma unroll
      for (int j = 0; j < kAhead; ++j)
        vn[j] = *reinterpret_cast<const float4*>(vrow + (size_t)min(j0 + kAhead + j, n - 1) * kLd);
#pragma unroll
      for (int j = 0; j < kAhead; ++j) {
        if (j0 + j >= n) break;  // uniform
        const float4 s4 = *reinterpret_cast<const float4*>(sbuf[w][j0 + j]);
        const float4 v4 = vq[j];
        const float s[kHeads] = {s4.x, s4.y, s4.z};
#pragma unroll
        for (int h = 0; h < kHeads; ++h) {
          const float a0 = s[h] * v4.x, a1 = s[h] * v4.y, a2 = s[h] * v4.z, a3 = s[h] * v4.w;
          acc[h][0] = acc[h][0] + a0;
          acc[h][1] = acc[h][1] + a1;
          acc[h][2] = acc[h][2] + a2;
          acc[h][3] = acc[h][3] + a3;
        }
      }
#pragma unroll
      for (int j = 0; j < kAhead; ++j) vq[j] = vn[j];
    }
    wave_lds_sync();
  }

  // Q8_0 of the context row (quants.c:97-177): block b of head h is
  // dimensions 32b .. 32b + 31, held by lanes 8b .. 8b + 7; the int8 values
  // go to the row-tile layout (24 blocks per row), the scales to cd[block][row].
#pragma unroll
  for (int h = 0; h < kHeads; ++h) {
    float amax = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) amax = fmaxf(amax, fabsf(acc[h][d]));
    amax = group8_max(amax);
    const float dq = div127(amax);
    const float id = amax != 0.0f ? 1.0f / dq : 0.0f;  // quants.c: an all-zero block stores zeros
    const int e = h * kHeadDim + 4 * lane;
    *reinterpret_cast<uint32_t*>(cq + q8_tile_offset(t, (unsigned)e, kEmbd / kQK)) =
        pack_i8x4(q8_round(acc[h][0] * id), q8_round(acc[h][1] * id), q8_round(acc[h][2] * id),
                  q8_round(acc[h][3] * id));
    if ((lane & 7) == 0) cd[(size_t)(e / kQK) * rows + t] = fp16_bits_to_fp32(fp32_to_fp16_bits(dq));
  }
}

// ---------------------------------------------------------------- host side

AttentionCounts attention_counts(const size_t* offsets, size_t batch) {
  AttentionCounts c{0, 0};
  for (size_t s = 0; s < batch; ++s) {
    const size_t len = offsets[s + 1] - offsets[s];
    c.items += (len + kKeyBlock - 1) / kKeyBlock * ((len + query_chunk(len) - 1) / query_chunk(len));
    c.score_floats += 3 * len * len;
  }
  return c;
}

bool build_attention_plan(const size_t* offsets, size_t batch, const AttentionCounts& cap, uint32_t* items,
                          uint32_t* tok, AttentionCounts* used) {
  const AttentionCounts need = attention_counts(offsets, batch);
  if (used) *used = need;
  if (need.items > cap.items || need.score_floats > cap.score_floats) return false;
  size_t n = 0, sbase = 0;
  for (size_t s = 0; s < batch; ++s) {
    const size_t lo = offsets[s], hi = offsets[s + 1], len = hi - lo, qc = query_chunk(len);
    for (size_t k0 = lo; k0 < hi; k0 += kKeyBlock)
      for (size_t q = lo; q < hi; q += qc) {
        uint32_t* it = items + 8 * n++;
        it[0] = (uint32_t)lo;
        it[1] = (uint32_t)hi;
        it[2] = (uint32_t)k0;
        it[3] = (uint32_t)q;
        it[4] = (uint32_t)std::min(hi, q + qc);
        it[5] = (uint32_t)sbase;
        it[6] = 0;
        it[7] = 0;
      }
    for (size_t t = lo; t < hi; ++t) {
      tok[4 * t] = (uint32_t)lo;
      tok[4 * t + 1] = (uint32_t)hi;
      tok[4 * t + 2] = (uint32_t)sbase;
      tok[4 * t + 3] = 0;
    }
    sbase += 3 * len * len;
  }
  return true;
}

AttentionCounts attention_capacity(size_t tokens, size_t batch) {
  // Items of a sequence of n tokens: ceil(n/64) ceil(n/qc(n)) <= (n/64 + 1)
  // (n/8 + 1) = n^2/512 + n (1/64 + 1/8) + 1; over sequences with sum n <=
  // tokens and at most `batch` of them, at most tokens^2/512 + 9 tokens/64 +
  // batch. Scores: 3 n^2 per sequence, at most 3 tokens^2.
  AttentionCounts c;
  c.items = tokens * tokens / 512 + 9 * tokens / 64 + batch + 1;
  c.score_floats = 3 * tokens * tokens;
  return c;
}

hipError_t launch_attention(const float* qkv, const uint32_t* items, const uint32_t* item_count, int grid,
                            const uint32_t* tok, int window, int rows, float* scores, int8_t* cq, float* cd,
                            hipStream_t st) {
  if (rows <= 0 || rows % 4 != 0 || grid <= 0 || window < 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_scores_kernel, dim3(grid), dim3(256), 0, st, qkv,
                     reinterpret_cast<const uint4*>(items), item_count, window, rows, scores);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(attention_context_kernel, dim3(rows / 4), dim3(256), 0, st, qkv, scores,
                     reinterpret_cast<const uint4*>(tok), window, rows, cq, cd);
  return hipGetLastError();
}

// ---------------------------------------------------------------- allocation-free form
//
// launch_attention_static keeps its plan and scores in `scratch`, a
// file-scope device array (one copy per GPU, alive until the process
// ends), and builds the plan on the device from device offsets, so a call
// allocates nothing. Layout: [item count | pad to 256 B][token records,
// 16 B x kStaticRows][work items, 32 B x kStaticItems][scores, 3 x
// kStaticRows^2 floats]. Any packing of at most kStaticRows rows into at
// most kStaticBatch sequences fits (the bounds of attention_capacity).
// Nothing in it has to start at zero: the plan kernel writes the count and
// every record the other two kernels read, and the context kernel reads
// only scores the scores kernel wrote in the same call. Calls that overlap
// on one GPU share the array and race.

constexpr size_t kStaticRows = 2048, kStaticBatch = 4096;
constexpr size_t kStaticItems = kStaticRows * kStaticRows / 512 + 9 * kStaticRows / 64 + kStaticBatch + 1;
constexpr size_t kStaticTokOff = 256;
constexpr size_t kStaticItemsOff = kStaticTokOff + 16 * kStaticRows;
constexpr size_t kStaticScoresOff = (kStaticItemsOff + 32 * kStaticItems + 255) / 256 * 256;
constexpr size_t kStaticBytes = kStaticScoresOff + sizeof(float) * 3 * kStaticRows * kStaticRows;
static_assert(kStaticItemsOff % 256 == 0, "sections stay 256-byte aligned");

static __device__ __align__(256) unsigned char scratch[kStaticBytes];

constexpr int kPlanThreads = 1024;

// Exclusive prefix (sum or max) of one value per thread over the workgroup,
// Hillis-Steele through `tmp` (kPlanThreads entries); `total` gets the
// reduction of all values.
template <bool MAX>
__device__ uint32_t plan_scan(uint32_t v, uint32_t* tmp, uint32_t& total) {
  const int tid = threadIdx.x;
  tmp[tid] = v;
  __syncthreads();
  for (int d = 1; d < kPlanThreads; d <<= 1) {
    const uint32_t o = tid >= d ? tmp[tid - d] : 0u;
    __syncthreads();
    if (tid >= d) tmp[tid] = MAX ? max(tmp[tid], o) : tmp[tid] + o;
    __syncthreads();
  }
  const uint32_t excl = MAX ? (tid > 0 ? tmp[tid - 1] : 0u) : tmp[tid] - v;
  total = tmp[kPlanThreads - 1];
  __syncthreads();  // tmp is free for the next scan
  return excl;
}

// Last index i in [0, n] with a[i] <= x for non-decreasing a with a[0] <= x.
__device__ __forceinline__ int last_le(const uint32_t* a, int n, uint32_t x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a[mid] <= x) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// The plan of build_attention_plan, on the device, in the same order. The
// offsets are read as sequence bounds with offsets[0] taken as 0,
// offsets[batch] as rows, each bound clamped to rows and raised to the one
// before it, so every row belongs to exactly one sequence and no record
// can address outside the rows or the scores section whatever the offsets
// hold. One workgroup of kPlanThreads; batch <= kStaticBatch.
__global__ void __launch_bounds__(kPlanThreads)
attention_plan_kernel(const uint32_t* __restrict__ offsets, int batch, int rows, uint32_t* __restrict__ count,
                      uint4* __restrict__ tok, uint4* __restrict__ items) {
  __shared__ uint32_t bound[kStaticBatch + 1], first_item[kStaticBatch + 1], first_score[kStaticBatch + 1];
  __shared__ uint32_t tmp[kPlanThreads];
  const int tid = threadIdx.x;
  const int nb = batch + 1, seg = (nb + kPlanThreads - 1) / kPlanThreads;
  const int b0 = min(tid * seg, nb), b1 = min(b0 + seg, nb);
  // Bounds: clamp, then the running maximum over the whole list.
  uint32_t run = 0;
  for (int i = b0; i < b1; ++i) {
    const uint32_t v = i == 0 ? 0u : (i == batch ? (uint32_t)rows : min(offsets[i], (uint32_t)rows));
    run = max(run, v);
    bound[i] = run;
  }
  uint32_t unused;
  const uint32_t before = plan_scan<true>(b1 > b0 ? run : 0u, tmp, unused);
  for (int i = b0; i < b1; ++i) bound[i] = max(bound[i], before);
  __syncthreads();
  // Items and score floats per sequence, and their exclusive prefixes.
  const int s0 = min(tid * seg, batch), s1 = min(s0 + seg, batch);
  uint32_t ni = 0, ns = 0;
  for (int s = s0; s < s1; ++s) {
    const uint32_t len = bound[s + 1] - bound[s], qc = (uint32_t)query_chunk(len);
    first_item[s] = ni;
    first_score[s] = ns;
    ni += (len + kKeyBlock - 1) / kKeyBlock * ((len + qc - 1) / qc);
    ns += 3 * len * len;
  }
  uint32_t total_items, total_scores;
  const uint32_t ibase = plan_scan<false>(ni, tmp, total_items);
  const uint32_t sbase = plan_scan<false>(ns, tmp, total_scores);
  for (int s = s0; s < s1; ++s) {
    first_item[s] += ibase;
    first_score[s] += sbase;
  }
  if (tid == 0) {
    first_item[batch] = total_items;
    first_score[batch] = total_scores;
    *count = total_items;
  }
  __syncthreads();
  for (uint32_t i = tid; i < total_items; i += kPlanThreads) {
    const int s = last_le(first_item, batch, i);  // a sequence with items has first_item[s] < first_item[s + 1]
    const uint32_t lo = bound[s], hi = bound[s + 1], len = hi - lo, qc = (uint32_t)query_chunk(len);
    const uint32_t nq = (len + qc - 1) / qc, local = i - first_item[s];
    const uint32_t k0 = lo + kKeyBlock * (local / nq), q = lo + qc * (local % nq);
    items[2 * i] = make_uint4(lo, hi, k0, q);
    items[2 * i + 1] = make_uint4(min(hi, q + qc), first_score[s], 0u, 0u);
  }
  for (uint32_t t = tid; t < (uint32_t)rows; t += kPlanThreads) {
    const int s = last_le(bound, batch, t);  // bound[s] <= t < bound[s + 1]
    tok[t] = make_uint4(bound[s], bound[s + 1], first_score[s], 0u);
  }
}

namespace {

constexpr int kMaxDevices = 64;

// The device address of `scratch` on the current device, looked up once per
// device. (The array's name in host code is not a device address.)
hipError_t static_scratch(unsigned char** out) {
  static std::mutex mu;
  static void* ptr[kMaxDevices] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    ptr[dev] = p;
  }
  *out = static_cast<unsigned char*>(ptr[dev]);
  return hipSuccess;
}

}  // namespace

hipError_t launch_attention_static(const float* qkv, const uint32_t* offsets, int batch, int window, int rows,
                                   int8_t* cq, float* cd, hipStream_t st) {
  if (rows <= 0 || rows % 4 != 0 || (size_t)rows > kStaticRows || batch <= 0 || (size_t)batch > kStaticBatch ||
      window < 0)
    return hipErrorInvalidValue;
  unsigned char* base = nullptr;
  hipError_t e = static_scratch(&base);
  if (e != hipSuccess) return e;
  uint32_t* count = reinterpret_cast<uint32_t*>(base);
  uint32_t* tok = reinterpret_cast<uint32_t*>(base + kStaticTokOff);
  uint32_t* items = reinterpret_cast<uint32_t*>(base + kStaticItemsOff);
  float* scores = reinterpret_cast<float*>(base + kStaticScoresOff);
  hipLaunchKernelGGL(attention_plan_kernel, dim3(1), dim3(kPlanThreads), 0, st, offsets, batch, rows, count,
                     reinterpret_cast<uint4*>(tok), reinterpret_cast<uint4*>(items));
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_attention(qkv, items, count, kAttentionScoreGrid, tok, window, rows, scores, cq, cd, st);
}

}  // namespace eg2
