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
// reproduce the order exactly.
//
// Products on the matrix cores. An fp32 MFMA with a zero accumulator and
// one product per output (v_mfma_f32_16x16x1_4b_f32) returns each product
// rounded once, exactly as the VALU multiply does (checked on 12 million
// random pairs including subnormal results); the ordered additions stay on
// the VALU. That halves the VALU work of both products (q.k and p.v).
//
// Operands: the rows [q0 q1 q2 | k | v] (1280 fp32) that QK-norm/RoPE
// leaves, one per token (q already scaled by 1/16). A (token t, head h)
// pair of a sequence starting at lo is numbered 3 (t - lo) + h.
//
// The kernels:
//  - attention_scores_kernel: work items of (sequence, 32 pairs, 32 keys),
//    listed pair block by pair block (an XCD's contiguous share of a long
//    sequence then needs a band of q rows and the k rows, which fit its L2).
//    The workgroup stages the q rows of its pairs and the k rows of its
//    keys in LDS by 16-byte DMA (no registers), 32 dimensions at a time,
//    laid out [16-row block][4-dimension chunk][row] so that the lane of
//    chain c and row r reads chunk s's element c with a 4-byte read and
//    the wave's 64 lanes hit 64 distinct banks. Each wave owns 16 pairs x
//    16 keys; per 4 dimensions one 4-block MFMA whose block c multiplies
//    chain c (lane group c feeds chain c's q and k values), and each lane
//    adds its 16 products to its 4 pairs' 4 chain sums. The scores go to a
//    scratch row per pair (row length rounded up to 4). A workgroup takes
//    items in turn (the workgroups of an XCD, a contiguous eighth of the
//    list) and stages the next stage of 32 dimensions (the next item's
//    first during the current item's last) while the current one computes.
//  - the softmax, one kernel in one of four forms picked by the wave's
//    longest sequence (the same operations in the same order in each):
//    each (token, head) pair's row maximum, p = expf(score - m) written
//    back over the scores, then the sum of the p row in key order (a serial
//    chain: one lane per pair, the workgroup's pairs sharing each add
//    instruction) and 1/sum into the scratch's head. Up to 512 keys the
//    workgroup's 16 pairs keep their p rows in LDS for the sums, with 16 or
//    32 lanes per pair up to 128 or 256 keys (attention_softmax_group_kernel)
//    and a wave per pair beyond (attention_softmax_kernel); longer rows
//    stream through a two-chunk LDS ring of 256 keys per pair, the first
//    wave adding chunk c while the workgroup computes chunk c + 1
//    (attention_softmax_ring_kernel, any length: every workgroup of a
//    2048-token wave is resident at once).
//  - attention_context_kernel: work items of (sequence, 32 pairs), each
//    taken by 4 workgroups of 64 dimensions (768 workgroups for a wave of
//    16 x 128 tokens or for one 2048-token sequence). Per 64-key chunk the
//    workgroup stages w = p * (1/sum) for its pairs through registers (0
//    for keys outside a pair's window, which adds +0 and changes no sum; a
//    chunk inside every pair's window, the usual case, skips those bounds)
//    and the chunk's v rows by LDS DMA into one of two buffers, the next
//    chunk's while the current one is computed (128 VGPRs and 40 KB of LDS:
//    four workgroups per CU); per 2 keys each
//    wave issues one 4-block MFMA (block b = pairs 16 (b % 2) .. + 15 of key
//    b / 2, columns = its 16 dimensions) and adds the products to its 8
//    accumulators, in key order. The Q8_0 epilogue quantizes 32-value
//    blocks over 4 lanes.
// A sequence's keys, scores and context depend only on its own tokens, so
// packing never changes a bit.
#include <algorithm>
#include <mutex>
#include <vector>

#include "eg2_device.hpp"
#include "eg2_kernels.hpp"
#include "eg2_libm.hpp"

namespace eg2 {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kLd = kQKVCols;  // floats per operand row [q0 q1 q2 | k | v]
constexpr int kKOff = kHeads * kHeadDim, kVOff = kKOff + kHeadDim;

constexpr int kSKeys = 32, kSPairs = 32;  // scores workgroup tile
constexpr int kCPairs = 32, kCDims = 64;  // context workgroup tile
constexpr int kCKeys = 64;                // keys per staged chunk (a multiple of 32)
constexpr int kCWKeys = kCKeys / 8;       // keys per thread in the w staging (8 threads per pair)
static_assert(kCKeys % 32 == 0, "whole float4s per staging thread, whole DMA instructions per wave");
constexpr int kCPitchV = kCDims + 4;       // floats per row of the context's epilogue tile
constexpr int kShortSoftmax = kSoftmaxWave;  // longest row of the softmax forms that keep p rows in LDS
constexpr int kCBatch = 4;                // context MFMAs in flight per wave
constexpr uint32_t kXcdCount = 8;         // MI355X: 8 XCDs, workgroup b on XCD b % 8

// Work items of any packing of `tokens` rows into at most `batch`
// sequences: per sequence of n tokens, ceil(n/32) ceil(3n/32) <= 3n^2/1024
// + n/8 + 1 score items (32 x 32 tiles) and ceil(3n/kCPairs) <= 3n/kCPairs
// + 1 context items; summed over sequences with sum n <= tokens.
constexpr size_t item_bound(size_t tokens, size_t batch) {
  static_assert(kSKeys == 32 && kSPairs == 32, "the score-item bound assumes 32 x 32 tiles");
  return 3 * tokens * tokens / 1024 + tokens / 8 + 3 * tokens / kCPairs + 2 * batch + 2;
}

// Floats of a sequence's score row (its length rounded up to 4, so that
// rows are 16-byte aligned), and of the 1/sum area at the scratch's head.
__host__ __device__ inline uint32_t score_pitch(uint32_t len) { return (len + 3u) & ~3u; }
__host__ __device__ inline size_t inv_floats(size_t rows) { return (3 * rows + 3) & ~(size_t)3; }

// Key range of query token t in its sequence [lo, hi) (kernels.c:330-336
// in packed coordinates): the sequence, or |t - kt| <= window/2.
__host__ __device__ inline void key_range(uint32_t t, uint32_t lo, uint32_t hi, int window, uint32_t& first,
                                          uint32_t& last) {
  const uint32_t half = window > 0 ? (uint32_t)(window / 2) : 0u;
  first = window > 0 && t - lo > half ? t - half : lo;
  last = window > 0 && t + half + 1 < hi ? t + half + 1 : hi;
}

// ----------------------------------------------------------------- scores

// The scores' staging: per item, eight stages of 32 dimensions, each a
// plain copy by 16-byte LDS DMA into blocks of 16 rows (block 0, 1: the q
// rows of pairs pair0 .. + 15, + 16 .. + 31; block 2, 3: the k rows of keys
// key0 .. + 15, + 16 .. + 31), laid out [block][chunk][row] with a chunk =
// 4 dimensions (all four chains at one step). A lane of chain g and row
// r16 reads its step-s value with one 4-byte read at chunk s, row r16,
// element g: the wave's 64 lanes touch 64 distinct banks. Two buffers of
// 8 KB: at 16 KB per workgroup the kernel leaves room on a CU for the
// other lanes' kernels (with 64-dimension stages, 32 KB, it ran 1-7%
// slower at 16-512 keys and the 16 x 128 forward 0.8% slower).
constexpr int kSQDims = 32;
constexpr int kSQChunks = kSQDims / 4;
constexpr int kSBlockFloats = kSQChunks * 16 * 4;  // one block of 16 rows

// One stage of the wave's 16 pairs x 16 keys: per kSBatch steps
// that many MFMAs into separate registers, then their adds, with the next
// steps' operands read from LDS before the adds.
constexpr int kSBatch = 2;
__device__ __forceinline__ void scores_stage(const float* qa, const float* kb, float (&acc)[4][4]) {
  const floatx16 zero = {};
  float qv[kSBatch], kv[kSBatch];
#pragma unroll
  for (int e = 0; e < kSBatch; ++e) {
    qv[e] = qa[64 * e];
    kv[e] = kb[64 * e];
  }
#pragma unroll
  for (int s = 0; s < kSQChunks; s += kSBatch) {
    floatx16 prod[kSBatch];
#pragma unroll
    for (int e = 0; e < kSBatch; ++e)  // block c: chain c; rows = pairs, columns = keys
      prod[e] = __builtin_amdgcn_mfma_f32_16x16x1f32(qv[e], kv[e], zero, 0, 0, 0);
    if (s + kSBatch < kSQChunks) {
#pragma unroll
      for (int e = 0; e < kSBatch; ++e) {
        qv[e] = qa[64 * (s + kSBatch + e)];
        kv[e] = kb[64 * (s + kSBatch + e)];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int e = 0; e < kSBatch; ++e)
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[c][r] = acc[c][r] + prod[e][4 * c + r];
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The wave's 16 x 16 scores ((chain 0 + chain 2) + (chain 1 + chain 3),
// kernels.c:35-39) for the (pair, key)s inside the pair's window. Stored
// through a buffer resource over the sequence's score rows (a scalar base
// and a 32-bit offset per lane) when they span less than 4 GiB, which every
// sequence of up to 18,900 tokens does.
__device__ __forceinline__ void store_scores(const float (&acc)[4][4], uint32_t lo, uint32_t hi, uint32_t key0,
                                             uint32_t pair0, uint32_t pair1, size_t sbase, int window, int pr,
                                             int kr, int g, int r16, float* __restrict__ scores) {
  const uint32_t len = hi - lo, pitch = score_pitch(len);
  const uint32_t key = key0 + kr + r16;
  const bool small = (uint64_t)3 * len * pitch * 4 < 0x100000000ull;  // uniform
  const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(scores + sbase, 0xffffffffu);
  const uint32_t p0 = pair0 + pr + 4 * g, off0 = p0 * pitch + (key - lo);  // pair p0 + r at off0 + r pitch
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint32_t pair = p0 + r;
    const float score = (acc[0][r] + acc[2][r]) + (acc[1][r] + acc[3][r]);
    bool in = pair < pair1 && key < hi;
    if (window > 0) {  // uniform
      uint32_t first, last;
      key_range(lo + pair / 3, lo, hi, window, first, last);
      in = in && key >= first && key < last;
    }
    if (!in) continue;
    if (small)
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, score), rs, 4u * (off0 + r * pitch), 0, 0);
    else
      scores[sbase + (size_t)pair * pitch + (key - lo)] = score;
  }
}

// A score item's tile, its fields clamped to the wave (so a malformed list
// cannot address outside the rows); valid is 0 for an empty or malformed
// item and for a tile with no (pair, key) inside the window.
struct ScoreTile {  // all 32-bit fields: no padding bytes for a copy to carry
  uint32_t lo, hi, key0, pair0, pair1, sbase, valid;
};
__device__ __forceinline__ ScoreTile score_tile(const uint4* __restrict__ items, uint32_t item, int window,
                                                int rows) {
  const uint4 a = items[2 * item], b = items[2 * item + 1];
  ScoreTile t;
  t.hi = min(a.y, (uint32_t)rows);
  t.lo = min(a.x, t.hi);
  const uint32_t len = t.hi - t.lo;
  t.key0 = a.z;
  t.pair1 = min(b.x, 3 * len);
  t.pair0 = a.w;
  t.sbase = b.y;
  t.valid = len != 0 && t.key0 >= t.lo && t.key0 < t.hi && t.pair0 < t.pair1 ? 1u : 0u;
  if (t.valid && window > 0) {
    const int half = window / 2;
    const int tmin = (int)(t.lo + t.pair0 / 3), tmax = (int)(t.lo + (t.pair1 - 1) / 3);
    const int kmin = (int)t.key0, kmax = (int)min(t.key0 + kSKeys, t.hi) - 1;
    t.valid = kmax < tmin - half || kmin > tmax + half ? 0u : 1u;
  }
  return t;
}

// Float offset of staging row r of tile t from the sequence's first row
// (r < 32: the q row of pair pair0 + r, else the k row of key key0 + r -
// 32), clamped (the rows past the tile's end are computed and not stored).
// Relative to the sequence, so that the DMA's 32-bit byte offsets hold for
// any row count (a planned sequence is below 37,838 rows: 194 MB of qkv).
__device__ __forceinline__ uint32_t stage_row(const ScoreTile& t, uint32_t r) {
  if (r < (uint32_t)kSPairs) {
    const uint32_t spair = min(t.pair0 + r, t.pair1 - 1);
    return spair / 3 * kLd + (spair % 3) * kHeadDim;
  }
  return (min(t.key0 + r - kSPairs, t.hi - 1) - t.lo) * kLd + kKOff;
}

// The first item from `item` on (stride `stride`) below `count` that has
// work, its tile in t; count when none is left. Uniform over the workgroup.
__device__ __forceinline__ uint32_t next_score_item(const uint4* __restrict__ items, uint32_t item, uint32_t count,
                                                    uint32_t stride, int window, int rows, ScoreTile& t) {
  for (; item < count; item += stride) {
    t = score_tile(items, item, window, rows);
    if (t.valid) break;
  }
  return item;
}

// The workgroup takes items in turn (grid-stride); each stage's rows are
// staged by DMA into one of two LDS buffers while the previous stage
// computes (the next item's first stage during the current item's last).
__global__ void __launch_bounds__(256)
attention_scores_kernel(const float* __restrict__ qkv, const uint4* __restrict__ items,
                                 const uint32_t* __restrict__ item_count, int window, int rows,
                                 float* __restrict__ scores) {
  __shared__ __align__(16) float stg[2][4 * kSBlockFloats];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r16 = lane & 15;
  const int pr = 16 * (w >> 1), kr = 16 * (w & 1);
  // XCD-aware order (a grid that is a multiple of 8): workgroup b runs on
  // XCD b % 8, which takes the contiguous eighth of the item list, so an
  // XCD's L2 holds the rows of few sequences; any other grid strides over
  // the whole list.
  const bool by_xcd = gridDim.x % kXcdCount == 0;
  const uint32_t total = item_count[0], xcd = blockIdx.x % kXcdCount;
  const uint32_t count = by_xcd ? total * (xcd + 1) / kXcdCount : total;
  const uint32_t stride = by_xcd ? gridDim.x / kXcdCount : gridDim.x;
  const unsigned stg0 = (unsigned)(uintptr_t)&stg[0][0];
  // Wave w stages block w: per instruction 4 chunks of its 16 rows, lane L
  // row L % 16, chunk 4 j + L / 16, i.e. LDS position 64 j + L of the block.
  const float* seq = qkv;
  uint32_t roff = 0;  // the lane's row, in bytes from the sequence's first row
  auto locate = [&](const ScoreTile& t) {
    seq = qkv + (size_t)t.lo * kLd;
    roff = 4 * stage_row(t, 16 * (uint32_t)w + (uint32_t)r16) + 16 * (uint32_t)g;
  };
  auto issue = [&](int q, int buf) {
#pragma unroll
    for (int j = 0; j < kSQChunks / 4; ++j)
      dma16(seq, roff + 4 * (uint32_t)(kSQDims * q + 16 * j),
            stg0 + (unsigned)((buf * 4 + w) * kSBlockFloats + 256 * j) * 4u);
  };
  ScoreTile t;
  uint32_t item = next_score_item(items, by_xcd ? total * xcd / kXcdCount + blockIdx.x / kXcdCount : blockIdx.x,
                                  count, stride, window, rows, t);
  if (item < count) {
    locate(t);
    issue(0, 0);
  }
  int buf = 0;
  while (item < count) {
    float acc[4][4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[c][r] = 0.0f;
    ScoreTile nt = t;
    uint32_t nitem = count;
#pragma unroll 1
    for (int q = 0; q < kHeadDim / kSQDims; ++q) {
      // This wave's DMA of the stage has landed; after the barrier every
      // wave's has, and the other buffer is no longer read.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (q + 1 < kHeadDim / kSQDims) {
        issue(q + 1, buf ^ 1);
      } else {
        nitem = next_score_item(items, item + stride, count, stride, window, rows, nt);
        if (nitem < count) {
          locate(nt);
          issue(0, buf ^ 1);
        }
      }
      const float* base = stg[buf] + 4 * r16 + g;  // chunk s of row r16 at 64 s + 4 r16
      scores_stage(base + (w >> 1) * kSBlockFloats, base + (2 + (w & 1)) * kSBlockFloats, acc);
      buf ^= 1;
    }
    store_scores(acc, t.lo, t.hi, t.key0, t.pair0, t.pair1, t.sbase, window, pr, kr, g, r16, scores);
    item = nitem;
    t = nt;
  }
}

// ---------------------------------------------------------------- softmax

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// The softmax of waves of sequences up to kShortSoftmax tokens: one wave per
// (token, head) pair, 16 pairs per workgroup. Each wave takes the row
// maximum, then every lane's p = expf(score - m) for its keys, written back
// over the scores and into the pair's LDS row; then lane i of the first
// wave adds pair i's p values in key order (a serial chain: the
// workgroup's pairs share each add instruction) and writes 1/sum into the
// scratch's head. A longer row (a packing longer than the caller's
// `longest`) is summed from the scores in global memory instead: slower,
// same bits.
constexpr int kWavePairs = 16;

__global__ void __launch_bounds__(64 * kWavePairs)
attention_softmax_kernel(float* __restrict__ scores, const uint4* __restrict__ tok, int window, int rows) {
  __shared__ uint64_t tab[32];
  __builtin_amdgcn_s_setprio(3);  // latency-bound (max, exp, serial sums): issued first on its SIMDs
  __shared__ __align__(16) float prow[kWavePairs][kShortSoftmax + 4];  // each pair's p values (4 banks apart)
  __shared__ uint32_t plen[kWavePairs];                                // and their count (0: no such pair)
  __shared__ uint32_t pbase[kWavePairs];                               // index in scores of the row's first key
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (tid < 32) tab[tid] = libm::kExp2Tab.t[tid];
  __syncthreads();
  // XCD-aware order (a grid that is a multiple of 8): XCD b % 8 takes the
  // contiguous eighth of the pair blocks, the pairs whose scores its L2
  // holds from the scores kernel.
  const uint32_t blk = gridDim.x % kXcdCount == 0
                           ? (blockIdx.x % kXcdCount) * (gridDim.x / kXcdCount) + blockIdx.x / kXcdCount
                           : blockIdx.x;
  const uint32_t pair = kWavePairs * blk + w, t = pair / 3, h = pair % 3;
  uint32_t n = 0, base = 0;
  if (t < (uint32_t)rows) {
    const uint4 meta = tok[t];
    const uint32_t hi = min(meta.y, (uint32_t)rows), lo = min(meta.x, hi);
    if (t >= lo && t < hi) {  // else a malformed entry: nothing is written for this token
      uint32_t first, last;
      key_range(t, lo, hi, window, first, last);
      float* srow = scores + meta.z + ((size_t)3 * (t - lo) + h) * score_pitch(hi - lo);  // key kt at srow[kt - lo]
      n = last - first;
      base = meta.z + (3 * (t - lo) + h) * score_pitch(hi - lo) + (first - lo);
      // The maximum, then the exps, each a pass over the row (the second
      // from the L2).
      float m = -__builtin_inff();
      uint32_t kt = first + lane;
      for (; kt + 192 < last; kt += 256) {
        const float a = srow[kt - lo], b = srow[kt - lo + 64], c = srow[kt - lo + 128], d = srow[kt - lo + 192];
        m = fmaxf(m, fmaxf(fmaxf(a, b), fmaxf(c, d)));
      }
      for (; kt < last; kt += 64) m = fmaxf(m, srow[kt - lo]);
      m = wave_max(m);
      const bool to_lds = n <= (uint32_t)kShortSoftmax;
      for (uint32_t k = first + lane; k < last; k += 64) {
        const float p = libm::expf_tab(srow[k - lo] - m, tab);
        srow[k - lo] = p;
        if (to_lds) prow[w][k - first] = p;
      }
    }
  }
  if (lane == 0) {
    plen[w] = n;
    pbase[w] = base;
  }
  __syncthreads();
  if (w == 0 && lane < kWavePairs) {
    const uint32_t cnt = plen[lane];
    const uint32_t own = kWavePairs * blk + lane;
    if (cnt > 0) {
      float sum = 0.0f;
      if (cnt <= (uint32_t)kShortSoftmax) {
        // One 16-byte read at a time (22 VGPRs: the kernel shares its CUs
        // with other lanes' work).
        const float* pr = prow[lane];
        uint32_t j = 0;
#pragma unroll 2
        for (; j + 4 <= cnt; j += 4) {
          const float4 p4 = *reinterpret_cast<const float4*>(pr + j);
          sum = sum + p4.x;
          sum = sum + p4.y;
          sum = sum + p4.z;
          sum = sum + p4.w;
        }
        for (; j < cnt; ++j) sum = sum + pr[j];
      } else {
        const float* pr = scores + pbase[lane];
#pragma unroll 1
        for (uint32_t j = 0; j < cnt; ++j) sum = sum + pr[j];
      }
      scores[own] = 1.0f / sum;
    }
  }
}

// The softmax for waves of short sequences: LANES (16 or 32) lanes per
// (token, head) pair, 64 / LANES pairs per wave, 16 pairs per workgroup, so
// several pairs share each instruction of the per-pair set-up and of the
// maximum's combination. Lane j of a pair's LANES takes keys
// first + j + LANES i, held in registers: the row maximum (order-free;
// combined over the pair's lanes by DPP), then p = expf(score - m) written
// back over the scores and into the pair's LDS row (as long as the form's
// bound, kSoftmaxLanes16 or kSoftmaxLanes32 keys: 8 or 17 KB per workgroup,
// which leaves room on a CU for other lanes' kernels; +0 past the row);
// then lane i of the first wave adds pair i's p values in key order, 16 at
// a time from two register sets, and writes 1/sum into the scratch's head. A longer
// row (a packing longer than the caller's `longest`) is summed from the
// scores in global memory instead: slower, same bits. The same
// operations in the same order as attention_softmax_kernel, which takes
// waves of longer sequences (fewer pairs per wave hide more latency there).
constexpr int kGroupPairs = 16;  // pairs per workgroup

template <int CTRL>
__device__ __forceinline__ float dpp_move(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}
// Maximum over each aligned group of LANES lanes, on every lane of it (all
// 64 lanes active): quad permutations, the other quad of each 8 lanes
// (row_half_mirror), the other 8 of each 16 (row_mirror), then for 32 the
// other 16 (a swizzle).
template <int LANES>
__device__ __forceinline__ float group_max(float m) {
  static_assert(LANES == 16 || LANES == 32, "16 or 32 lanes per pair");
  m = fmaxf(m, dpp_move<0xB1>(m));   // quad_perm [1,0,3,2]
  m = fmaxf(m, dpp_move<0x4E>(m));   // quad_perm [2,3,0,1]
  m = fmaxf(m, dpp_move<0x141>(m));  // row_half_mirror
  m = fmaxf(m, dpp_move<0x140>(m));  // row_mirror
  if constexpr (LANES == 32) m = fmaxf(m, __shfl_xor(m, 16, 64));
  return m;
}

template <int LANES>
__global__ void __launch_bounds__(LANES * kGroupPairs)
attention_softmax_group_kernel(float* __restrict__ scores, const uint4* __restrict__ tok, int window, int rows) {
  __shared__ uint64_t tab[32];
  constexpr int kRow = LANES == 16 ? kSoftmaxLanes16 : kSoftmaxLanes32;  // the form's longest row
  __shared__ __align__(16) float prow[kGroupPairs][kRow + 4];  // each pair's p values (4 banks apart)
  __shared__ uint32_t plen[kGroupPairs];                                // and their count (0: no such pair)
  __shared__ uint32_t pbase[kGroupPairs];                               // index in scores of the row's first key
  __builtin_amdgcn_s_setprio(3);  // latency-bound (max, exp, serial sums): issued first on its SIMDs
  const int tid = threadIdx.x, slot = tid / LANES, sub = tid % LANES;
  // XCD-aware order, as in attention_softmax_kernel.
  const uint32_t blk = gridDim.x % kXcdCount == 0
                           ? (blockIdx.x % kXcdCount) * (gridDim.x / kXcdCount) + blockIdx.x / kXcdCount
                           : blockIdx.x;
  const uint32_t pair = kGroupPairs * blk + slot, t = pair / 3, h = pair % 3;
  uint32_t n = 0, base = 0;
  if (t < (uint32_t)rows) {
    const uint4 meta = tok[t];
    const uint32_t hi = min(meta.y, (uint32_t)rows), lo = min(meta.x, hi);
    if (t >= lo && t < hi) {  // else a malformed entry: nothing is written for this token
      uint32_t first, last;
      key_range(t, lo, hi, window, first, last);
      n = last - first;
      base = meta.z + (3 * (t - lo) + h) * score_pitch(hi - lo) + (first - lo);
    }
  }
  float* row = scores + base;  // key first + j at row[j]
  float* lrow = prow[slot];
  const bool to_lds = n <= (uint32_t)kRow;
  // A row of at most kRow keys is read once into registers (kPer keys per
  // lane), its maximum taken and its p computed from them; a longer one (a
  // packing longer than the caller's `longest`) is read twice from global
  // memory. The exp table is staged while the first reads are in flight.
  constexpr int kPer = kRow / LANES;
  float v[kPer];
  float m = -__builtin_inff();
  if (to_lds) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint32_t j = sub + LANES * i;
      v[i] = j < n ? row[j] : -__builtin_inff();
      m = fmaxf(m, v[i]);
    }
  } else {
    uint32_t j = sub;
    for (; j + 3 * LANES < n; j += 4 * LANES) {
      const float a = row[j], b = row[j + LANES], c = row[j + 2 * LANES], d = row[j + 3 * LANES];
      m = fmaxf(m, fmaxf(fmaxf(a, b), fmaxf(c, d)));
    }
    for (; j < n; j += LANES) m = fmaxf(m, row[j]);
  }
  if (tid < 32) tab[tid] = libm::kExp2Tab.t[tid];
  m = group_max<LANES>(m);
  __syncthreads();  // tab
  if (to_lds) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint32_t j = sub + LANES * i;
      const float p = libm::expf_tab(v[i] - m, tab);  // computed for every slot: no branch per key
      if (j < n) row[j] = p;
      lrow[j] = j < n ? p : 0.0f;  // +0 past the row: the sum below adds whole batches
    }
  } else {
    for (uint32_t j = sub; j < n; j += LANES) row[j] = libm::expf_tab(row[j] - m, tab);
  }
  if (sub == 0) {
    plen[slot] = n;
    pbase[slot] = base;
  }
  __syncthreads();
  if (tid < kGroupPairs) {
    const uint32_t cnt = plen[tid];
    const uint32_t own = kGroupPairs * blk + tid;
    if (cnt > 0) {
      float sum = 0.0f;
      if (cnt <= (uint32_t)kRow) {
        // Whole batches of 16 keys (the row's LDS slots past cnt hold +0,
        // and adding +0 to a sum of non-negative values changes no bit),
        // from two register sets: a set is reloaded right after it is
        // added, so its reads are in flight during the other set's adds.
        const float4* p4 = reinterpret_cast<const float4*>(prow[tid]);
        constexpr uint32_t kB = 4, kSets = kRow / (4 * kB);
        const uint32_t nb = (cnt + 4 * kB - 1) / (4 * kB);
        float4 a[kB], b[kB];
        auto fill = [&](float4 (&x)[kB], uint32_t batch) {
#pragma unroll
          for (uint32_t i = 0; i < kB; ++i) x[i] = p4[kB * min(batch, kSets - 1) + i];
        };
        auto add = [&](const float4 (&x)[kB]) {
#pragma unroll
          for (uint32_t i = 0; i < kB; ++i) {
            sum = sum + x[i].x;
            sum = sum + x[i].y;
            sum = sum + x[i].z;
            sum = sum + x[i].w;
          }
        };
        fill(a, 0);
        fill(b, 1);
        for (uint32_t bt = 0; bt < nb; bt += 2) {
          add(a);
          __builtin_amdgcn_sched_barrier(0);
          fill(a, bt + 2);
          __builtin_amdgcn_sched_barrier(0);
          if (bt + 1 < nb) add(b);
          __builtin_amdgcn_sched_barrier(0);
          fill(b, bt + 3);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
        const float* pr = scores + pbase[tid];
#pragma unroll 1
        for (uint32_t k = 0; k < cnt; ++k) sum = sum + pr[k];
      }
      scores[own] = 1.0f / sum;
    }
  }
}

// The softmax of rows of any length, streamed through LDS: one wave per
// (token, head) pair, kRingPairs pairs per workgroup. Each wave takes its
// row's maximum, then p = expf(score - m) a chunk of kRingKeys keys at a
// time, written back over the scores and into the pair's slot of a
// two-chunk LDS ring; lane i of the first wave adds pair i's p values in
// key order from the ring, chunk c while the waves compute chunk c + 1 (a
// barrier per chunk). The ring is 17 KB per workgroup where whole rows of
// 2048 keys take 66 KB, so every pair of a 2048-token wave has its
// workgroup resident at once and the serial sums run in one round. The same
// operations in the same order as attention_softmax_kernel.
constexpr int kRingPairs = 8;
constexpr int kRingKeys = 256;

// Six waves per SIMD (at most 80 VGPRs): three workgroups per CU, every
// pair of a 2048-token wave resident at once.
__global__ void __launch_bounds__(64 * kRingPairs, 6)
attention_softmax_ring_kernel(float* __restrict__ scores, const uint4* __restrict__ tok, int window, int rows) {
  __shared__ uint64_t tab[32];
  __shared__ __align__(16) float ring[2][kRingPairs][kRingKeys + 4];  // pairs' chunks, 4 banks apart
  __shared__ uint32_t plen[kRingPairs];                                // keys per pair (0: no such pair)
  __builtin_amdgcn_s_setprio(3);  // latency-bound (max, exp, serial sums): issued first on its SIMDs
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (tid < 32) tab[tid] = libm::kExp2Tab.t[tid];
  // XCD-aware order, as in attention_softmax_kernel.
  const uint32_t blk = gridDim.x % kXcdCount == 0
                           ? (blockIdx.x % kXcdCount) * (gridDim.x / kXcdCount) + blockIdx.x / kXcdCount
                           : blockIdx.x;
  const uint32_t pair = kRingPairs * blk + w, t = pair / 3, h = pair % 3;
  uint32_t n = 0, base = 0;
  if (t < (uint32_t)rows) {
    const uint4 meta = tok[t];
    const uint32_t hi = min(meta.y, (uint32_t)rows), lo = min(meta.x, hi);
    if (t >= lo && t < hi) {  // else a malformed entry: nothing is written for this token
      uint32_t first, last;
      key_range(t, lo, hi, window, first, last);
      n = last - first;
      base = meta.z + (3 * (t - lo) + h) * score_pitch(hi - lo) + (first - lo);
    }
  }
  if (lane == 0) plen[w] = n;
  __syncthreads();
  uint32_t chunks = 0;  // the workgroup's chunk count: its longest row's
#pragma unroll
  for (int i = 0; i < kRingPairs; ++i) chunks = max(chunks, (plen[i] + kRingKeys - 1) / kRingKeys);
  float* row = scores + base;  // key first + k at row[k]
  float m = -__builtin_inff();
  uint32_t k = lane;
  for (; k + 192 < n; k += 256) {
    const float a = row[k], b = row[k + 64], c = row[k + 128], d = row[k + 192];
    m = fmaxf(m, fmaxf(fmaxf(a, b), fmaxf(c, d)));
  }
  for (; k < n; k += 64) m = fmaxf(m, row[k]);
  m = wave_max(m);
  // Chunk c of this wave's row: lane l takes keys kRingKeys c + l + 64 j.
  constexpr int kPer = kRingKeys / 64;
  float s[kPer];
  auto load = [&](uint32_t c) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const uint32_t kk = kRingKeys * c + (uint32_t)lane + 64 * j;
      s[j] = kk < n ? row[kk] : 0.0f;
    }
  };
  auto put = [&](uint32_t c) {
    float* slot = ring[c & 1][w];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const uint32_t kk = kRingKeys * c + (uint32_t)lane + 64 * j;
      const float p = libm::expf_tab(s[j] - m, tab);  // computed for every slot: no branch per key
      if (kk < n) {
        row[kk] = p;
        slot[lane + 64 * j] = p;
      }
    }
  };
  if (chunks > 0) {
    load(0);
    put(0);
  }
  __syncthreads();
  const bool adder = w == 0 && lane < kRingPairs;
  const uint32_t cnt = adder ? plen[lane] : 0;
  float sum = 0.0f;
  for (uint32_t c = 0; c < chunks; ++c) {
    if (c + 1 < chunks) load(c + 1);
    if (adder && kRingKeys * c < cnt) {
      const float* pr = ring[c & 1][lane];
      const uint32_t m4 = min((uint32_t)kRingKeys, cnt - kRingKeys * c);
      uint32_t j = 0;
      // Batches of 32 keys in two register sets: a set is reloaded right
      // after it is added and added again only after the other set's 32
      // adds, which cover the read's latency (reads past the chunk's end
      // stay inside the slot and are not added).
      const float4* p4 = reinterpret_cast<const float4*>(pr);
      constexpr uint32_t kB = 8, kSets = kRingKeys / (4 * kB);
      const uint32_t nb = m4 / (4 * kB);
      float4 a[kB], b[kB];
      auto fill = [&](float4 (&x)[kB], uint32_t batch) {
#pragma unroll
        for (uint32_t i = 0; i < kB; ++i) x[i] = p4[kB * min(batch, kSets - 1) + i];
      };
      auto add = [&](const float4 (&x)[kB]) {
#pragma unroll
        for (uint32_t i = 0; i < kB; ++i) {
          sum = sum + x[i].x;
          sum = sum + x[i].y;
          sum = sum + x[i].z;
          sum = sum + x[i].w;
        }
      };
      if (nb > 0) {
        fill(a, 0);
        fill(b, 1);
        for (uint32_t bt = 0; bt + 2 <= nb; bt += 2) {
          add(a);
          __builtin_amdgcn_sched_barrier(0);
          fill(a, bt + 2);
          __builtin_amdgcn_sched_barrier(0);
          add(b);
          __builtin_amdgcn_sched_barrier(0);
          fill(b, bt + 3);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (nb & 1) add(a);
        j = 4 * kB * nb;
      }
      for (; j < m4; ++j) sum = sum + pr[j];
    }
    if (c + 1 < chunks) put(c + 1);
    __syncthreads();
  }
  if (adder && cnt > 0) scores[kRingPairs * blk + (uint32_t)lane] = 1.0f / sum;
}

// ---------------------------------------------------------------- context

__global__ void __launch_bounds__(256)
attention_context_kernel(const float* __restrict__ qkv, const float* __restrict__ scores,
                         const uint4* __restrict__ items, const uint32_t* __restrict__ item_count, int window,
                         int rows, int8_t* __restrict__ cq, float* __restrict__ cd) {
  __shared__ __align__(16) float wl[kCKeys * kCPairs];      // [key][pair]: w = p * (1/sum), 0 outside the window
  __shared__ __align__(16) float vl[2][kCKeys * kCDims];    // [key][dimension], two chunks, filled by DMA
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r16 = lane & 15;
  const uint4* citems = items + 2 * (size_t)item_count[0];  // the context items follow the score items
  // XCD-aware order as in the scores kernel when the plan asks for it (the
  // first context item's it[5]: a packing whose contiguous eighths of
  // units cost alike): XCD b % 8 takes the contiguous eighth of the work
  // (items x 4 dimension quarters). Otherwise the plain stride, which
  // spreads every sequence's units over the XCDs.
  const uint32_t total = 4 * item_count[1], xcd = blockIdx.x % kXcdCount;
  const bool by_xcd = total > 0 && citems[1].y == 1u && gridDim.x % kXcdCount == 0;
  const uint32_t count = by_xcd ? total * (xcd + 1) / kXcdCount : total;
  const uint32_t stride = by_xcd ? gridDim.x / kXcdCount : gridDim.x;
  const unsigned vl0 = (unsigned)(uintptr_t)&vl[0][0];  // LDS byte address of the v chunks
  const floatx16 zero = {};
  for (uint32_t work = by_xcd ? total * xcd / kXcdCount + blockIdx.x / kXcdCount : blockIdx.x; work < count;
       work += stride) {
    const uint4 a = citems[2 * (work >> 2)], b = citems[2 * (work >> 2) + 1];
    const uint32_t hi = min(a.y, (uint32_t)rows), lo = min(a.x, hi), len = hi - lo;
    const uint32_t pair1 = min(a.w, 3 * len), pair0 = a.z;
    if (len == 0 || pair0 >= pair1) continue;  // uniform
    const size_t sbase = b.x;
    const uint32_t pitch = score_pitch(len);
    const int dblk = (int)(work & 3) * kCDims;  // the workgroup's 64 dimensions of each head
    // Key ranges (ranges grow with the token): the keys the item needs, from
    // a multiple of 4 past lo so that the float4 reads of the p rows align,
    // to the last pair's last key; a chunk inside every pair's window (from
    // the last pair's first key to the first pair's last key) needs no
    // bound on its keys: its p rows lie inside the sequence and every w is
    // p * (1/sum).
    uint32_t f0, l0, fl, ll;
    key_range(lo + pair0 / 3, lo, hi, window, f0, l0);
    key_range(lo + (pair1 - 1) / 3, lo, hi, window, fl, ll);
    const uint32_t kfirst = lo + ((f0 - lo) & ~3u), klast = ll, in_first = fl, in_last = l0;
    auto inside = [&](uint32_t c0) { return c0 >= in_first && c0 + kCKeys <= in_last; };
    float acc[8];  // pairs 16 (v / 4) + 4 g + v % 4, dimension dblk + 16 w + r16
#pragma unroll
    for (int v = 0; v < 8; ++v) acc[v] = 0.0f;
    // w staging: thread (pair tid % 32, the 8 keys 8 (tid / 32) ..), from
    // registers loaded while the previous chunk is computed.
    const uint32_t wp = (uint32_t)tid & (kCPairs - 1), wk = kCWKeys * ((uint32_t)tid / kCPairs);
    const uint32_t wpair = min(pair0 + wp, pair1 - 1);
    const float winv = scores[3 * (size_t)(lo + wpair / 3) + wpair % 3];
    const float* wsrc = scores + sbase + (size_t)wpair * pitch;
    uint32_t wfirst, wlast;
    key_range(lo + wpair / 3, lo, hi, window, wfirst, wlast);
    if (pair0 + wp >= pair1) wlast = wfirst;  // no such pair: w = 0
    float4 pw[kCWKeys / 4];
    auto load_w = [&](uint32_t c0) {
      if (inside(c0)) {  // uniform: no bound
#pragma unroll
        for (int j4 = 0; j4 < kCWKeys / 4; ++j4)
          pw[j4] = *reinterpret_cast<const float4*>(wsrc + (c0 + wk + 4 * j4 - lo));
        return;
      }
#pragma unroll
      for (int j4 = 0; j4 < kCWKeys / 4; ++j4) {
        const uint32_t k4 = c0 + wk + 4 * j4;  // 4 keys, 16-byte aligned in the row
        pw[j4] = k4 - lo < pitch ? *reinterpret_cast<const float4*>(wsrc + (k4 - lo))
                                 : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    };
    // v staging by DMA, no registers: wave w moves keys c0 + R w .. + R - 1
    // of the chunk (R = kCKeys / 4), 4 keys (64 lanes x 16 bytes) per
    // instruction. Keys past the
    // sequence read its last row: every pair's w is 0 there (a finite v
    // times +0 adds +0 or -0, which changes no sum). Byte offsets are taken
    // from the sequence's first row, so that 32 bits hold them for any row
    // count (a planned sequence is below 37,838 rows: 194 MB of qkv).
    const float* seq = qkv + (size_t)lo * kLd;
    // Row min(c0 + R w + 4 i + lane / 16, hi - 1) as a scalar base row
    // (clamped) plus a per-lane step of 0..3 (clamped to what is left).
    auto issue_v = [&](uint32_t c0, int buf) {
#pragma unroll
      for (int i = 0; i < kCKeys / 16; ++i) {
        const uint32_t brow = min(c0 - lo + (kCKeys / 4) * (uint32_t)w + 4 * i, hi - 1 - lo);  // uniform
        const uint32_t step = min((uint32_t)(lane >> 4), hi - 1 - lo - brow);
        dma16(seq + (size_t)brow * kLd, __umul24(step, kLd * 4u) + (uint32_t)(kVOff + dblk) * 4u + 16u * (uint32_t)(lane & 15),
              vl0 + (unsigned)buf * (kCKeys * kCDims * 4) + ((kCKeys / 4) * w + 4 * i) * (kCDims * 4));
      }
    };
    __syncthreads();  // the previous item's epilogue tile (in vl) is no longer read
    if (kfirst < klast) {
      issue_v(kfirst, 0);
      load_w(kfirst);
    }
    int buf = 0;
    for (uint32_t c0 = kfirst; c0 < klast; c0 += kCKeys, buf ^= 1) {
      // This wave's v DMA and w loads of the chunk have landed; after the
      // barrier every wave's have, and the previous chunk is no longer read.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (inside(c0)) {
#pragma unroll
        for (int j4 = 0; j4 < kCWKeys / 4; ++j4) {
          const float pr[4] = {pw[j4].x, pw[j4].y, pw[j4].z, pw[j4].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) wl[(wk + 4 * j4 + e) * kCPairs + wp] = pr[e] * winv;
        }
      } else {
#pragma unroll
        for (int j4 = 0; j4 < kCWKeys / 4; ++j4) {
          const float pr[4] = {pw[j4].x, pw[j4].y, pw[j4].z, pw[j4].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t kt = c0 + wk + 4 * j4 + e;
            const float wv = pr[e] * winv;
            wl[(wk + 4 * j4 + e) * kCPairs + wp] = kt >= wfirst && kt < wlast ? wv : 0.0f;
          }
        }
      }
      __syncthreads();
      if (c0 + kCKeys < klast) {
        issue_v(c0 + kCKeys, buf ^ 1);
        load_w(c0 + kCKeys);
      }
      // Keys in groups of 8 (keys past klast carry w = 0 for every pair and
      // add +0): per 2 keys one MFMA whose block b holds pairs 16 (b % 2) ..
      // + 15 (rows) x the wave's 16 dimensions for key 2 i + b / 2; the
      // group's MFMAs into separate registers, the next group's operands
      // read from LDS, then the adds in key order; the chunk's groups as
      // straight-line code (one uniform test per group, no loop counter).
      const int n8 = (int)((min((uint32_t)kCKeys, klast - c0) + 7) & ~7u);
      const float* wa = wl + (g >> 1) * kCPairs + 16 * (g & 1) + r16;
      const float* vb = vl[buf] + (g >> 1) * kCDims + 16 * w + r16;
      float an[4], bn[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        an[e] = wa[2 * e * kCPairs];
        bn[e] = vb[2 * e * kCDims];
      }
      auto group = [&](int j, bool more) {
#pragma unroll
        for (int e0 = 0; e0 < 4; e0 += kCBatch) {
          floatx16 prod[kCBatch];
#pragma unroll
          for (int e = 0; e < kCBatch; ++e)  // keys j + 2 e, j + 2 e + 1
            prod[e] = __builtin_amdgcn_mfma_f32_16x16x1f32(an[e0 + e], bn[e0 + e], zero, 0, 0, 0);
          if (e0 + kCBatch == 4 && more) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              an[e] = wa[(j + 8 + 2 * e) * kCPairs];
              bn[e] = vb[(j + 8 + 2 * e) * kCDims];
            }
          }
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int e = 0; e < kCBatch; ++e)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)  // key j + 2 (e0 + e) + kk: blocks 2 kk, 2 kk + 1
#pragma unroll
              for (int v = 0; v < 8; ++v) acc[v] = acc[v] + prod[e][8 * kk + v];
          __builtin_amdgcn_sched_barrier(0);
        }
      };
#pragma unroll
      for (int j = 0; j < kCKeys; j += 8)
        if (j < n8) group(j, j + 8 < kCKeys);  // the operands of a group past n8 are read, not used
    }
    // Through LDS (the v chunks' space) to [pair][64 dimensions], then
    // Q8_0: block (32 values) of 4 lanes x 8 values.
    static_assert(kCPairs * kCPitchV <= 2 * kCKeys * kCDims, "the epilogue tile fits in the v buffers");
    __syncthreads();
    float* tile = &vl[0][0];  // kCPairs x kCPitchV floats
#pragma unroll
    for (int v = 0; v < 8; ++v) tile[(16 * (v >> 2) + 4 * g + (v & 3)) * kCPitchV + 16 * w + r16] = acc[v];
    __syncthreads();
    const uint32_t qp = (uint32_t)tid >> 3, qb = ((uint32_t)tid >> 2) & 1, part = (uint32_t)tid & 3;
    float vals[8];
#pragma unroll
    for (int i = 0; i < 8; i += 4) {
      const float4 x4 = *reinterpret_cast<const float4*>(tile + qp * kCPitchV + 32 * qb + 8 * part + i);
      vals[i] = x4.x;
      vals[i + 1] = x4.y;
      vals[i + 2] = x4.z;
      vals[i + 3] = x4.w;
    }
    const uint32_t pair = min(pair0 + qp, pair1 - 1);
    const uint32_t t = lo + pair / 3, h = pair % 3;
    const unsigned e = h * kHeadDim + (unsigned)dblk + 32 * qb + 8 * part;
    quantize_block_part<4>(vals, pair0 + qp < pair1, cq + q8_tile_offset(t, e, kEmbd / kQK),
                           cd + (size_t)(e / kQK) * rows + t);
  }
}

// ---------------------------------------------------------------- host side

namespace {

// Per-sequence counts of the plan.
struct SeqPlan {
  size_t score_items, context_items, score_floats;
};
__host__ __device__ inline SeqPlan seq_plan(size_t len) {
  const size_t pairs = 3 * len;
  return {(len + kSKeys - 1) / kSKeys * ((pairs + kSPairs - 1) / kSPairs), (pairs + kCPairs - 1) / kCPairs,
          pairs * score_pitch((uint32_t)len)};
}

}  // namespace

AttentionCounts attention_counts(const size_t* offsets, size_t batch) {
  AttentionCounts c{0, inv_floats(batch ? offsets[batch] : 0), 0};
  size_t ctx = 0;
  for (size_t s = 0; s < batch; ++s) {
    const SeqPlan p = seq_plan(offsets[s + 1] - offsets[s]);
    c.score_items += p.score_items;
    ctx += p.context_items;
    c.score_floats += p.score_floats;
  }
  c.items = c.score_items + ctx;
  return c;
}

bool build_attention_plan(const size_t* offsets, size_t batch, const AttentionCounts& cap, uint32_t* items,
                          uint32_t* tok, AttentionCounts* used) {
  const AttentionCounts need = attention_counts(offsets, batch);
  if (used) *used = need;
  if (need.items > cap.items || need.score_floats > cap.score_floats) return false;
  // The records hold 32-bit score indices and counts: a packing whose
  // scores or items exceed them (sequences of some 37k tokens) is refused.
  if (need.score_floats > 0xFFFFFFFFull || need.items > 0xFFFFFFFFull) return false;
  size_t ns = 0, nc = need.score_items, sbase = inv_floats(batch ? offsets[batch] : 0);
  for (size_t s = 0; s < batch; ++s) {
    const size_t lo = offsets[s], hi = offsets[s + 1], len = hi - lo, pairs = 3 * len;
    for (size_t p0 = 0; p0 < pairs; p0 += kSPairs)
      for (size_t k0 = lo; k0 < hi; k0 += kSKeys) {
        uint32_t* it = items + 8 * ns++;
        it[0] = (uint32_t)lo;
        it[1] = (uint32_t)hi;
        it[2] = (uint32_t)k0;
        it[3] = (uint32_t)p0;
        it[4] = (uint32_t)std::min(pairs, p0 + kSPairs);
        it[5] = (uint32_t)sbase;
        it[6] = it[7] = 0;
      }
    for (size_t p0 = 0; p0 < pairs; p0 += kCPairs) {
      uint32_t* it = items + 8 * nc++;
      it[0] = (uint32_t)lo;
      it[1] = (uint32_t)hi;
      it[2] = (uint32_t)p0;
      it[3] = (uint32_t)std::min(pairs, p0 + kCPairs);
      it[4] = (uint32_t)sbase;
      it[5] = it[6] = it[7] = 0;
    }
    for (size_t t = lo; t < hi; ++t) {
      tok[4 * t] = (uint32_t)lo;
      tok[4 * t + 1] = (uint32_t)hi;
      tok[4 * t + 2] = (uint32_t)sbase;
      tok[4 * t + 3] = 0;
    }
    sbase += seq_plan(len).score_floats;
  }
  // The context kernel's unit order: its units (4 per context item, one per
  // 64 dimensions) cost about their sequence's 64-key chunks. When the eight
  // contiguous eighths of the unit list cost alike (waves of equal
  // sequences), each XCD takes one (its L2 then holds few sequences' rows);
  // otherwise the workgroups stride over the whole list, so each XCD gets a
  // share of every sequence (a contiguous split of a mixed packing loads
  // some XCDs with its long sequences: 1.5x the time on 16 log-uniform
  // segments). The decision rides in the context items (it[5]).
  const size_t citems = need.items - need.score_items, units = 4 * citems;
  if (units > 0) {
    std::vector<size_t> prefix(units + 1, 0);
    for (size_t u = 0; u < units; ++u) {
      const uint32_t* it = items + 8 * (need.score_items + u / 4);
      prefix[u + 1] = prefix[u] + (it[1] - it[0] + kCKeys - 1) / kCKeys;
    }
    size_t most = 0;
    for (size_t x = 0; x < kXcdCount; ++x)
      most = std::max(most, prefix[units * (x + 1) / kXcdCount] - prefix[units * x / kXcdCount]);
    const bool by_xcd = units >= kXcdCount && most * kXcdCount <= prefix[units] + prefix[units] / 32;
    for (size_t c = 0; c < citems; ++c) items[8 * (need.score_items + c) + 5] = by_xcd ? 1u : 0u;
  }
  return true;
}

AttentionCounts attention_capacity(size_t tokens, size_t batch) {
  // Score floats: 3n (n + 3) per sequence, at most 3 tokens^2 + 9 tokens,
  // plus the 1/sum area of 3 tokens rounded up to 4.
  AttentionCounts c;
  c.items = item_bound(tokens, batch);
  c.score_floats = 3 * tokens * tokens + 12 * tokens + 4;
  c.score_items = 0;
  return c;
}

hipError_t launch_attention_scores(const float* qkv, const uint32_t* items, const uint32_t* item_count, int grid,
                                   int window, int rows, float* scores, hipStream_t st) {
  if (rows <= 0 || rows % 4 != 0 || grid <= 0 || window < 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_scores_kernel, dim3(grid), dim3(256), 0, st, qkv,
                     reinterpret_cast<const uint4*>(items), item_count, window, rows, scores);
  return hipGetLastError();
}

template <int LANES>
hipError_t launch_group_softmax(const uint32_t* tok, int window, int rows, float* scores, hipStream_t st) {
  hipLaunchKernelGGL(attention_softmax_group_kernel<LANES>, dim3((3 * rows + kGroupPairs - 1) / kGroupPairs),
                     dim3(LANES * kGroupPairs), 0, st, scores, reinterpret_cast<const uint4*>(tok), window, rows);
  return hipGetLastError();
}

hipError_t launch_attention_softmax(const uint32_t* tok, int window, int rows, int longest, float* scores,
                                    hipStream_t st) {
  if (rows <= 0 || rows % 4 != 0 || window < 0 || longest < 0) return hipErrorInvalidValue;
  if (longest > 0 && longest <= kSoftmaxLanes16) return launch_group_softmax<16>(tok, window, rows, scores, st);
  if (longest > 0 && longest <= kSoftmaxLanes32) return launch_group_softmax<32>(tok, window, rows, scores, st);
  if (longest > 0 && longest <= kShortSoftmax) {
    hipLaunchKernelGGL(attention_softmax_kernel, dim3((3 * rows + kWavePairs - 1) / kWavePairs), dim3(64 * kWavePairs),
                       0, st, scores, reinterpret_cast<const uint4*>(tok), window, rows);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(attention_softmax_ring_kernel, dim3((3 * rows + kRingPairs - 1) / kRingPairs),
                     dim3(64 * kRingPairs), 0, st, scores, reinterpret_cast<const uint4*>(tok), window, rows);
  return hipGetLastError();
}

hipError_t launch_attention_context(const float* qkv, const uint32_t* items, const uint32_t* item_count, int grid,
                                    int window, int rows, const float* scores, int8_t* cq, float* cd,
                                    hipStream_t st) {
  if (rows <= 0 || rows % 4 != 0 || grid <= 0 || window < 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_context_kernel, dim3(grid), dim3(256), 0, st, qkv, scores,
                     reinterpret_cast<const uint4*>(items), item_count, window, rows, cq, cd);
  return hipGetLastError();
}

hipError_t launch_attention(const float* qkv, const uint32_t* items, const uint32_t* item_count, int grid,
                            const uint32_t* tok, int window, int rows, int longest, float* scores, int8_t* cq,
                            float* cd, hipStream_t st) {
  if (rows <= 0 || rows % 4 != 0 || grid <= 0 || window < 0 || longest < 0) return hipErrorInvalidValue;
  hipError_t e = launch_attention_scores(qkv, items, item_count, grid, window, rows, scores, st);
  if (e != hipSuccess) return e;
  e = launch_attention_softmax(tok, window, rows, longest, scores, st);
  if (e != hipSuccess) return e;
  return launch_attention_context(qkv, items, item_count, grid, window, rows, scores, cq, cd, st);
}

// ---------------------------------------------------------------- allocation-free form
//
// launch_attention_static keeps its plan and scores in `scratch`, a
// file-scope device array (one copy per GPU, alive until the process
// ends), and builds the plan on the device from device offsets, so a call
// allocates nothing. Layout: [item counts | pad to 256 B][token records,
// 16 B x kStaticRows][work items, 32 B x kStaticItems][scores]. Any packing
// of at most kStaticRows rows into at most kStaticBatch sequences fits
// (the bounds of attention_capacity). Nothing in it has to start at zero:
// the plan kernel writes the counts and every record the other kernels
// read, the softmax kernel every 1/sum the context kernel reads, and the
// softmax and context kernels use only scores written in the same call.
// Calls that overlap on one GPU share the array and race.

constexpr size_t kStaticRows = 2048, kStaticBatch = 2048;
constexpr size_t kStaticItems = item_bound(kStaticRows, kStaticBatch);
constexpr size_t kStaticScoreFloats = 3 * kStaticRows * kStaticRows + 12 * kStaticRows + 4;
constexpr size_t kStaticTokOff = 256;
constexpr size_t kStaticItemsOff = kStaticTokOff + 16 * kStaticRows;
constexpr size_t kStaticScoresOff = (kStaticItemsOff + 32 * kStaticItems + 255) / 256 * 256;
constexpr size_t kStaticBytes = kStaticScoresOff + sizeof(float) * kStaticScoreFloats;
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
attention_plan_kernel(const uint32_t* __restrict__ offsets, int batch, int rows, uint32_t* __restrict__ counts,
                      uint4* __restrict__ tok, uint4* __restrict__ items) {
  __shared__ uint32_t bound[kStaticBatch + 1], first_sitem[kStaticBatch + 1], first_citem[kStaticBatch + 1];
  __shared__ uint32_t first_score[kStaticBatch + 1];
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
  uint32_t ni = 0, nc = 0, ns = 0;
  for (int s = s0; s < s1; ++s) {
    const SeqPlan p = seq_plan(bound[s + 1] - bound[s]);
    first_sitem[s] = ni;
    first_citem[s] = nc;
    first_score[s] = ns;
    ni += (uint32_t)p.score_items;
    nc += (uint32_t)p.context_items;
    ns += (uint32_t)p.score_floats;
  }
  uint32_t total_sitems, total_citems, total_scores;
  const uint32_t ibase = plan_scan<false>(ni, tmp, total_sitems);
  const uint32_t cbase = plan_scan<false>(nc, tmp, total_citems);
  const uint32_t sbase = plan_scan<false>(ns, tmp, total_scores);
  const uint32_t score0 = (uint32_t)inv_floats((size_t)rows);
  for (int s = s0; s < s1; ++s) {
    first_sitem[s] += ibase;
    first_citem[s] += cbase;
    first_score[s] += sbase + score0;
  }
  if (tid == 0) {
    first_sitem[batch] = total_sitems;
    first_citem[batch] = total_citems;
    first_score[batch] = total_scores + score0;
    counts[0] = total_sitems;
    counts[1] = total_citems;
  }
  __syncthreads();
  for (uint32_t i = tid; i < total_sitems; i += kPlanThreads) {
    const int s = last_le(first_sitem, batch, i);  // a sequence with items has first_sitem[s] < first_sitem[s + 1]
    const uint32_t lo = bound[s], hi = bound[s + 1], pairs = 3 * (hi - lo);
    const uint32_t nk = (hi - lo + kSKeys - 1) / kSKeys, local = i - first_sitem[s];
    const uint32_t p0 = kSPairs * (local / nk), k0 = lo + kSKeys * (local % nk);
    items[2 * i] = make_uint4(lo, hi, k0, p0);
    items[2 * i + 1] = make_uint4(min(pairs, p0 + kSPairs), first_score[s], 0u, 0u);
  }
  for (uint32_t i = tid; i < total_citems; i += kPlanThreads) {
    const int s = last_le(first_citem, batch, i);
    const uint32_t lo = bound[s], hi = bound[s + 1], pairs = 3 * (hi - lo);
    const uint32_t p0 = kCPairs * (i - first_citem[s]);
    items[2 * (total_sitems + i)] = make_uint4(lo, hi, p0, min(pairs, p0 + kCPairs));
    items[2 * (total_sitems + i) + 1] = make_uint4(first_score[s], 0u, 0u, 0u);
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
  uint32_t* counts = reinterpret_cast<uint32_t*>(base);
  uint32_t* tok = reinterpret_cast<uint32_t*>(base + kStaticTokOff);
  uint32_t* items = reinterpret_cast<uint32_t*>(base + kStaticItemsOff);
  float* scores = reinterpret_cast<float*>(base + kStaticScoresOff);
  hipLaunchKernelGGL(attention_plan_kernel, dim3(1), dim3(kPlanThreads), 0, st, offsets, batch, rows, counts,
                     reinterpret_cast<uint4*>(tok), reinterpret_cast<uint4*>(items));
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_attention(qkv, items, counts, kAttentionGrid, tok, window, rows, 0, scores, cq, cd, st);
}

}  // namespace eg2
