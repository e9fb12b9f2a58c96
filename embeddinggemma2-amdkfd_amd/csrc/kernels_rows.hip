// Row kernels of the packed encoder forward. They are HBM-bound; each one
// fuses the element-wise work between two GEMMs so a token row is read and
// written once, and each reproduces the reference's operation order, so its
// results are bit-identical to the CPU path for identical inputs (the GeGLU
// kernel decides most Q8_0 values from a bounded tanh approximation and
// evaluates the host libm's tanhf for the rest: the same bits, see
// geglu_quantize_part4).
//
// Work mapping. One 64-lane wave per 768-wide token row (a 2048-token wave
// gives two waves per SIMD), so latency, not bandwidth, is what the design
// fights:
//  * element-wise work runs one float4 per lane per 256 columns, coalesced,
//    with the row kept in registers from load to store;
//  * the SSE2-order sum of squares (kernels.c:82-94) runs one lane per
//    chain: a lane owns chain c (the sequential sum of row[8t + c]^2) over
//    the row staged transposed in LDS (24 16-byte reads per lane, in three
//    groups of eight issued before their dependent additions), and an 8-lane
//    group combines a row's eight chains with DPP moves. The residual kernel
//    stages eight rows per workgroup and its first wave runs all 64 chains
//    (8 rows x 8 chains);
//    the embedding kernel's single wave runs its row's chains in every
//    8-lane group, so every lane ends with the total without an LDS round
//    trip;
//  * Q8_0 quantization works on the registers: a 32-value block is 8 lanes
//    x 4 values, its maximum combined by DPP, and each lane stores its 4
//    int8 values as one 32-bit word of the row tiles.
#include <algorithm>

#include "eg2_device.hpp"
#include "eg2_kernels.hpp"

namespace eg2 {

constexpr int kBlocks = kEmbd / kQK;                   // 24 blocks per row
constexpr int kVec = kEmbd / 256;                      // float4 per lane per row

// ---------------------------------------------------------------- 768-wide rows
// A 768-float token row is held one float4 per lane per 256 columns (lane L
// has elements 4L..4L+3 + 256r, r = 0..2). Its SSE2 sum of squares
// (kernels.c:82-94) needs chain c = the sequential sum over t of
// row[8t + c]^2: the row's squares (each rounded, as the reference's) are
// staged transposed in LDS, tr[c][t] = row[8t + c]^2, by every lane of the
// row, so the lane that runs chain c reads its 96 squares with 24
// ds_read_b128 and only adds. The 104-float pitch
// puts the eight chain rows 40 banks apart (conflict-free reads) and the
// two lanes of a pair 32 banks apart (conflict-free transposed writes).
constexpr int kChain = kEmbd / 8;  // 96
constexpr int kTPitch = kChain + 8;
typedef float TRow[kTPitch];

__device__ __forceinline__ void stage_squares(TRow* tr, const float4 (&v)[kVec]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int r = 0; r < kVec; ++r) {
    const float c4[4] = {v[r].x * v[r].x, v[r].y * v[r].y, v[r].z * v[r].z, v[r].w * v[r].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = 4 * (lane + 64 * r) + k;
      tr[e & 7][e >> 3] = c4[k];
    }
  }
}

// Chain c of the SSE2 sum of squares from the staged squares, read in three
// groups of eight float4, each group's reads issued before its additions.
// The rolled outer loop keeps 32 registers of reads in flight, not 96: the
// residual kernel's register count (and so how many of its waves fit beside
// other streams' kernels on a CU) is set by this chain.
__device__ __forceinline__ float squares_chain(const TRow* tr, int c) {
  float s = 0.0f;
#pragma unroll 1
  for (int g = 0; g < kChain / 32; ++g) {
    float4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = *reinterpret_cast<const float4*>(&tr[c][32 * g + 4 * j]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      s = s + v[j].x;
      s = s + v[j].y;
      s = s + v[j].z;
      s = s + v[j].w;
    }
  }
  return s;
}

// DPP moves within 16-lane rows: quad permutation, shift left/right by n
// lanes. `dpp` writes every lane (lanes shifted in from outside the row
// read 0 and are not used); `dpp_into` writes only the lanes of the 4-lane
// banks in BANKS and keeps `old` elsewhere. Choosing lanes by bank mask,
// not by a select on the lane index, keeps every source lane active: the
// compiler may turn a select of two DPP results into an EXEC-masked branch,
// and a DPP move reads 0 from lanes that EXEC disables.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}
template <int CTRL, int BANKS>
__device__ __forceinline__ float dpp_into(float old, float src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, src), CTRL, 0xf, BANKS,
                                                               false));
}
constexpr int kQuad1032 = 0xB1, kQuad2301 = 0x4E;  // quad_perm [1,0,3,2], [2,3,0,1]
constexpr int kQuad0000 = 0x00, kQuad1111 = 0x55, kQuad2222 = 0xAA, kQuad3333 = 0xFF;
constexpr int kRowShl4 = 0x104, kRowShr4 = 0x114;  // lane i reads lane i + 4 / i - 4
constexpr int kBanks02 = 0x5, kBanks13 = 0xA;      // lanes 0-3 and 8-11 / 4-7 and 12-15 of a row

// The value of lane i ^ 4: the other 4-lane half of each aligned 8-lane group.
__device__ __forceinline__ float other_quad(float x) {
  return dpp_into<kRowShr4, kBanks13>(dpp_into<kRowShl4, kBanks02>(x, x), x);
}

// sse2_combine with DPP instead of LDS shuffles: lanes 8g..8g+7 hold chains
// 0..7 (chains 0-3 are the first 4-wide accumulator, 4-7 the second);
// v[j] = acc0[j] + acc1[j], total (v0 + v2) + (v1 + v3) (kernels.c:35-39),
// returned to every lane of the group.
__device__ __forceinline__ float sse2_combine_dpp(float s) {
  const float v = s + dpp<kRowShl4>(s);  // lanes 0-3 of the group: v[0..3]
  const float total = (dpp<kQuad0000>(v) + dpp<kQuad2222>(v)) + (dpp<kQuad1111>(v) + dpp<kQuad3333>(v));
  return dpp_into<kRowShr4, kBanks13>(total, total);  // lanes 4-7 take lanes 0-3's
}

// Maximum over each aligned group of 8 lanes, on every lane of the group.
__device__ __forceinline__ float group8_max(float m) {
  m = fmaxf(m, dpp<kQuad1032>(m));
  m = fmaxf(m, dpp<kQuad2301>(m));
  return fmaxf(m, other_quad(m));
}

// quants.c:97-177 (scalar path) on the row held as float4 per lane: block b
// (32 values) is lanes 8(b % 8)..+7 of register r = b / 8, four values per
// lane; the block maximum is combined over those 8 lanes. A group's three
// blocks get their scale computed once each: lane 8i + r takes block
// (r, i)'s maximum, computes d = amax / 127, 1/d and the fp16 scale, and
// stores the latter's float value at d[b * ld]; the group's lanes take the
// three 1/d back by swizzle broadcasts (an LDS-unit permute, no VALU work).
// Each lane stores its 4 int8 values (contiguous in the row-tile layout)
// for row t of q. v[r] must already hold the values to quantize; all 64
// lanes must be active.
template <int R>
__device__ __forceinline__ float group8_lane(float x) {
  // ds_swizzle bitmask mode within 32 lanes: source lane (lane & 0x18) | R
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x18 | (R << 5)));
}
__device__ __forceinline__ void quantize_row_lanes(const float4 (&v)[kVec], int t, int8_t* __restrict__ q,
                                                   float* __restrict__ d, int ld) {
  static_assert(kVec == 3, "three blocks per 8-lane group");
  const int lane = threadIdx.x & 63, r8 = lane & 7;
  float amax[kVec];
#pragma unroll
  for (int r = 0; r < kVec; ++r)
    amax[r] = group8_max(fmaxf(fmaxf(fabsf(v[r].x), fabsf(v[r].y)), fmaxf(fabsf(v[r].z), fabsf(v[r].w))));
  const float am = r8 == 0 ? amax[0] : (r8 == 1 ? amax[1] : amax[2]);  // lanes 8i + 3 .. 7: block 2 again, unused
  const float dd = div127(am);
  const float id_own = am != 0.0f ? 1.0f / dd : 0.0f;  // 0 for an all-zero block, whose values quantize to 0
  if (r8 < kVec) d[(size_t)((lane >> 3) + 8 * r8) * ld] = fp16_bits_to_fp32(fp32_to_fp16_bits(dd));
  const float ids[kVec] = {group8_lane<0>(id_own), group8_lane<1>(id_own), group8_lane<2>(id_own)};
#pragma unroll
  for (int r = 0; r < kVec; ++r) {
    const float id = ids[r];
    const int e = 4 * (lane + 64 * r);
    const int32_t q0 = q8_value(v[r].x, id), q1 = q8_value(v[r].y, id), q2 = q8_value(v[r].z, id),
                  q3 = q8_value(v[r].w, id);
    *reinterpret_cast<uint32_t*>(q + q8_tile_offset(t, e, kBlocks)) = pack_i8x4(q0, q1, q2, q3);
  }
}

// engine.c:288-295 + kernels.c:139-151 (the first projection's input):
// x = (fp16(d) * sqrt(768)) * q from the raw GGUF Q8_0 row of token_embd,
// then the layer-0 attn_norm RMSNorm quantized to Q8_0.
__global__ void __launch_bounds__(64)
embed_norm_quant_kernel(const uint8_t* __restrict__ table, const int32_t* __restrict__ ids, float embed_scale,
                        const float* __restrict__ norm_w, float eps, float* __restrict__ x,
                        int8_t* __restrict__ xq, float* __restrict__ xd) {
  constexpr int kRaw = kBlocks * 34;  // 816 bytes = 51 x 16
  __shared__ __align__(16) uint8_t raw[kRaw];
  __shared__ __align__(16) float tr[8][kTPitch];
  const int t = blockIdx.x, lane = threadIdx.x;
  float4 wv[kVec];
#pragma unroll
  for (int r = 0; r < kVec; ++r) wv[r] = *reinterpret_cast<const float4*>(norm_w + 4 * (lane + 64 * r));
  // GGUF rows of this tensor are 16-byte aligned: 816 = 16 * 51 and tensor
  // data is 32-byte aligned.
  if (lane < kRaw / 16)
    reinterpret_cast<uint4*>(raw)[lane] = reinterpret_cast<const uint4*>(table + (size_t)ids[t] * kRaw)[lane];
  __syncthreads();
  float4 v[kVec];
#pragma unroll
  for (int r = 0; r < kVec; ++r) {
    const int e = 4 * (lane + 64 * r);
    const uint8_t* blk = raw + (e / kQK) * 34;
    const float dd = fp16_bits_to_fp32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8)) * embed_scale;  // quants.c:67
    const uint8_t* qs = blk + 2 + e % kQK;
    v[r].x = dd * (float)(int8_t)qs[0];  // quants.c:87
    v[r].y = dd * (float)(int8_t)qs[1];
    v[r].z = dd * (float)(int8_t)qs[2];
    v[r].w = dd * (float)(int8_t)qs[3];
    *reinterpret_cast<float4*>(x + (size_t)t * kEmbd + e) = v[r];
  }
  stage_squares(tr, v);
  __syncthreads();
  const float inv = rms_inverse(sse2_combine_dpp(squares_chain(tr, lane & 7)), kEmbd, eps);
  // (x*w)*inv (kernels.c:124-133, SSE2 branch), then Q8_0 (kernels.c:139-151).
#pragma unroll
  for (int r = 0; r < kVec; ++r) {
    const float p0 = v[r].x * wv[r].x, p1 = v[r].y * wv[r].y, p2 = v[r].z * wv[r].z, p3 = v[r].w * wv[r].w;
    v[r] = make_float4(p0 * inv, p1 * inv, p2 * inv, p3 * inv);
  }
  quantize_row_lanes(v, t, xq, xd + t, (int)gridDim.x);
}

// Eight token rows per workgroup (one wave each) share the SSE2 chains: each
// wave stages its row transposed, then wave 0 runs all 64 chains (lane
// 8 k + c: chain c of token k) and combines each token's eight with DPP,
// so the 96-step chains issue once per eight tokens instead of once per
// token. A token's rows start 4 floats past the previous token's (its 8
// chain rows span 8 x kTPitch + 4 floats), so the 16 rows read in one LDS
// cycle fall in distinct banks.
constexpr int kRowsPerGroup = 8;
constexpr int kTokStride = 8 * kTPitch + 4;  // floats per token in the staging area

__device__ __forceinline__ float* token_rows(float* tr, int k) { return tr + k * kTokStride; }

// Wave 0: inv[k] = rms_inverse of token k's staged row, k = 0..7.
__device__ __forceinline__ void group_rms_inverse(float* tr, float* inv, float eps) {
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  const TRow* rows = reinterpret_cast<const TRow*>(token_rows(tr, lane >> 3));
  const float r = rms_inverse(sse2_combine_dpp(squares_chain(rows, lane & 7)), kEmbd, eps);
  if ((lane & 7) == 0) inv[lane >> 3] = r;
}

// kernels.c:163-188 (SSE2 build: scalar branch, residual += (h*inv)*w), then
// kernels.c:139-151 with the next norm weight on the updated residual. With
// next_w == nullptr only the residual update runs. Rows past `rows` in the
// last workgroup load nothing and store nothing; their waves still join
// every barrier. The two norm weight vectors are staged once per workgroup
// in LDS (threads 0-191 and 192-383, one float4 each) rather than held in
// every wave's registers.
__global__ void __launch_bounds__(64 * kRowsPerGroup)
residual_norm_quant_kernel(float* __restrict__ x, const float* __restrict__ h, const float* __restrict__ post_w,
                           const float* __restrict__ next_w, float eps, int8_t* __restrict__ xq,
                           float* __restrict__ xd, int rows) {
  __shared__ __align__(16) float tr[kRowsPerGroup * kTokStride];
  __shared__ float inv_s[2][kRowsPerGroup];
  __shared__ float4 wl[2][kEmbd / 4];
  // Highest issue priority on its SIMDs: this short, latency-bound kernel
  // (loads, two serial chains, stores) sits on each wave's critical path
  // and shares the SIMDs with other streams' GEMM and attention waves,
  // whose throughput-bound work fills the gaps it leaves.
  __builtin_amdgcn_s_setprio(3);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // XCD-aware order (a grid that is a multiple of 8): XCD b % 8 takes the
  // contiguous eighth of the row groups, the rows the O and down GEMMs
  // computed on it (their tile grid splits into 8 row parts).
  const int grp = gridDim.x % 8 == 0 ? (int)((blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8) : (int)blockIdx.x;
  const int t = grp * kRowsPerGroup + w;
  const bool live = t < rows;
  if (threadIdx.x < kEmbd / 4) {
    wl[0][threadIdx.x] = reinterpret_cast<const float4*>(post_w)[threadIdx.x];
  } else if (threadIdx.x < kEmbd / 2 && next_w) {
    wl[1][threadIdx.x - kEmbd / 4] = reinterpret_cast<const float4*>(next_w)[threadIdx.x - kEmbd / 4];
  }
  float4 hv[kVec], xv[kVec];
#pragma unroll
  for (int r = 0; r < kVec; ++r) {
    const int e = 4 * (lane + 64 * r);
    hv[r] = live ? *reinterpret_cast<const float4*>(h + (size_t)t * kEmbd + e) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    xv[r] = live ? *reinterpret_cast<const float4*>(x + (size_t)t * kEmbd + e) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  float* mine = token_rows(tr, w);
  stage_squares(reinterpret_cast<TRow*>(mine), hv);
  __syncthreads();
  group_rms_inverse(tr, inv_s[0], eps);
  __syncthreads();
  const float inv_h = inv_s[0][w];
#pragma unroll
  for (int r = 0; r < kVec; ++r) {
    const int e = 4 * (lane + 64 * r);
    const float a0 = hv[r].x * inv_h, a1 = hv[r].y * inv_h, a2 = hv[r].z * inv_h, a3 = hv[r].w * inv_h;
    const float4 wr = wl[0][lane + 64 * r];
    const float b0 = a0 * wr.x, b1 = a1 * wr.y, b2 = a2 * wr.z, b3 = a3 * wr.w;
    xv[r] = make_float4(xv[r].x + b0, xv[r].y + b1, xv[r].z + b2, xv[r].w + b3);
    if (live) *reinterpret_cast<float4*>(x + (size_t)t * kEmbd + e) = xv[r];
  }
  if (!next_w) return;  // uniform over the grid
  // Wave 0 read every token's rows before the barrier above.
  stage_squares(reinterpret_cast<TRow*>(mine), xv);
  __syncthreads();
  group_rms_inverse(tr, inv_s[1], eps);
  __syncthreads();
  const float inv = inv_s[1][w];
  // (x*w)*inv (kernels.c:124-133, SSE2 branch), then Q8_0 (kernels.c:139-151).
#pragma unroll
  for (int r = 0; r < kVec; ++r) {
    const float4 nr = wl[1][lane + 64 * r];
    const float p0 = xv[r].x * nr.x, p1 = xv[r].y * nr.y, p2 = xv[r].z * nr.z, p3 = xv[r].w * nr.w;
    xv[r] = make_float4(p0 * inv, p1 * inv, p2 * inv, p3 * inv);
  }
  if (live) quantize_row_lanes(xv, t, xq, xd + t, rows);
}

constexpr int kHeadStride = kHeadDim + 8;  // LDS row of one head: 8 banks apart

// kernels.c:233-264 on one token of the fused QKV projection output
// [q0 q1 q2 | k | v] (fp32, kQKVCols wide): per-head RMS with the weight
// applied before the inverse, NeoX rotation of pairs (d, d+128) with the
// host-built cos/sin row of this token's position, Q scaled by 0.0625 after
// rotation; v unchanged. The results (bit-identical to the reference) go to
// the same layout in `out`, which may be `qkv` itself: the row is read in
// full before any of it is written.
__global__ void __launch_bounds__(64)
qk_norm_rope_kernel(const float* qkv, const float* __restrict__ q_w, const float* __restrict__ k_w,
                    const float* __restrict__ rope, const int32_t* __restrict__ pos, float eps, float* out) {
  constexpr int kRows = kHeads + 1;  // q heads, then k
  constexpr int half = kHeadDim / 2;
  __shared__ __align__(16) float rows[kRows][kHeadStride];
  const int t = blockIdx.x, lane = threadIdx.x;
  const float* src = qkv + (size_t)t * kQKVCols;
  float* dst = out + (size_t)t * kQKVCols;
  const float* cs = rope + (size_t)pos[t] * kHeadDim;  // [cos 0..127 | sin 0..127]
  const float c0 = cs[lane], c1 = cs[lane + 64], s0 = cs[half + lane], s1 = cs[half + lane + 64];
#pragma unroll
  for (int r = 0; r < kRows * kHeadDim / 256; ++r) {
    const int e = 4 * (lane + 64 * r);
    *reinterpret_cast<float4*>(&rows[e / kHeadDim][e % kHeadDim]) = *reinterpret_cast<const float4*>(src + e);
  }
  const float4 v = *reinterpret_cast<const float4*>(src + kRows * kHeadDim + 4 * lane);
  __syncthreads();
  *reinterpret_cast<float4*>(dst + kRows * kHeadDim + 4 * lane) = v;
  // lanes 8r..8r+7 run the chains of head row r (r < 4); the rest repeat row 0
  const int hr = (lane >> 3) < kRows ? (lane >> 3) : 0;
  const float ss = sse2_combine(sse2_chain<kHeadDim>(rows[hr], lane & 7));
  float inv[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) inv[r] = rms_inverse(__shfl(ss, 8 * r, 64), kHeadDim, eps);
#pragma unroll
  for (int hd = 0; hd < kRows; ++hd) {
    const float* w = hd < kHeads ? q_w : k_w;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int d = lane + 64 * j;
      const float c = j ? c1 : c0, s = j ? s1 : s0;
      const float x0 = rows[hd][d] * w[d] * inv[hd];
      const float x1 = rows[hd][d + half] * w[d + half] * inv[hd];
      const float a0 = x0 * c, a1 = x1 * s;
      const float b0 = x0 * s, b1 = x1 * c;
      float lo = a0 - a1, hi = b0 + b1;
      if (hd < kHeads) {
        lo = lo * 0.0625f;
        hi = hi * 0.0625f;
      }
      dst[hd * kHeadDim + d] = lo;
      dst[hd * kHeadDim + d + half] = hi;
    }
  }
}

// kernels.c:367-371 and :373-391: gelu_tanh(gate) * up, quantized to Q8_0,
// each 32-value block over 4 lanes (8 values each; geglu_quantize_part4,
// which evaluates the exact tanhf only where the Q8_0 result depends on
// it), values in the row-tile layout, block scales transposed ([block][row]).
// gu rows hold [gate 0..1151 | up 0..1151].
__global__ void __launch_bounds__(256)
gelu_quant_kernel(const float* __restrict__ gu, int8_t* __restrict__ gq, float* __restrict__ gd, int n_rows) {
  constexpr int kB = kFF / kQK;  // 36 blocks per row
  const int j = blockIdx.x * 256 + threadIdx.x;  // quarter block
  const int jb = min(j >> 2, n_rows * kB - 1);   // the last wave may run past the end: repeat, store nothing
  const int t = jb / kB, b = jb - t * kB, e0 = b * kQK + (j & 3) * 8;
  const float* g = gu + (size_t)t * (2 * kFF) + e0;
  const float* u = g + kFF;
  float gs[8], us[8];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float4 g4 = *reinterpret_cast<const float4*>(g + 4 * i);
    const float4 u4 = *reinterpret_cast<const float4*>(u + 4 * i);
    gs[4 * i] = g4.x, gs[4 * i + 1] = g4.y, gs[4 * i + 2] = g4.z, gs[4 * i + 3] = g4.w;
    us[4 * i] = u4.x, us[4 * i + 1] = u4.y, us[4 * i + 2] = u4.z, us[4 * i + 3] = u4.w;
  }
  geglu_quantize_part4(gs, us, (j >> 2) < n_rows * kB, gq + q8_tile_offset(t, e0, kB), gd + (size_t)b * n_rows + t);
}

// quants.c:97-177 on rows of width k (k % 32 == 0), each block over 4 lanes;
// values in the row-tile layout, block scales transposed ([block][row]).
__global__ void __launch_bounds__(256)
quantize_rows_kernel(const float* __restrict__ x, int k, int8_t* __restrict__ q, float* __restrict__ d,
                     int n_rows) {
  const int nb = k / kQK;
  const int j = blockIdx.x * 256 + threadIdx.x;
  const int jb = min(j >> 2, n_rows * nb - 1);
  const int t = jb / nb, b = jb - t * nb, e0 = b * kQK + (j & 3) * 8;
  const float* src = x + (size_t)t * k + e0;
  float v[8];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float4 x4 = *reinterpret_cast<const float4*>(src + 4 * i);
    v[4 * i + 0] = x4.x;
    v[4 * i + 1] = x4.y;
    v[4 * i + 2] = x4.z;
    v[4 * i + 3] = x4.w;
  }
  quantize_block_part<4>(v, (j >> 2) < n_rows * nb, q + q8_tile_offset(t, e0, nb), d + (size_t)b * n_rows + t);
}

// kernels.c:153-161 in place on a token row: x = (x*w)*inv.
__global__ void __launch_bounds__(64)
rms_norm_rows_kernel(float* __restrict__ x, const float* __restrict__ w, float eps) {
  __shared__ __align__(16) float tr[8][kTPitch];
  const int t = blockIdx.x, lane = threadIdx.x;
  float4 xv[kVec];
#pragma unroll
  for (int r = 0; r < kVec; ++r) xv[r] = *reinterpret_cast<const float4*>(x + (size_t)t * kEmbd + 4 * (lane + 64 * r));
  stage_squares(tr, xv);
  __syncthreads();
  const float inv = rms_inverse(sse2_combine_dpp(squares_chain(tr, lane & 7)), kEmbd, eps);
#pragma unroll
  for (int r = 0; r < kVec; ++r) {
    const int e = 4 * (lane + 64 * r);
    const float4 wv = *reinterpret_cast<const float4*>(w + e);
    const float p0 = xv[r].x * wv.x, p1 = xv[r].y * wv.y, p2 = xv[r].z * wv.z, p3 = xv[r].w * wv.w;
    *reinterpret_cast<float4*>(x + (size_t)t * kEmbd + e) = make_float4(p0 * inv, p1 * inv, p2 * inv, p3 * inv);
  }
}

// kernels.c:417-427 after the per-token RMS (rms_norm_rows_kernel): one
// workgroup per sequence, one thread per column, sums the normalised rows in
// token order (two batches of kPoolBatch rows in flight), scales by 1/n,
// then L2-normalises in the SSE2 order (kernels.c:393-396).
constexpr int kPoolBatch = 32;

// Column e of rows [lo, hi) summed in token order; the loads of the next
// batch of rows are in flight while the current batch is added.
__device__ __forceinline__ float column_sum(const float* __restrict__ x, uint32_t lo, uint32_t hi, int e) {
  float sum = 0.0f;
  float v[2][kPoolBatch];
  auto load = [&](float (&b)[kPoolBatch], uint32_t t) {
#pragma unroll
    for (int i = 0; i < kPoolBatch; ++i) b[i] = t + i < hi ? x[(size_t)(t + i) * kEmbd + e] : 0.0f;
  };
  load(v[0], lo);
  for (uint32_t t = lo; t < hi; t += 2 * kPoolBatch) {
    load(v[1], t + kPoolBatch);
#pragma unroll
    for (int i = 0; i < kPoolBatch; ++i)
      if (t + i < hi) sum = sum + v[0][i];
    load(v[0], t + 2 * kPoolBatch);
#pragma unroll
    for (int i = 0; i < kPoolBatch; ++i)
      if (t + kPoolBatch + i < hi) sum = sum + v[1][i];
  }
  return sum;
}

__global__ void __launch_bounds__(kEmbd)
pool_l2_kernel(const float* __restrict__ x, const uint32_t* __restrict__ offsets, float* __restrict__ out) {
  __shared__ float acc[kEmbd];
  __shared__ float total;
  const int s = blockIdx.x, e = threadIdx.x;
  const uint32_t lo = offsets[s], hi = offsets[s + 1];
  const float sum = column_sum(x, lo, hi, e);
  const float scale = 1.0f / (float)(hi - lo);
  acc[e] = sum * scale;
  __syncthreads();
  if (e < 64) {
    const float ss = sse2_combine(sse2_chain<kEmbd>(acc, e & 7));
    if (e == 0) total = ss;
  }
  __syncthreads();
  const float ss = total;
  out[(size_t)s * kEmbd + e] = ss != 0.0f ? acc[e] * (1.0f / __builtin_sqrtf(ss)) : acc[e];
}

// The mean of pool_l2_kernel alone, one workgroup per (sequence, 64
// columns): a sequence's rows are read by 12 CUs instead of one, which is
// what bounds pool_l2_kernel on long sequences. Followed by
// l2_prefix_kernel over the full width (the same arithmetic as the second
// half of pool_l2_kernel), the result is pool_l2_kernel's bit for bit.
__global__ void __launch_bounds__(64)
pool_mean_kernel(const float* __restrict__ x, const uint32_t* __restrict__ offsets, float* __restrict__ out) {
  const int s = blockIdx.x, e = 64 * blockIdx.y + threadIdx.x;
  const uint32_t lo = offsets[s], hi = offsets[s + 1];
  const float sum = column_sum(x, lo, hi, e);
  const float scale = 1.0f / (float)(hi - lo);
  out[(size_t)s * kEmbd + e] = sum * scale;
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

namespace {
dim3 quarter_block_groups(int blocks) { return dim3((4 * blocks + 255) / 256); }
}  // namespace

hipError_t launch_embed_norm_quant(const uint8_t* table, const int32_t* ids, int rows, float embed_scale,
                                   const float* norm_w, float eps, float* x, int8_t* xq, float* xd,
                                   hipStream_t st) {
  hipLaunchKernelGGL(embed_norm_quant_kernel, dim3(rows), dim3(64), 0, st, table, ids, embed_scale, norm_w, eps, x,
                     xq, xd);
  return hipGetLastError();
}

hipError_t launch_residual_norm_quant(float* x, const float* h, const float* post_w, const float* next_w,
                                      float eps, int8_t* xq, float* xd, int rows, hipStream_t st) {
  hipLaunchKernelGGL(residual_norm_quant_kernel, dim3((rows + kRowsPerGroup - 1) / kRowsPerGroup),
                     dim3(64 * kRowsPerGroup), 0, st, x, h, post_w, next_w, eps, xq, xd, rows);
  return hipGetLastError();
}

// The restated libm functions (eg2_libm.hpp) on n floats, for comparison
// with the host's: e[i] = expf(x[i]), t[i] = tanhf(x[i]) in the branch-free
// form the GELU uses.
__global__ void __launch_bounds__(256)
libm_eval_kernel(const float* __restrict__ x, unsigned n, float* __restrict__ e, float* __restrict__ t) {
  for (unsigned i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    e[i] = libm::expf(x[i]);
    t[i] = libm::tanhf_flat(x[i]);
  }
}

hipError_t launch_libm_eval(const float* x, unsigned n, float* e, float* t, hipStream_t st) {
  if (n == 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(libm_eval_kernel, dim3(std::min(4096u, (n + 255) / 256)), dim3(256), 0, st, x, n, e, t);
  return hipGetLastError();
}

// max over every finite float x of |tanh_approx(x) - tanhf(x)| (the restated
// host tanhf), as the bit pattern of the float, reduced by an atomic max (the
// bit patterns of non-negative floats order as the floats do). *out must
// start at 0.
__global__ void __launch_bounds__(256) tanh_approx_error_kernel(uint32_t* __restrict__ out) {
  const uint64_t threads = (uint64_t)gridDim.x * 256, per = (1ull << 32) / threads;
  const uint64_t first = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * per;
  float worst = 0.0f;
  for (uint64_t i = 0; i < per; ++i) {
    const float x = __uint_as_float((uint32_t)(first + i));
    if (!(fabsf(x) <= 3.40282347e38f)) continue;  // NaN or infinite
    worst = fmaxf(worst, fabsf(tanh_approx(x) - libm::tanhf_flat(x)));
  }
  atomicMax(out, __float_as_uint(worst));
}

hipError_t launch_tanh_approx_error(uint32_t* out, hipStream_t st) {
  hipLaunchKernelGGL(tanh_approx_error_kernel, dim3(16384), dim3(256), 0, st, out);  // 2^32 / (16384 * 256) each
  return hipGetLastError();
}

hipError_t launch_qk_norm_rope(const float* qkv, const float* q_w, const float* k_w, const float* rope,
                               const int32_t* pos, float eps, float* out, int rows, hipStream_t st) {
  if (rows <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(rows), dim3(64), 0, st, qkv, q_w, k_w, rope, pos, eps, out);
  return hipGetLastError();
}

hipError_t launch_gelu_quant(const float* gu, int8_t* gq, float* gd, int rows, hipStream_t st) {
  hipLaunchKernelGGL(gelu_quant_kernel, quarter_block_groups(rows * (kFF / kQK)), dim3(256), 0, st, gu, gq, gd,
                     rows);
  return hipGetLastError();
}

hipError_t launch_quantize_rows(const float* x, int k, int8_t* q, float* d, int rows, hipStream_t st) {
  hipLaunchKernelGGL(quantize_rows_kernel, quarter_block_groups(rows * (k / kQK)), dim3(256), 0, st, x, k, q, d,
                     rows);
  return hipGetLastError();
}

hipError_t launch_rms_norm_rows(float* x, const float* w, float eps, int rows, hipStream_t st) {
  hipLaunchKernelGGL(rms_norm_rows_kernel, dim3(rows), dim3(64), 0, st, x, w, eps);
  return hipGetLastError();
}

hipError_t launch_pool_l2(const float* x, const uint32_t* offsets, float* out, int batch, hipStream_t st) {
  hipLaunchKernelGGL(pool_l2_kernel, dim3(batch), dim3(kEmbd), 0, st, x, offsets, out);
  return hipGetLastError();
}

hipError_t launch_pool_mean(const float* x, const uint32_t* offsets, float* out, int batch, hipStream_t st) {
  hipLaunchKernelGGL(pool_mean_kernel, dim3(batch, kEmbd / 64), dim3(64), 0, st, x, offsets, out);
  return hipGetLastError();
}

hipError_t launch_l2_prefix(float* x, int width, int dims, int rows, hipStream_t st) {
  hipLaunchKernelGGL(l2_prefix_kernel, dim3(rows), dim3(64), (size_t)dims * sizeof(float), st, x, width, dims);
  return hipGetLastError();
}

}  // namespace eg2
