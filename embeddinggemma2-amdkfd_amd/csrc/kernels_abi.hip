// The operator set of the reference's by-name kernel interface (the
// kernels/abi.h records, the kernel names and launch geometry of
// kernels/eg2.c) on this library's own gfx950 designs.
//
// Each kernel takes its record by value, so its kernarg segment has the
// record's layout and a code object built from this file can be dispatched
// by symbol name ("eg2_mm64x64.kd", ...) with the same records, grids and
// workgroup sizes the reference executor uses (src/gemma2_kfd.cpp:160-165,
// 248-336) and its operator test uses (tests/kernels.cpp:36-137). The
// results meet that test's tolerances (2e-5 absolute against exact
// references; 2e-6 between a fused operator and its unfused sequence); they
// are not the reference kernels' bits.
//
// Designs:
//  - projections (eg2_mm*): fp32 MFMA (v_mfma_f32_16x16x4f32) on LDS-staged
//    32-deep K slices of the activations and of the weights decoded to fp32
//    (F32, F16, BF16 or Q8_0 blocks over the flattened matrix), zero-padded
//    past k. The MFMA's k index is a permutation of the slice chosen so that
//    each lane reads contiguous float4s of its row: lane group g (lanes
//    16g .. 16g+15) feeds slice elements g*KW/4 .. (g+1)*KW/4 - 1, one per
//    MFMA. The 16x16 tile splits the slice over its four waves and adds
//    their partial tiles at the end; the wider tiles give each wave its own
//    16x16 blocks.
//  - attention: keys in chunks of 64, one per lane: every lane computes its
//    key's whole dot product against q (broadcast from LDS), so a chunk
//    costs one wave max and one wave sum instead of one reduction per key;
//    then the softmax weights of the chunk (exp through the host libm's
//    expf restated in eg2_libm.hpp, rescaled by the running maximum between
//    chunks) go through LDS to the context, where lanes own dimensions.
//  - row operators (norm, norm_residual, norm_rope): one wave per row with
//    the row held in registers as float4s (a single read of the row), the
//    sum of squares reduced by DPP within 16-lane rows and a 4-way add
//    across them, correctly rounded division and square root. The fused
//    forms share the helpers of the unfused ones, so fused = unfused.
//  - element-wise operators (saxpy, gathers, rope, element, pool): one
//    element per work-item, as the launch contract gives; GELU is the
//    tanh form with the host libm's tanhf restated (eg2_device.hpp).
//
// Launch contract (grid counted in workgroups, as the reference counts it):
//   eg2_saxpy, eg2_gather, eg2_rope, eg2_element, eg2_pool, eg2_gather768:
//       1-D, any workgroup size, one element per work-item
//   eg2_mm       256 work-items, grid (ceil(m/16), ceil(n/16))  16x16 tile
//   eg2_mm64     256 work-items, grid (ceil(m/64), ceil(n/16))  16x64 tile
//   eg2_mm64x64, eg2_mmstep8
//                256 work-items, grid (ceil(m/64), ceil(n/64))  64x64 tile
//   eg2_norm, eg2_norm_residual, eg2_norm_rope
//                one 64-wide wave per row, grid = rows
//   eg2_attention256, eg2_attention512
//                one wave per (token, query head), grid = 4n
//   eg2_attention256x3 (the 3 query / 1 KV head, d 256 variant)
//                one wave per (token, query head), grid = 3n
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "abi.h"
#include "eg2_device.hpp"

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ unsigned flat_index() { return threadIdx.x + blockIdx.x * blockDim.x; }

// Element i of a GGML-typed weight matrix (type 0 F32, 1 F16, 30 BF16,
// otherwise Q8_0: 34-byte blocks of a little-endian fp16 scale and 32 int8
// values, running over the flattened matrix), as fp32. The Q8_0 value
// fp16(d) * q is exact in fp32.
__device__ __forceinline__ float weight_at(const void* w, size_t i, unsigned type) {
  switch (type) {
    case 0:
      return static_cast<const float*>(w)[i];
    case 1:
      return eg2::fp16_bits_to_fp32(static_cast<const uint16_t*>(w)[i]);
    case 30:
      return __uint_as_float((uint32_t)static_cast<const uint16_t*>(w)[i] << 16);
    default: {
      const unsigned char* blk = static_cast<const unsigned char*>(w) + (i >> 5) * 34;
      const float d = eg2::fp16_bits_to_fp32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
      return d * (float)reinterpret_cast<const signed char*>(blk + 2)[i & 31];
    }
  }
}

// ------------------------------------------------------------ projections

constexpr int kSlice = 32;           // K values per LDS stage
constexpr int kPitch = kSlice + 4;   // floats per staged row

// out[n x m] = x[n x k] . W[m x k]^T for a TH x TW tile per 256-thread
// workgroup (4 waves).
template <int TH, int TW>
__device__ void mm_mfma(const EgMM& p) {
  static_assert((TH == 16 && (TW == 16 || TW == 64)) || (TH == 64 && TW == 64), "tile shapes of the contract");
  __shared__ __align__(16) float xs[TH * kPitch];
  __shared__ __align__(16) float ws[TW * kPitch];
  __shared__ __align__(16) floatx4 part[(TH == 16 && TW == 16) ? 3 * 64 : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const unsigned row0 = blockIdx.y * TH, col0 = blockIdx.x * TW;

  // Wave geometry: row blocks (16 rows) and column blocks (16 columns) it
  // owns, and the part of each slice it reads.
  constexpr bool kSplit = TH == 16 && TW == 16;  // the four waves split each slice
  constexpr int RB = TH == 64 ? 2 : 1, CB = TH == 64 ? 2 : 1;
  constexpr int KW = kSplit ? kSlice / 4 : kSlice;  // slice values per wave
  constexpr int PER = KW / 4;                       // values per lane group = MFMAs per slice
  const int rbase = TH == 64 ? 32 * (wave >> 1) : 0;
  const int cbase = TH == 64 ? 32 * (wave & 1) : (TW == 64 ? 16 * wave : 0);
  const int kbase = kSplit ? KW * wave : 0;

  floatx4 acc[RB][CB];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  for (unsigned base = 0; base < p.k; base += kSlice) {
    for (int idx = tid; idx < TH * kSlice; idx += 256) {
      const int rr = idx / kSlice, kk = idx % kSlice;
      const unsigned row = row0 + rr, kx = base + kk;
      xs[rr * kPitch + kk] = row < p.n && kx < p.k ? p.x[(size_t)row * p.k + kx] : 0.0f;
    }
    for (int idx = tid; idx < TW * kSlice; idx += 256) {
      const int cc = idx / kSlice, kk = idx % kSlice;
      const unsigned col = col0 + cc, kx = base + kk;
      ws[cc * kPitch + kk] = col < p.m && kx < p.k ? weight_at(p.weight, (size_t)col * p.k + kx, p.type) : 0.0f;
    }
    __syncthreads();
    float a[RB][PER], b[CB][PER];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
      for (int e = 0; e < PER; ++e) a[i][e] = xs[(rbase + 16 * i + r16) * kPitch + kbase + g * PER + e];
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int e = 0; e < PER; ++e) b[j][e] = ws[(cbase + 16 * j + r16) * kPitch + kbase + g * PER + e];
#pragma unroll
    for (int e = 0; e < PER; ++e)
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][e], b[j][e], acc[i][j], 0, 0, 0);
    __syncthreads();
  }

  if constexpr (kSplit) {
    // Waves 1-3 hand their partial tiles to wave 0, which adds them in order.
    if (wave > 0) part[(wave - 1) * 64 + lane] = acc[0][0];
    __syncthreads();
    if (wave > 0) return;
    acc[0][0] = ((acc[0][0] + part[lane]) + part[64 + lane]) + part[128 + lane];
  }
  // MFMA 16x16 output: lane holds rows 4g .. 4g + 3 of column r16.
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < CB; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const unsigned row = row0 + rbase + 16 * i + 4 * g + v, col = col0 + cbase + 16 * j + r16;
        if (row < p.n && col < p.m) p.out[(size_t)row * p.m + col] = acc[i][j][v];
      }
}

// -------------------------------------------------------------- row sums

// Sum over the 64 lanes: DPP exchanges within each 16-lane row (lanes
// i^1, i^2, then the mirrored half-row and row), then the four row totals
// added as (r0 + r1) + (r2 + r3). Wave-uniform result.
__device__ __forceinline__ float dpp_wave_sum(float v) {
  auto dpp = [](float x, int ctrl) -> float {
    switch (ctrl) {
      case 0:
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));  // quad [1,0,3,2]
      case 1:
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));  // quad [2,3,0,1]
      case 2:
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, false));  // row_half_mirror
      default:
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xF, 0xF, false));  // row_mirror
    }
  };
  v = v + dpp(v, 0);
  v = v + dpp(v, 1);
  v = v + dpp(v, 2);
  v = v + dpp(v, 3);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float dpp_wave_max(float v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// A row of d floats held by one wave: float4 chunks c = lane + 64 j
// (elements 4c .. 4c + 3) for j < kRowChunks when d % 4 == 0 and d <=
// 256 kRowChunks; other widths are read element-wise in two passes.
constexpr int kRowChunks = 4;

struct Row {
  floatx4 v[kRowChunks];
};

__device__ __forceinline__ bool row_in_registers(unsigned d) { return d % 4 == 0 && d <= 256u * kRowChunks; }

__device__ __forceinline__ Row load_row(const float* x, unsigned d, unsigned lane) {
  Row r;
#pragma unroll
  for (int j = 0; j < kRowChunks; ++j) {
    const unsigned c = lane + 64u * j;
    r.v[j] = 4 * c < d ? *reinterpret_cast<const floatx4*>(x + 4 * c) : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  return r;
}

// 1 / sqrt(mean((x * pre)^2) + 1e-6) of a row.
__device__ __forceinline__ float row_inverse_rms(const float* x, unsigned d, float pre, unsigned lane, const Row* r) {
  float ss = 0.0f;
  if (r) {
#pragma unroll
    for (int j = 0; j < kRowChunks; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = r->v[j][e] * pre;
        ss = __builtin_fmaf(v, v, ss);
      }
  } else {
    for (unsigned z = lane; z < d; z += 64) {
      const float v = x[z] * pre;
      ss = __builtin_fmaf(v, v, ss);
    }
  }
  return eg2::rms_inverse(dpp_wave_sum(ss), (int)d, 1.0e-6f);
}

// The normalized value of element z: ((x * pre) * inv) * w.
__device__ __forceinline__ float normed(float x, float pre, float inv, const float* w, unsigned z) {
  const float v = (x * pre) * inv;
  return w ? v * w[z] : v;
}

// NeoX rotation of the pair (a, b) by (c, s).
__device__ __forceinline__ void rotate(float a, float b, float c, float s, float& ra, float& rb) {
  const float ac = a * c, bs = b * s, as = a * s, bc = b * c;
  ra = ac - bs;
  rb = as + bc;
}

// --------------------------------------------------------------- attention

// One wave per (token t, query head h): out = softmax(q . K^T) V over the
// keys [bounds[2t], bounds[2t+1]) clipped to |t - s| <= window (window >
// 0). q rows of D floats per (t, h); K/V rows of KVS floats with head h's
// KV block at (h / GROUP) * D.
template <int D, int HEADS, int KVS, int GROUP>
__device__ void attention_chunked(const EgAttention& p) {
  static_assert(D % 256 == 0, "lanes own float4s of the context");
  constexpr int CV = D / 256;  // float4 of the context per lane
  __shared__ __align__(16) floatx4 qs[D / 4];
  __shared__ float ps[64];
  const unsigned row = blockIdx.x, lane = threadIdx.x;
  const unsigned t = row / HEADS, h = row % HEADS, kv = (h / GROUP) * D;
  if (t >= p.n) return;
  unsigned lo = p.bounds[2 * t], hi = p.bounds[2 * t + 1];
  if (p.window) {
    if (t > p.window) lo = max(lo, t - p.window);
    hi = min(hi, t + p.window + 1);
  }
  for (unsigned c = lane; c < D / 4; c += 64) qs[c] = reinterpret_cast<const floatx4*>(p.q + (size_t)row * D)[c];
  __syncthreads();
  float run_max = -__builtin_inff(), den = 0.0f;
  floatx4 acc[CV];
#pragma unroll
  for (int u = 0; u < CV; ++u) acc[u] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  for (unsigned c0 = lo; c0 < hi; c0 += 64) {
    const unsigned key = c0 + lane;
    float score = -__builtin_inff();
    if (key < hi) {
      const floatx4* kr = reinterpret_cast<const floatx4*>(p.k + (size_t)key * KVS + kv);
      floatx4 s4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
      for (int c = 0; c < D / 4; ++c) {
        const floatx4 k4 = kr[c], q4 = qs[c];
#pragma unroll
        for (int e = 0; e < 4; ++e) s4[e] = __builtin_fmaf(q4[e], k4[e], s4[e]);
      }
      score = (s4[0] + s4[1]) + (s4[2] + s4[3]);
    }
    const float next = fmaxf(run_max, dpp_wave_max(score));  // finite: the chunk has a key
    const float alpha = eg2::libm::expf(run_max - next);     // 0 for the first chunk
    const float pk = key < hi ? eg2::libm::expf(score - next) : 0.0f;
    den = den * alpha + dpp_wave_sum(pk);
    ps[lane] = pk;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < CV; ++u) acc[u] = acc[u] * alpha;
    const unsigned count = min(64u, hi - c0);
    const float* vbase = p.v + (size_t)c0 * KVS + kv + 4 * lane;
    for (unsigned j = 0; j < count; ++j) {
      const float w = ps[j];
#pragma unroll
      for (int u = 0; u < CV; ++u) {
        const floatx4 v4 = *reinterpret_cast<const floatx4*>(vbase + (size_t)j * KVS + 256 * u);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[u][e] = __builtin_fmaf(w, v4[e], acc[u][e]);
      }
    }
    __syncthreads();  // ps is rewritten by the next chunk
    run_max = next;
  }
  const float inv = hi > lo ? 1.0f / den : 0.0f;
#pragma unroll
  for (int u = 0; u < CV; ++u)
    *reinterpret_cast<floatx4*>(p.out + (size_t)row * D + 4 * lane + 256 * u) = acc[u] * inv;
}

}  // namespace

// y = a x + y.
extern "C" __global__ void eg2_saxpy(float* y, const float* x, float a, unsigned n) {
  const unsigned i = flat_index();
  if (i < n) y[i] = __builtin_fmaf(a, x[i], y[i]);
}

// Rows of 512 values of a Q8_0 table: (fp16(d) * q) * sqrt(512)
// (kernels/eg2.c:36-39 semantics).
extern "C" __global__ void eg2_gather(EgGather p) {
  const unsigned i = flat_index();
  if (i >= p.n * 512u) return;
  const unsigned r = i >> 9, z = i & 511;
  p.out[i] = weight_at(p.weight, (size_t)p.ids[r] * 512 + z, 8) * 22.62741699796952f;
}

// Rows of 768 values with the 768-wide CPU path's order (engine.c:288-295,
// quants.c:67,86-88): (fp16(d) * sqrt(768)) * q.
extern "C" __global__ void eg2_gather768(EgGather p) {
  const unsigned i = flat_index();
  if (i >= p.n * 768u) return;
  const unsigned r = i / 768u, z = i - 768u * r;
  const unsigned char* blk = static_cast<const unsigned char*>(p.weight) + ((size_t)p.ids[r] * 24 + z / 32) * 34;
  const float d = eg2::fp16_bits_to_fp32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
  p.out[i] = (d * 27.712812921102035f) * (float)reinterpret_cast<const signed char*>(blk + 2)[z & 31];
}

// kernels/eg2.c:41-119 semantics, four tile shapes.
extern "C" __global__ void __launch_bounds__(256) eg2_mm(EgMM p) { mm_mfma<16, 16>(p); }
extern "C" __global__ void __launch_bounds__(256) eg2_mm64(EgMM p) { mm_mfma<16, 64>(p); }
extern "C" __global__ void __launch_bounds__(256) eg2_mm64x64(EgMM p) { mm_mfma<64, 64>(p); }
extern "C" __global__ void __launch_bounds__(256) eg2_mmstep8(EgMM p) { mm_mfma<64, 64>(p); }

// out = ((x * scale) * inv) * w, inv = 1/sqrt(mean((x * scale)^2) + 1e-6);
// w may be NULL (= 1); out == x is valid (kernels/eg2.c:121-133 semantics).
extern "C" __global__ void __launch_bounds__(64) eg2_norm(EgNorm p) {
  const unsigned row = blockIdx.x, lane = threadIdx.x;
  if (row >= p.rows) return;
  const float* x = p.x + (size_t)row * p.d;
  float* out = p.out + (size_t)row * p.d;
  if (row_in_registers(p.d)) {
    const Row r = load_row(x, p.d, lane);
    const float inv = row_inverse_rms(x, p.d, p.scale, lane, &r);
#pragma unroll
    for (int j = 0; j < kRowChunks; ++j) {
      const unsigned c = lane + 64u * j;
      if (4 * c >= p.d) break;
      floatx4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = normed(r.v[j][e], p.scale, inv, p.weight, 4 * c + e);
      *reinterpret_cast<floatx4*>(out + 4 * c) = o;
    }
  } else {
    const float inv = row_inverse_rms(x, p.d, p.scale, lane, nullptr);
    for (unsigned z = lane; z < p.d; z += 64) out[z] = normed(x[z], p.scale, inv, p.weight, z);
  }
}

// NeoX rotation of pairs (z, z + d/2), table row of token row/heads =
// [cos(d/2) | sin(d/2)] (kernels/eg2.c:135-143 semantics).
extern "C" __global__ void eg2_rope(EgRope p) {
  const unsigned i = flat_index(), half = p.d / 2;
  if (i >= p.n * p.heads * half) return;
  const unsigned z = i % half, row = i / half, t = row / p.heads;
  const float* tab = p.table + (size_t)t * p.d;
  float* x = p.x + (size_t)row * p.d;
  rotate(x[z], x[half + z], tab[z], tab[half + z], x[z], x[half + z]);
}

// kernels/eg2.c:145-170 semantics: 4 query heads per token; d 256 reads KV
// head h/2 of two, d 512 the single KV head (K/V rows of 512 floats).
extern "C" __global__ void __launch_bounds__(64) eg2_attention256(EgAttention p) {
  attention_chunked<256, 4, 512, 2>(p);
}
extern "C" __global__ void __launch_bounds__(64) eg2_attention512(EgAttention p) {
  attention_chunked<512, 4, 512, 4>(p);
}
// 3 query heads sharing one KV head of 256 (K/V rows of 256 floats).
extern "C" __global__ void __launch_bounds__(64) eg2_attention256x3(EgAttention p) {
  attention_chunked<256, 3, 256, 3>(p);
}

// Mode 0: (x + other) * scale; 1: gelu(x) * other; 2: gelu(x) * the
// per-layer gate other[(i/512 * 24 + layer) * 512 + i % 512]
// (kernels/eg2.c:172-179 semantics). Both loads come before the mode
// branch: with the x load inside a three-way branch, hipcc (ROCm 7.2, -O3)
// left the mode-2 path's x address undefined.
extern "C" __global__ void eg2_element(EgElement p) {
  const unsigned i = flat_index();
  if (i >= p.n) return;
  const size_t o = p.mode == 2 ? ((size_t)(i >> 9) * 24 + p.layer) * 512 + (i & 511) : (size_t)i;
  const float xv = p.x[i], ov = p.other[o];
  p.out[i] = p.mode == 0 ? (xv + ov) * p.scale : eg2::gelu_mul(xv, ov);
}

// Mean over rows [offsets[s], offsets[s+1]) of width 768, in row order
// (kernels/eg2.c:181-188 semantics); four rows' loads in flight at a time.
extern "C" __global__ void eg2_pool(EgPool p) {
  const unsigned i = flat_index(), seq = i / 768u, z = i - 768u * seq;
  if (seq >= p.batch) return;
  const unsigned lo = p.offsets[seq], hi = p.offsets[seq + 1];
  const float* col = p.x + z;
  float sum = 0.0f;
  unsigned t = lo;
  for (; t + 4 <= hi; t += 4) {
    const float a = col[(size_t)t * 768], b = col[(size_t)(t + 1) * 768];
    const float c = col[(size_t)(t + 2) * 768], d = col[(size_t)(t + 3) * 768];
    sum = sum + a;
    sum = sum + b;
    sum = sum + c;
    sum = sum + d;
  }
  for (; t < hi; ++t) sum = sum + col[(size_t)t * 768];
  p.out[i] = sum / (float)(hi - lo);
}

// out = (out + (x * inv) * w) * scale (kernels/eg2.c:190-202 semantics):
// the normalized values of eg2_norm with scale 1, added to the residual.
extern "C" __global__ void __launch_bounds__(64) eg2_norm_residual(EgNormResidual p) {
  const unsigned row = blockIdx.x, lane = threadIdx.x;
  if (row >= p.rows) return;
  const float* x = p.x + (size_t)row * p.d;
  float* out = p.out + (size_t)row * p.d;
  if (row_in_registers(p.d)) {
    const Row r = load_row(x, p.d, lane);
    const float inv = row_inverse_rms(x, p.d, 1.0f, lane, &r);
#pragma unroll
    for (int j = 0; j < kRowChunks; ++j) {
      const unsigned c = lane + 64u * j;
      if (4 * c >= p.d) break;
      floatx4 o = *reinterpret_cast<const floatx4*>(out + 4 * c);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (o[e] + normed(r.v[j][e], 1.0f, inv, p.weight, 4 * c + e)) * p.scale;
      *reinterpret_cast<floatx4*>(out + 4 * c) = o;
    }
  } else {
    const float inv = row_inverse_rms(x, p.d, 1.0f, lane, nullptr);
    for (unsigned z = lane; z < p.d; z += 64) out[z] = (out[z] + normed(x[z], 1.0f, inv, p.weight, z)) * p.scale;
  }
}

// Per-row RMS with the row weight, then the NeoX rotation with the table
// row of token row/heads, in place (kernels/eg2.c:204-217 semantics): the
// normalized row goes through LDS so that each lane can take its pairs.
extern "C" __global__ void __launch_bounds__(64) eg2_norm_rope(EgNormRope p) {
  constexpr unsigned kMaxD = 4096;
  __shared__ float nrow[kMaxD];
  const unsigned row = blockIdx.x, lane = threadIdx.x, half = p.d / 2;
  if (row >= p.rows || p.d > kMaxD) return;
  float* x = p.x + (size_t)row * p.d;
  if (row_in_registers(p.d)) {
    const Row r = load_row(x, p.d, lane);
    const float inv = row_inverse_rms(x, p.d, 1.0f, lane, &r);
#pragma unroll
    for (int j = 0; j < kRowChunks; ++j) {
      const unsigned c = lane + 64u * j;
      if (4 * c >= p.d) break;
#pragma unroll
      for (int e = 0; e < 4; ++e) nrow[4 * c + e] = normed(r.v[j][e], 1.0f, inv, p.weight, 4 * c + e);
    }
  } else {
    const float inv = row_inverse_rms(x, p.d, 1.0f, lane, nullptr);
    for (unsigned z = lane; z < p.d; z += 64) nrow[z] = normed(x[z], 1.0f, inv, p.weight, z);
  }
  __syncthreads();
  const float* tab = p.table + (size_t)(row / p.heads) * p.d;
  for (unsigned z = lane; z < half; z += 64) rotate(nrow[z], nrow[half + z], tab[z], tab[half + z], x[z], x[half + z]);
}

// ---------------------------------------------------------------- dispatch

#include <cstring>

#include "eg2_ops.h"

namespace {

enum class Block { kAny, k64, k256 };

struct OpEntry {
  const char* name;
  const void* fn;
  size_t record_size;
  Block block;
  bool (*valid)(const void* record);
};

template <class R>
const R& as(const void* r) {
  return *static_cast<const R*>(r);
}

bool valid_saxpy(const void* r) { return as<EgSaxpy>(r).y && as<EgSaxpy>(r).x; }
bool valid_gather(const void* r) { return as<EgGather>(r).out && as<EgGather>(r).weight && as<EgGather>(r).ids; }
bool valid_mm(const void* r) {
  const EgMM& p = as<EgMM>(r);
  return p.out && p.x && p.weight && (p.type == 0 || p.type == 1 || p.type == 8 || p.type == 30);
}
bool valid_norm(const void* r) { return as<EgNorm>(r).out && as<EgNorm>(r).x && as<EgNorm>(r).d > 0; }
bool valid_rope(const void* r) {
  const EgRope& p = as<EgRope>(r);
  return p.x && p.table && p.d > 0 && p.d % 2 == 0;
}
bool valid_attention(const void* r) {
  const EgAttention& p = as<EgAttention>(r);
  return p.out && p.q && p.k && p.v && p.bounds;
}
bool valid_element(const void* r) {
  const EgElement& p = as<EgElement>(r);
  return p.out && p.x && p.other && p.mode <= 2;
}
bool valid_pool(const void* r) { return as<EgPool>(r).out && as<EgPool>(r).x && as<EgPool>(r).offsets; }
bool valid_norm_residual(const void* r) {
  const EgNormResidual& p = as<EgNormResidual>(r);
  return p.out && p.x && p.weight && p.d > 0;
}
bool valid_norm_rope(const void* r) {
  const EgNormRope& p = as<EgNormRope>(r);
  return p.x && p.weight && p.table && p.d > 0 && p.d % 2 == 0 && p.d <= 4096 && p.heads > 0;
}

const OpEntry kOps[] = {
    {"eg2_saxpy", reinterpret_cast<const void*>(&eg2_saxpy), sizeof(EgSaxpy), Block::kAny, valid_saxpy},
    {"eg2_gather", reinterpret_cast<const void*>(&eg2_gather), sizeof(EgGather), Block::kAny, valid_gather},
    {"eg2_gather768", reinterpret_cast<const void*>(&eg2_gather768), sizeof(EgGather), Block::kAny, valid_gather},
    {"eg2_mm", reinterpret_cast<const void*>(&eg2_mm), sizeof(EgMM), Block::k256, valid_mm},
    {"eg2_mm64", reinterpret_cast<const void*>(&eg2_mm64), sizeof(EgMM), Block::k256, valid_mm},
    {"eg2_mm64x64", reinterpret_cast<const void*>(&eg2_mm64x64), sizeof(EgMM), Block::k256, valid_mm},
    {"eg2_mmstep8", reinterpret_cast<const void*>(&eg2_mmstep8), sizeof(EgMM), Block::k256, valid_mm},
    {"eg2_norm", reinterpret_cast<const void*>(&eg2_norm), sizeof(EgNorm), Block::k64, valid_norm},
    {"eg2_rope", reinterpret_cast<const void*>(&eg2_rope), sizeof(EgRope), Block::kAny, valid_rope},
    {"eg2_attention256", reinterpret_cast<const void*>(&eg2_attention256), sizeof(EgAttention), Block::k64,
     valid_attention},
    {"eg2_attention512", reinterpret_cast<const void*>(&eg2_attention512), sizeof(EgAttention), Block::k64,
     valid_attention},
    {"eg2_attention256x3", reinterpret_cast<const void*>(&eg2_attention256x3), sizeof(EgAttention), Block::k64,
     valid_attention},
    {"eg2_element", reinterpret_cast<const void*>(&eg2_element), sizeof(EgElement), Block::kAny, valid_element},
    {"eg2_pool", reinterpret_cast<const void*>(&eg2_pool), sizeof(EgPool), Block::kAny, valid_pool},
    {"eg2_norm_residual", reinterpret_cast<const void*>(&eg2_norm_residual), sizeof(EgNormResidual), Block::k64,
     valid_norm_residual},
    {"eg2_norm_rope", reinterpret_cast<const void*>(&eg2_norm_rope), sizeof(EgNormRope), Block::k64,
     valid_norm_rope},
};
constexpr unsigned kOpCount = sizeof(kOps) / sizeof(kOps[0]);

}  // namespace

extern "C" int eg2_op_launch(const char* name, const void* record, size_t record_size, unsigned grid_x,
                             unsigned grid_y, unsigned block, void* stream) {
  if (!name || !record || grid_x == 0 || grid_y == 0 || block == 0 || block > 1024) return (int)hipErrorInvalidValue;
  for (const OpEntry& op : kOps) {
    if (std::strcmp(op.name, name) != 0) continue;
    if (record_size != op.record_size) return (int)hipErrorInvalidValue;
    if ((op.block == Block::k64 && block != 64) || (op.block == Block::k256 && block != 256))
      return (int)hipErrorInvalidValue;
    if (!op.valid(record)) return (int)hipErrorInvalidValue;
    // The kernarg segment is the record itself: copy it so the caller's
    // buffer may be reused as soon as this returns.
    alignas(16) unsigned char kernarg[64];
    std::memcpy(kernarg, record, record_size);
    if (op.fn == reinterpret_cast<const void*>(&eg2_saxpy)) {
      EgSaxpy s;
      std::memcpy(&s, kernarg, sizeof(s));
      void* args[] = {&s.y, &s.x, &s.a, &s.n};
      return (int)hipLaunchKernel(op.fn, dim3(grid_x, grid_y), dim3(block), args, 0,
                                  reinterpret_cast<hipStream_t>(stream));
    }
    void* args[] = {kernarg};
    return (int)hipLaunchKernel(op.fn, dim3(grid_x, grid_y), dim3(block), args, 0,
                                reinterpret_cast<hipStream_t>(stream));
  }
  return (int)hipErrorInvalidValue;
}

extern "C" unsigned eg2_op_count(void) { return kOpCount; }

extern "C" const char* eg2_op_name(unsigned index) { return index < kOpCount ? kOps[index].name : nullptr; }
