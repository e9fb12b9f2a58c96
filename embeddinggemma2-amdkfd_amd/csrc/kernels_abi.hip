// The reference's operator set (kernels/abi.h records, kernels/eg2.c kernel
// names and launch geometry) as gfx950 kernels.
//
// Each kernel takes its record by value, so its kernarg segment has the
// record's layout and a code object built from this file can be dispatched
// by symbol name ("eg2_mm.kd", ...) with the same records, grids and
// workgroup sizes the reference executor uses (src/gemma2_kfd.cpp:160-165,
// 248-336) and its operator test uses (tests/kernels.cpp:36-137).
//
// Per output element the arithmetic is the reference kernel's: the same
// operations in the same order with the same roundings, including the fused
// multiply-adds its compiler forms under the default -ffp-contract=on
// (written out here as fmaf), the hardware v_rsq_f32 / v_exp_f32 the
// reference calls through __builtin_amdgcn_rsqf / exp2f, correctly rounded
// division, and the xor-butterfly wave sum. The projection kernels add the
// same zero padding of the K loop (k rounded up to the variant's step).
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

namespace {

constexpr unsigned kWave = 64;

__device__ __forceinline__ unsigned flat_index() { return threadIdx.x + blockIdx.x * blockDim.x; }

// GGML element decode of the reference's weight() (kernels/eg2.c:9-17):
// 1 F16, 0 F32, 30 BF16; every other id is read as Q8_0 (34-byte blocks of a
// little-endian fp16 scale and 32 int8 values, blocks running over the
// flattened matrix). The Q8_0 product fp16(d) * q is exact in fp32.
__device__ __forceinline__ float decode_weight(const void* w, unsigned i, unsigned type) {
  if (type == 1) return (float)static_cast<const _Float16*>(w)[i];
  if (type == 0) return static_cast<const float*>(w)[i];
  if (type == 30) return __uint_as_float((uint32_t)static_cast<const uint16_t*>(w)[i] << 16);
  const unsigned char* b = static_cast<const unsigned char*>(w) + (size_t)(i / 32) * 34;
  const uint16_t bits = (uint16_t)(b[0] | (b[1] << 8));
  const float d = (float)__builtin_bit_cast(_Float16, bits);
  return d * (float)(int)reinterpret_cast<const signed char*>(b + 2)[i % 32];
}

// Xor-butterfly sum over the 64 lanes; every lane ends with the same value.
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int s = kWave / 2; s > 0; s >>= 1) x = x + __shfl_xor(x, s, kWave);
  return x;
}

__device__ __forceinline__ float exp_e(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// gelu_tanh as x / (1 + e^(-2u)), u = sqrt(2/pi) (x + 0.044715 x^3)
// (kernels/eg2.c:25-29); the inner x + c*x*x*x is one fused multiply-add.
__device__ __forceinline__ float gelu_exp(float x) {
  const float cube = (0.044715f * x) * x;
  const float u = 0.7978845608028654f * fmaf(cube, x, x);
  return x / (1.0f + exp_e(-2.0f * u));
}

// Sum of squares of row[lane + 64 j] * pre (pre = 1: the raw values), one
// fused multiply-add per term when FUSED, then the wave sum.
template <bool FUSED>
__device__ __forceinline__ float row_sum_squares(const float* row, unsigned d, float pre, unsigned lane) {
  float ss = 0.0f;
  for (unsigned z = lane; z < d; z += kWave) {
    const float v = row[z] * pre;
    if constexpr (FUSED) {
      ss = fmaf(v, v, ss);
    } else {
      const float sq = v * v;
      ss = ss + sq;
    }
  }
  return wave_sum(ss);
}

__device__ __forceinline__ float rms_inverse(float ss, unsigned d) {
  return __builtin_amdgcn_rsqf(ss / (float)d + 1.0e-6f);
}

// Projection tile: TH x TW outputs per 256-thread workgroup, K staged
// through LDS STEP columns at a time (zero-padded past k, as the reference
// variants pad). Each output accumulates fmaf(x, w, acc) in ascending k.
template <int TH, int TW, int STEP>
__device__ void mm_tile(const EgMM& p) {
  constexpr int RI = TH / 16, CJ = TW / 16;
  __shared__ float xs[TH][STEP + 1];
  __shared__ float ws[TW][STEP + 1];
  const unsigned tid = threadIdx.x, r = tid / 16, c = tid % 16;
  const unsigned row0 = blockIdx.y * TH, col0 = blockIdx.x * TW;
  float acc[RI][CJ];
#pragma unroll
  for (int i = 0; i < RI; ++i)
#pragma unroll
    for (int j = 0; j < CJ; ++j) acc[i][j] = 0.0f;
  for (unsigned base = 0; base < p.k; base += STEP) {
    for (unsigned idx = tid; idx < (unsigned)(TH * STEP); idx += 256) {
      const unsigned rr = idx / STEP, kk = idx % STEP, row = row0 + rr;
      xs[rr][kk] = row < p.n && base + kk < p.k ? p.x[(size_t)row * p.k + base + kk] : 0.0f;
    }
    for (unsigned idx = tid; idx < (unsigned)(TW * STEP); idx += 256) {
      const unsigned cc = idx / STEP, kk = idx % STEP, col = col0 + cc;
      ws[cc][kk] = col < p.m && base + kk < p.k ? decode_weight(p.weight, col * p.k + base + kk, p.type) : 0.0f;
    }
    __syncthreads();
#pragma unroll 4
    for (int j = 0; j < STEP; ++j) {
#pragma unroll
      for (int i = 0; i < RI; ++i) {
        const float xv = xs[r + 16 * i][j];
#pragma unroll
        for (int o = 0; o < CJ; ++o) acc[i][o] = fmaf(xv, ws[c + 16 * o][j], acc[i][o]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < RI; ++i)
#pragma unroll
    for (int o = 0; o < CJ; ++o) {
      const unsigned row = row0 + r + 16 * i, col = col0 + c + 16 * o;
      if (row < p.n && col < p.m) p.out[(size_t)row * p.m + col] = acc[i][o];
    }
}

// Streaming-softmax attention of one (token, query head) per wave
// (kernels/eg2.c:145-170): keys [bounds[2t], bounds[2t+1]) clipped to
// |t - s| <= window when window > 0; q row stride D, K/V row stride KV_STRIDE
// with the head's KV block at kh * D. Lane owns elements lane + 64 j.
template <int D, int HEADS, int KV_STRIDE>
__device__ void attention_row(const EgAttention& p, unsigned kh_div) {
  constexpr int J = D / kWave;
  const unsigned row = blockIdx.x, lane = threadIdx.x;
  const unsigned t = row / HEADS, h = row % HEADS, kh = h / kh_div;
  if (t >= p.n) return;
  unsigned lo = p.bounds[2 * t], hi = p.bounds[2 * t + 1];
  if (p.window && t > p.window && lo < t - p.window) lo = t - p.window;
  if (p.window && hi > t + p.window + 1) hi = t + p.window + 1;
  float q[J], acc[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    q[j] = p.q[(size_t)row * D + lane + j * kWave];
    acc[j] = 0.0f;
  }
  float run_max = -__builtin_inff(), den = 0.0f;
  for (unsigned s = lo; s < hi; ++s) {
    const float* krow = p.k + (size_t)s * KV_STRIDE + kh * D;
    const float* vrow = p.v + (size_t)s * KV_STRIDE + kh * D;
    float vv[J];
    float dot = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      dot = fmaf(q[j], krow[lane + j * kWave], dot);
      vv[j] = vrow[lane + j * kWave];
    }
    dot = wave_sum(dot);
    const float next = fmaxf(run_max, dot);
    const float alpha = exp_e(run_max - next), beta = exp_e(dot - next);
    den = fmaf(den, alpha, beta);
#pragma unroll
    for (int j = 0; j < J; ++j) acc[j] = fmaf(acc[j], alpha, beta * vv[j]);
    run_max = next;
  }
#pragma unroll
  for (int j = 0; j < J; ++j) p.out[(size_t)row * D + lane + j * kWave] = acc[j] / den;
}

}  // namespace

// kernels/eg2.c:31-34: y = a*x + y (one fused multiply-add).
extern "C" __global__ void eg2_saxpy(float* y, const float* x, float a, unsigned n) {
  const unsigned i = flat_index();
  if (i < n) y[i] = fmaf(a, x[i], y[i]);
}

// kernels/eg2.c:36-39: rows of 512 values, (fp16(d) * q) * sqrt(512).
extern "C" __global__ void eg2_gather(EgGather p) {
  const unsigned i = flat_index();
  if (i < p.n * 512u) p.out[i] = decode_weight(p.weight, (unsigned)p.ids[i / 512] * 512u + i % 512, 8) * 22.62741699796952f;
}

// Width-768 gather with the order of the 768-wide CPU path
// (engine.c:288-295, quants.c:67,86-88): (fp16(d) * sqrt(768)) * q.
extern "C" __global__ void eg2_gather768(EgGather p) {
  const unsigned i = flat_index();
  if (i >= p.n * 768u) return;
  const unsigned e = (unsigned)p.ids[i / 768] * 768u + i % 768;
  const unsigned char* b = static_cast<const unsigned char*>(p.weight) + (size_t)(e / 32) * 34;
  const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(b[0] | (b[1] << 8)));
  p.out[i] = (d * 27.712812921102035f) * (float)(int)reinterpret_cast<const signed char*>(b + 2)[e % 32];
}

// kernels/eg2.c:41-119: out[n x m] = x[n x k] . W[m x k]^T, four tilings.
extern "C" __global__ void __launch_bounds__(256) eg2_mm(EgMM p) { mm_tile<16, 16, 16>(p); }
extern "C" __global__ void __launch_bounds__(256) eg2_mm64(EgMM p) { mm_tile<16, 64, 32>(p); }
extern "C" __global__ void __launch_bounds__(256) eg2_mm64x64(EgMM p) { mm_tile<64, 64, 32>(p); }
extern "C" __global__ void __launch_bounds__(256) eg2_mmstep8(EgMM p) { mm_tile<64, 64, 8>(p); }

// kernels/eg2.c:121-133: out = ((x*scale) * inv) * w, inv = rsq(mean((x*scale)^2) + 1e-6);
// weight may be NULL (= 1). In place (out == x) is valid.
extern "C" __global__ void __launch_bounds__(64) eg2_norm(EgNorm p) {
  const unsigned row = blockIdx.x, lane = threadIdx.x;
  if (row >= p.rows) return;
  const float* x = p.x + (size_t)row * p.d;
  const float inv = rms_inverse(row_sum_squares<true>(x, p.d, p.scale, lane), p.d);
  for (unsigned z = lane; z < p.d; z += kWave) {
    const float v = (x[z] * p.scale) * inv;
    p.out[(size_t)row * p.d + z] = v * (p.weight ? p.weight[z] : 1.0f);
  }
}

// kernels/eg2.c:135-143: NeoX rotation of pairs (z, z + d/2) with the table
// row of token row/heads = [cos(d/2) | sin(d/2)].
extern "C" __global__ void eg2_rope(EgRope p) {
  const unsigned i = flat_index(), half = p.d / 2;
  if (i >= p.n * p.heads * half) return;
  const unsigned z = i % half, row = i / half, t = row / p.heads;
  const float c = p.table[(size_t)t * p.d + z], s = p.table[(size_t)t * p.d + half + z];
  float* x = p.x + (size_t)row * p.d;
  const float a = x[z], b = x[half + z];
  x[z] = fmaf(a, c, -(b * s));
  x[half + z] = fmaf(a, s, b * c);
}

// kernels/eg2.c:145-170: 4 query heads per token; d 256 reads KV head h/2
// of two, d 512 the single KV head (K/V rows of 512 floats).
extern "C" __global__ void __launch_bounds__(64) eg2_attention256(EgAttention p) { attention_row<256, 4, 512>(p, 2); }
extern "C" __global__ void __launch_bounds__(64) eg2_attention512(EgAttention p) { attention_row<512, 4, 512>(p, 4); }
// 3 query heads sharing one KV head of 256 (K/V rows of 256 floats).
extern "C" __global__ void __launch_bounds__(64) eg2_attention256x3(EgAttention p) { attention_row<256, 3, 256>(p, 3); }

// kernels/eg2.c:172-179: mode 0 (x + other) * scale, 1 gelu(x) * other,
// 2 gelu(x) * other[(i/512*24 + layer)*512 + i%512].
extern "C" __global__ void eg2_element(EgElement p) {
  const unsigned i = flat_index();
  if (i >= p.n) return;
  if (p.mode == 0) {
    p.out[i] = (p.x[i] + p.other[i]) * p.scale;
  } else if (p.mode == 1) {
    p.out[i] = gelu_exp(p.x[i]) * p.other[i];
  } else {
    p.out[i] = gelu_exp(p.x[i]) * p.other[((size_t)(i / 512) * 24 + p.layer) * 512 + i % 512];
  }
}

// kernels/eg2.c:181-188: mean over rows [offsets[s], offsets[s+1]) of width 768.
extern "C" __global__ void eg2_pool(EgPool p) {
  const unsigned i = flat_index(), seq = i / 768, z = i % 768;
  if (seq >= p.batch) return;
  const unsigned lo = p.offsets[seq], hi = p.offsets[seq + 1];
  float sum = 0.0f;
  for (unsigned t = lo; t < hi; ++t) sum = sum + p.x[(size_t)t * 768 + z];
  p.out[i] = sum / (float)(hi - lo);
}

// kernels/eg2.c:190-202: out = (out + (x*inv)*w) * scale, no fused operations.
extern "C" __global__ void __launch_bounds__(64) eg2_norm_residual(EgNormResidual p) {
  const unsigned row = blockIdx.x, lane = threadIdx.x;
  if (row >= p.rows) return;
  const float* x = p.x + (size_t)row * p.d;
  const float inv = rms_inverse(row_sum_squares<false>(x, p.d, 1.0f, lane), p.d);
  for (unsigned z = lane; z < p.d; z += kWave) {
    const size_t i = (size_t)row * p.d + z;
    const float nv = (x[z] * inv) * p.weight[z];
    p.out[i] = (p.out[i] + nv) * p.scale;
  }
}

// kernels/eg2.c:204-217: per-row RMS with the row weight, then the NeoX
// rotation with the table row of token row/heads; in place.
extern "C" __global__ void __launch_bounds__(64) eg2_norm_rope(EgNormRope p) {
  const unsigned row = blockIdx.x, lane = threadIdx.x, half = p.d / 2;
  if (row >= p.rows) return;
  float* x = p.x + (size_t)row * p.d;
  const float inv = rms_inverse(row_sum_squares<true>(x, p.d, 1.0f, lane), p.d);
  const unsigned t = row / p.heads;
  for (unsigned z = lane; z < half; z += kWave) {
    const float a = (x[z] * inv) * p.weight[z];
    const float b = (x[half + z] * inv) * p.weight[half + z];
    const float c = p.table[(size_t)t * p.d + z], s = p.table[(size_t)t * p.d + half + z];
    x[z] = fmaf(a, c, -(b * s));
    x[half + z] = fmaf(a, s, b * c);
  }
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
  return p.x && p.weight && p.table && p.d > 0 && p.d % 2 == 0 && p.heads > 0;
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
