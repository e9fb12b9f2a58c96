// Device-side helpers shared by the gfx950 kernels.
//
// Every kernel is compiled with -ffp-contract=off and without fast-math, so a
// float expression is evaluated in the order written with one rounding per
// operation; where an operation order below mirrors a reference function it
// says which (paths relative to vendor/embeddinggemma.c/src/).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "eg2_libm.hpp"

namespace eg2 {

constexpr int kEmbd = 768;      // model.h:9
constexpr int kFF = 1152;       // model.h:10
constexpr int kHeads = 3;       // model.h:11
constexpr int kHeadDim = 256;   // model.h:13
constexpr int kCtx = 2048;      // model.h:14 and the executor's wave cap
constexpr int kVocab = 262144;  // model.h:15
constexpr int kQK = 32;         // Q8_0 block length (quants.h:6)
constexpr int kQKVCols = kEmbd + 2 * kHeadDim;  // fused Q|K|V projection width
constexpr int kDenseFF = 3072;                  // dense head hidden width

// Q8_0 values of activations and weights are stored as int8 "row tiles",
// [rows/32][k/32][2][32][16]: each block of 32 rows x 32 values is 1 KB in
// the register order of the int8 MFMA operand. Byte offset of value e of
// row r in a buffer with nb = k/32 blocks per row (rows padded to 32).
__host__ __device__ inline size_t q8_tile_offset(size_t r, unsigned e, unsigned nb) {
  return (((r >> 5) * nb + (e >> 5)) * 2 + ((e >> 4) & 1)) * 512 + (r & 31) * 16 + (e & 15);
}

// LDS DMA from a wave-uniform global base (SGPR pair) plus a per-lane byte
// offset, 16 bytes per lane, to the wave-uniform LDS address `lds` (+16
// bytes per lane), which the instruction takes from M0 (the attention
// kernels' staging). Written
// as asm, not as __builtin_amdgcn_global_load_lds: with this compiler (ROCm
// 7.2 clang) the builtin's write to LDS is invisible to the optimizer, which
// then folded away a later read of the same LDS words in a test kernel.
// The asm declares M0 clobbered (the compiler warns that M0 is reserved):
// nothing in the kernels that call these uses M0 otherwise (their LDS
// accesses are plain ds_read/ds_write and ds_bpermute, which need no M0 on
// gfx950), so the value this code leaves there is never read by
// compiler-generated code; a test compiles them and checks the ISA. A
// kernel that adds an M0 user (s_movrels, LDS-direct, GWS) must not call
// these. The DMA is not tracked by the compiler: callers wait for it with
// s_waitcnt vmcnt and a barrier of their own before reading the LDS.
__device__ __forceinline__ void dma16(const void* base, unsigned off, unsigned lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
               : "memory", "m0");
}

// A raw buffer resource over `bytes` bytes from `base` (gfx9 descriptor:
// stride 0, word 3 = 0x00020000, 32-bit data format). Loads through it take
// a per-lane offset and a scalar one, so a loop's advance costs no vector
// registers; offsets at or past `bytes` read 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Four int8 values (low byte of each) in one little-endian word.
__device__ __forceinline__ uint32_t pack_i8x4(int32_t a, int32_t b, int32_t c, int32_t d) {
  return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
         ((uint32_t)(d & 0xff) << 24);
}

// fp32 -> fp16 bits with the reference's rounding (quants.c:13-37): the
// dropped mantissa bits round half-up in magnitude (not to nearest-even),
// and any value of 2^16 or more with a nonzero mantissa maps to a NaN.
// Written without branches (every case computed, one selected) so that it
// costs a few VALU operations inside quantizing epilogues; identical to the
// branching form for all 2^32 inputs.
__host__ __device__ inline uint32_t fp32_to_fp16_bits(float f) {
#ifdef __HIP_DEVICE_COMPILE__
  const uint32_t x = __float_as_uint(f);
#else
  uint32_t x;
  __builtin_memcpy(&x, &f, 4);
#endif
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t mant = x & 0x007FFFFFu;
  const int32_t e = (int32_t)((x >> 23) & 0xFFu) - 127 + 15;
  // normal: the rounding carry may step into the exponent (up to 0x7C00)
  const uint32_t normal = (((uint32_t)e << 10) | (mant >> 13)) + ((mant >> 12) & 1u);
  // subnormal (-10 <= e <= 0): shift 14 - e in [14, 24]
  const uint32_t m = mant | 0x00800000u;
  const uint32_t sh = (uint32_t)(14 - (e < -10 ? -10 : (e > 0 ? 0 : e)));
  const uint32_t sub = (m >> sh) + ((m >> (sh - 1u)) & 1u);
  const uint32_t big = 0x7C00u | (mant ? ((mant >> 13) | 1u) : 0u);
  const uint32_t mag = e >= 31 ? big : (e > 0 ? normal : (e >= -10 ? sub : 0u));
  return sign | mag;
}

// Exact fp16 bits -> fp32 (common.h:17-40); the hardware conversion is exact
// for every fp16 value including subnormals.
__device__ __forceinline__ float fp16_bits_to_fp32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// The Q8_0 scale amax / 127 (quants.c:97-177), correctly rounded like the
// IEEE division, in three instructions: q = amax * RN(1/127), then one FMA
// correction with the exact remainder amax - 127 q. Equal to amax / 127.0f
// for every non-negative finite float (checked over all of them).
__device__ __forceinline__ float div127(float amax) {
  constexpr float r = 1.0f / 127.0f;
  const float q = amax * r;
  return __builtin_fmaf(__builtin_fmaf(-q, 127.0f, amax), r, q);
}

// Round-half-away-from-zero like C roundf, clamped to int8 (quants.c:169-174).
// roundf(v) == truncf(v + copysignf(0.5 - 2^-25, v)) for every finite float
// (checked over all 2^32 bit patterns): adding the largest float below 0.5
// carries into the next integer exactly when |frac(v)| >= 0.5, and the
// conversion truncates (saturating; NaN converts to 0). Four VALU
// instructions instead of the eight of truncf/compare/select.
__device__ __forceinline__ int32_t q8_round(float v) {
  int32_t q = (int32_t)(v + __builtin_copysignf(0x1.fffffep-2f, v));
  q = q < -128 ? -128 : q;
  q = q > 127 ? 127 : q;
  return q;
}

// The quantized value q = (int)roundf(v * id), clamped (quants.c:169-174),
// including the x86 conversion the reference runs on: cvttss2si turns NaN
// and out-of-range values into INT_MIN, which the clamp makes -128. Within a
// block that only happens when 1 / d overflows (d = amax / 127 below 2^-128,
// a block of subnormal-sized values), where every v * id is +-inf or, for
// v = 0, NaN: every value of such a block quantizes to -128.
__device__ __forceinline__ int32_t q8_value(float v, float id) {
  return id > 3.40282347e38f ? -128 : q8_round(v * id);
}

// v combined (op: max or +) with its copies in lanes l ^ 16 and l ^ 32,
// i.e. over the four 16-lane rows, on the VALU: v_permlane16_swap and
// v_permlane32_swap of v with itself leave v of lane l and of its partner in
// the two results (in an order that differs between the rows, so op must
// be commutative; + of two floats is). Same values as two __shfl_xor steps
// (16, then 32) without the LDS round trips.
template <typename Op>
__device__ __forceinline__ float rows4_reduce(float v, Op op) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = op(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return op(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows4_max(float v) {
  return rows4_reduce(v, [](float x, float y) { return fmaxf(x, y); });
}
__device__ __forceinline__ float rows4_sum(float v) {
  return rows4_reduce(v, [](float x, float y) { return x + y; });
}

// Max over the 32 lanes of each half-wave (lanes 0-31 and 32-63 separately).
__device__ __forceinline__ float half_wave_max(float v) {
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// Quantizes one Q8_0 block whose 32 values sit one per lane in a half-wave
// (quants.c:97-177, scalar path). Every lane of the half-wave receives the
// block's stored scale (as the float value of its fp16) and its own int8.
struct Q8Lane {
  float d;
  int32_t q;
};
__device__ __forceinline__ Q8Lane q8_quantize_lane(float x) {
  const float amax = half_wave_max(fabsf(x));
  const float d = div127(amax);
  Q8Lane r;
  r.d = fp16_bits_to_fp32(fp32_to_fp16_bits(d));
  if (amax == 0.0f) {
    r.q = 0;
  } else {
    const float id = 1.0f / d;
    r.q = q8_value(x, id);
  }
  return r;
}

// quants.c:97-177 (scalar path) on one block spread over P adjacent lanes
// (lanes P*i .. P*i+P-1, all active), each holding N = 32/P consecutive
// values: amax, d = amax/127 stored as fp16 (round-half-up), id = 1/d,
// q = roundf(v*id) clamped; an all-zero block stores d = 0 and q = 0. Each
// lane writes its N int8 values at q (N-byte aligned, consecutive in the
// row-tile layout since N <= 16); the first lane of the group writes the
// float value of the stored scale.
template <int P>
__device__ __forceinline__ void quantize_block_part(const float (&v)[kQK / P], bool store, int8_t* __restrict__ q,
                                                    float* __restrict__ d_out) {
  constexpr int N = kQK / P;
  static_assert(N == 8 || N == 16, "8 or 16 values per lane");
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
  for (int m = 1; m < P; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
  const float d = div127(amax);
  const float id = amax != 0.0f ? 1.0f / d : 0.0f;
  if (!store) return;
  if ((threadIdx.x & (P - 1)) == 0) *d_out = fp16_bits_to_fp32(fp32_to_fp16_bits(d));
  int32_t qi[N];
#pragma unroll
  for (int i = 0; i < N; ++i) qi[i] = q8_value(v[i], id);  // id = 0 for an all-zero block
  uint32_t w[N / 4];
#pragma unroll
  for (int i = 0; i < N / 4; ++i) w[i] = pack_i8x4(qi[4 * i], qi[4 * i + 1], qi[4 * i + 2], qi[4 * i + 3]);
  if constexpr (N == 16)
    *reinterpret_cast<uint4*>(q) = make_uint4(w[0], w[1], w[2], w[3]);
  else
    *reinterpret_cast<uint2*>(q) = make_uint2(w[0], w[1]);
}

// kernels.c:367-371 gelu_tanh(g) = 0.5 g (1 + tanhf(z)), z = s g (1 + a g^2),
// times u (engine.c's GeGLU), each operation in the reference's order with
// the host libm's own tanhf (eg2_libm.hpp, its branch-free form, since the
// lanes of a wave take different cases): bit-identical to the CPU path.
constexpr float kGeluA = 0.044715f;
constexpr float kGeluS = 0.79788456080286535587989211986876f;
__device__ __forceinline__ float gelu_inner(float g) { return kGeluS * g * (1.0f + kGeluA * g * g); }
__device__ __forceinline__ float gelu_mul(float g, float u) {
  return 0.5f * g * (1.0f + libm::tanhf_flat(gelu_inner(g))) * u;
}

// A cheap tanh: 1 - 2 / (1 + 2^(2x log2 e)) by the hardware exp2 and
// reciprocal. |tanh_approx(x) - tanhf(x)| <= 2^-22 for every finite float x,
// tanhf being the host libm's (as restated in eg2_libm.hpp): the maximum over
// all 2^32 inputs, measured on the device (4 units of 2^-24, at x =
// -1.87318516); a GPU test repeats the exhaustive check against
// kTanhApproxBound, twice that.
__device__ __forceinline__ float tanh_approx(float x) {
  const float e = __builtin_amdgcn_exp2f(x * 2.8853900817779268f);
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + e);
}
constexpr float kTanhApproxBound = 0x1p-21f;

// Maximum over each aligned quad of lanes (4i .. 4i+3), on every lane of it,
// by two DPP quad permutations (all 64 lanes must be active).
__device__ __forceinline__ float quad_max(float m) {
  m = fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, m), 0xB1, 0xf, 0xf, true)));
  return fmaxf(m, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, m), 0x4E, 0xf, 0xf, true)));
}

// Exact GeGLU values (gelu_mul) of the pending values of each lane (bit i of
// pending = value i), one per pass over the wave, as many passes as the lane
// with the most. Q = false stores them in a[]; Q = true stores their
// quantized values q8_value(., id) in qi[].
template <bool Q>
__device__ __forceinline__ void geglu_exact_passes(const float (&g)[8], const float (&u)[8], uint32_t pending, float id,
                                                   float (&a)[8], int32_t (&qi)[8]) {
  while (__ballot(pending != 0)) {
    const int k = pending ? __builtin_ctz(pending) : 0;
    float gk = g[0], uk = u[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) {
      gk = k == i ? g[i] : gk;
      uk = k == i ? u[i] : uk;
    }
    const float x = gelu_mul(gk, uk);
    if constexpr (Q) {
      const int32_t qx = q8_value(x, id);
#pragma unroll
      for (int i = 0; i < 8; ++i) qi[i] = (pending & (1u << i)) && k == i ? qx : qi[i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = (pending & (1u << i)) && k == i ? x : a[i];
    }
    pending &= pending - 1;
  }
}

// The GeGLU of one 32-value block and its Q8_0 quantization (quants.c:97-177,
// scalar path), the block spread over 4 adjacent lanes with 8 (gate, up)
// pairs each, with the results of gelu_mul then quantize_block_part<4> bit
// for bit but without evaluating the exact tanhf for most values:
//  1. A = ((0.5 g)(1 + tanh_approx(z))) u for each value, and a bound B on
//     |A - gelu_mul(g, u)|: with |tanh_approx - tanhf| <= eta, one rounding
//     each of 1 + tanh, 0.5 g (1 + tanh) and the product with u gives
//     |A - exact| <= |0.5 g u| (eta + 2^-23) + 2^-22.9 |A| (plus a few
//     subnormal units); the bound used, |0.5 g u| (2^-21 + 2^-22) +
//     2^-21 |A| + 2^-146, is at least twice that: room for its own fp32
//     evaluation and for the roundings in step 3.
//  2. The block maximum needs exact values: every value whose |A| + B
//     reaches max(|A| - B) over the block may be the largest, so those
//     (usually one) are evaluated exactly; amax, the fp16 scale d and 1/d
//     follow from them as in the quantizer.
//  3. q = roundf(RN(v id)) of any other value is decided from y = RN(A id):
//     the exact value's product lies within B id of A id, which lies within
//     half an ulp of y, and roundf changes only at half-integers, so when y
//     is farther from the nearest half-integer h than B id plus the
//     roundings of y and of a product near h (2 ulp(y) for |y| >= 1/4,
//     at most |y| 2^-22; the test adds |y| 2^-21, and below 1/4 the
//     distance exceeds 1/4), the exact value's q is roundf(y); the distance
//     |(|y| - trunc|y|) - 1/2| is exact in fp32 for |y| >= 1/4. The rare
//     value closer than that (or non-finite) is evaluated exactly. A block whose
//     1/d overflows quantizes to -128 throughout (q8_value) and needs no
//     decision.
// Steps 1 and 2's candidate test of geglu_quantize_part4: the approximations
// a[], their bounds, and the candidate bits (every block has one: the value
// with the largest |A| - B passes the test).
__device__ __forceinline__ uint32_t geglu_approx_part4(const float (&g)[8], const float (&u)[8], float (&a)[8],
                                                       float (&bound)[8]) {
  float mlo = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float h = 0.5f * g[i];
    const float t = 1.0f + tanh_approx(gelu_inner(g[i]));
    a[i] = h * t * u[i];
    bound[i] = __builtin_fmaf(fabsf(h * u[i]), kTanhApproxBound + 0x1p-22f, __builtin_fmaf(fabsf(a[i]), 0x1p-21f, 0x1p-146f));
    mlo = fmaxf(mlo, fabsf(a[i]) - bound[i]);
  }
  mlo = quad_max(mlo);
  // A non-finite approximation (or bound) fails every comparison: such a
  // value is evaluated exactly.
  uint32_t cand = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) cand |= !(fabsf(a[i]) + bound[i] < mlo) ? 1u << i : 0u;
  return cand;
}

// Steps 2 (from the exact candidates in a[]) and 3 of geglu_quantize_part4,
// and the stores.
__device__ __forceinline__ void geglu_decide_part4(const float (&g)[8], const float (&u)[8], const float (&bound)[8],
                                                   uint32_t cand, float (&a)[8], bool store, int8_t* __restrict__ q,
                                                   float* __restrict__ d_out) {
  int32_t qi[8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, cand & (1u << i) ? fabsf(a[i]) : 0.0f);
  amax = quad_max(amax);
  const float d = div127(amax);
  const float id = amax != 0.0f ? 1.0f / d : 0.0f;
  const bool id_over = id > 3.40282347e38f;
  uint32_t undecided = 0;  // built without branches: every value is tested
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float y = a[i] * id, ay = fabsf(y);
    qi[i] = id_over ? -128 : q8_round(y);
    const float dist = fabsf((ay - truncf(ay)) - 0.5f);
    const float margin = __builtin_fmaf(bound[i], id, ay * 0x1p-21f);
    undecided |= dist > margin ? 0u : 1u << i;
  }
  undecided = id_over ? 0u : undecided & ~cand;
  geglu_exact_passes<true>(g, u, undecided, id, a, qi);
  if (!store) return;
  if ((threadIdx.x & 3) == 0) *d_out = fp16_bits_to_fp32(fp32_to_fp16_bits(d));
  *reinterpret_cast<uint2*>(q) = make_uint2(pack_i8x4(qi[0], qi[1], qi[2], qi[3]), pack_i8x4(qi[4], qi[5], qi[6], qi[7]));
}

__device__ __forceinline__ void geglu_quantize_part4(const float (&g)[8], const float (&u)[8], bool store,
                                                     int8_t* __restrict__ q, float* __restrict__ d_out) {
  float a[8], bound[8];
  const uint32_t cand = geglu_approx_part4(g, u, a, bound);
  int32_t unused[8];
  geglu_exact_passes<false>(g, u, cand, 0.0f, a, unused);  // a[] now exact for the candidates
  geglu_decide_part4(g, u, bound, cand, a, store, q, d_out);
}

// Chain c of the SSE2 sum of squares of an n-float row (kernels.c:82-94):
// the sequential sum over t of x[8t + c]^2, squares rounded then added.
template <int N>
__device__ __forceinline__ float sse2_chain(const float* row, int c) {
  float v[N / 8];
#pragma unroll
  for (int t = 0; t < N / 8; ++t) v[t] = row[8 * t + c];
  float s = 0.0f;
#pragma unroll
  for (int t = 0; t < N / 8; ++t) {
    const float p = v[t] * v[t];
    s = s + p;
  }
  return s;
}

// Horizontal step of the SSE2 sum for the 8-lane group holding chains 0..7
// (chains 0-3 are the first 4-wide accumulator, 4-7 the second):
// v[j] = acc0[j] + acc1[j], total (v0 + v2) + (v1 + v3) (kernels.c:35-39).
// Every lane of the group receives the total. All 64 lanes must call it.
__device__ __forceinline__ float sse2_combine(float s) {
  const int lane = threadIdx.x & 63, base = lane & ~7;
  const float up = __shfl(s, base + ((lane + 4) & 7), 64);
  const float v = s + up;
  const float v0 = __shfl(v, base, 64), v1 = __shfl(v, base + 1, 64);
  const float v2 = __shfl(v, base + 2, 64), v3 = __shfl(v, base + 3, 64);
  return (v0 + v2) + (v1 + v3);
}

// Sum of squares of an LDS row of n floats (n % 8 == 0) in the reference's
// SSE2 order (kernels.c:82-94): lane c < 8 runs the sequential chain over
// x[8t + c] (lanes 0-3 are the first 4-lane accumulator, 4-7 the second),
// then v[j] = acc0[j] + acc1[j] and the horizontal sum is
// (v0 + v2) + (v1 + v3) (kernels.c:35-39). The result is returned to every
// lane of the calling wave. All 64 lanes must call it.
__device__ __forceinline__ float sum_squares_sse2(const float* row, int n) {
  const int lane = threadIdx.x & 63;
  float s = 0.0f;
  if (lane < 8) {
    for (int t = 0; t < n / 8; ++t) {
      const float v = row[8 * t + lane];
      const float p = v * v;
      s = s + p;
    }
  }
  const float hi = __shfl(s, (lane + 4) & 63, 64);
  const float v = s + hi;  // lanes 0..3 hold v[0..3]
  const float v0 = __shfl(v, 0, 64), v1 = __shfl(v, 1, 64);
  const float v2 = __shfl(v, 2, 64), v3 = __shfl(v, 3, 64);
  return (v0 + v2) + (v1 + v3);
}

// 1 / sqrtf(ss / n + eps) with correctly rounded division and square root
// (kernels.c:144, :154, :165).
__device__ __forceinline__ float rms_inverse(float ss, int n, float eps) {
  return 1.0f / __builtin_sqrtf(ss / (float)n + eps);
}

}  // namespace eg2
