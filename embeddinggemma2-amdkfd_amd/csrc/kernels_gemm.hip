// Q8_0 x Q8_0 projection GEMM on MFMA (gfx950).
//
//   y[n][m] = sum_k X[n][k] * W[m][k]
//
// Both operands arrive as Q8_0 (int8 values + one scale per 32-element block
// along k): the activations from the fused quantizing row kernels, the
// weights repacked once at load from the GGUF blocks. Each 32-wide k-step is
// one Q8_0 block; it is staged from HBM as int8, dequantized to fp16 as
// fp16(q * d) (q * d is exact in fp32) while it is written to LDS, and fed to
// v_mfma_f32_32x32x16_f16 with fp32 accumulation. The reference's CPU dot
// (gemma2.c:120-141) sums exact int32 block dots scaled in fp32; this kernel
// rounds each dequantized operand to fp16 instead (relative error 2^-12 per
// operand), which keeps the kernel MFMA-bound rather than bound by per-block
// VALU scaling.
#include "eg2_device.hpp"
#include "eg2_kernels.hpp"

namespace eg2 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 32;            // one Q8_0 block per k-step
constexpr int kLdsStride = kBK + 8;  // fp16 elements per LDS row (padded against bank conflicts)

// 16 int8 values times one scale -> 16 fp16 values written as two 16-byte LDS stores.
__device__ __forceinline__ void dequant16_to_lds(const int4 raw, float d, _Float16* dst) {
  const int32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  half8 lo, hi;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int8_t q = (int8_t)((w[i / 4] >> (8 * (i % 4))) & 0xFF);
    lo[i] = (_Float16)((float)q * d);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int8_t q = (int8_t)((w[2 + i / 4] >> (8 * (i % 4))) & 0xFF);
    hi[i] = (_Float16)((float)q * d);
  }
  reinterpret_cast<half8*>(dst)[0] = lo;
  reinterpret_cast<half8*>(dst)[1] = hi;
}

// BN x BM output tile per workgroup, WN x WM waves, each wave owning a
// (BN/WN) x (BM/WM) sub-tile of 32x32 MFMA tiles. k must be a multiple of 32.
template <int BN, int BM, int WN, int WM>
__global__ void __launch_bounds__(WN * WM * 64)
gemm_q8_kernel(const int8_t* __restrict__ xq, const float* __restrict__ xd,
               const int8_t* __restrict__ wq, const float* __restrict__ wd,
               float* __restrict__ y, int n, int m, int k, int ldy) {
  constexpr int NT = WN * WM * 64;
  constexpr int TN = BN / WN / 32, TM = BM / WM / 32;
  constexpr int A_LOADS = (2 * BN + NT - 1) / NT;  // 16-byte half-block loads
  constexpr int B_LOADS = (2 * BM + NT - 1) / NT;
  __shared__ __align__(16) _Float16 As[2][BN * kLdsStride];
  __shared__ __align__(16) _Float16 Bs[2][BM * kLdsStride];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave / WM, wm = wave % WM;
  const int n0 = blockIdx.y * BN, m0 = blockIdx.x * BM;
  const int nb = k / kBK, kd = k / kQK;

  int4 ra[A_LOADS], rb[B_LOADS];
  float sa[A_LOADS], sb[B_LOADS];

  auto load = [&](int kb) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int idx = tid + i * NT, row = idx >> 1, part = idx & 1, g = n0 + row;
      const bool ok = idx < 2 * BN && g < n;
      ra[i] = ok ? *reinterpret_cast<const int4*>(xq + (size_t)g * k + kb * kBK + part * 16) : int4{0, 0, 0, 0};
      sa[i] = ok ? xd[(size_t)g * kd + kb] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int idx = tid + i * NT, row = idx >> 1, part = idx & 1, g = m0 + row;
      const bool ok = idx < 2 * BM && g < m;
      rb[i] = ok ? *reinterpret_cast<const int4*>(wq + (size_t)g * k + kb * kBK + part * 16) : int4{0, 0, 0, 0};
      sb[i] = ok ? wd[(size_t)g * kd + kb] : 0.0f;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int idx = tid + i * NT;
      if (idx < 2 * BN) dequant16_to_lds(ra[i], sa[i], &As[buf][(idx >> 1) * kLdsStride + (idx & 1) * 16]);
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int idx = tid + i * NT;
      if (idx < 2 * BM) dequant16_to_lds(rb[i], sb[i], &Bs[buf][(idx >> 1) * kLdsStride + (idx & 1) * 16]);
    }
  };

  floatx16 acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b) acc[a][b] = floatx16{};

  load(0);
  store(0);
  __syncthreads();
  const int g = lane >> 5, r32 = lane & 31;
  for (int kb = 0; kb < nb; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nb) load(kb + 1);
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 16) {
      half8 af[TN], bf[TM];
#pragma unroll
      for (int a = 0; a < TN; ++a)
        af[a] = *reinterpret_cast<const half8*>(&As[cur][(wn * TN * 32 + a * 32 + r32) * kLdsStride + ks + g * 8]);
#pragma unroll
      for (int b = 0; b < TM; ++b)
        bf[b] = *reinterpret_cast<const half8*>(&Bs[cur][(wm * TM * 32 + b * 32 + r32) * kLdsStride + ks + g * 8]);
#pragma unroll
      for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[a], bf[b], acc[a][b], 0, 0, 0);
    }
    if (kb + 1 < nb) store(cur ^ 1);
    __syncthreads();
  }

  // MFMA 32x32 output layout: lane holds column (lane & 31) and rows
  // 8*(v/4) + 4*(lane/32) + (v%4) for v = 0..15.
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b) {
      const int col = m0 + wm * TM * 32 + b * 32 + r32;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = n0 + wn * TN * 32 + a * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
        if (row < n && col < m) y[(size_t)row * ldy + col] = acc[a][b][v];
      }
    }
}

hipError_t launch_gemm_q8(const int8_t* xq, const float* xd, const int8_t* wq, const float* wd, float* y, int n,
                          int m, int k, int ldy, hipStream_t st) {
  if (n <= 0 || m <= 0 || k <= 0 || k % kBK != 0 || ldy < m) return hipErrorInvalidValue;
  const int big_tiles = ((m + 127) / 128) * ((n + 127) / 128);
  if (big_tiles >= 256) {
    hipLaunchKernelGGL((gemm_q8_kernel<128, 128, 2, 2>), dim3((m + 127) / 128, (n + 127) / 128), dim3(256), 0, st,
                       xq, xd, wq, wd, y, n, m, k, ldy);
  } else {
    hipLaunchKernelGGL((gemm_q8_kernel<64, 64, 2, 2>), dim3((m + 63) / 64, (n + 63) / 64), dim3(256), 0, st, xq,
                       xd, wq, wd, y, n, m, k, ldy);
  }
  return hipGetLastError();
}

}  // namespace eg2
