// Q8_0 x Q8_0 projection GEMM on MFMA (gfx950).
//
//   y[n][m] = sum over 32-blocks b of ((float)dot_b(n, m) * d_w[m][b]) * d_x[n][b]
//
// exactly as the reference's CPU dot (gemma2.c:120-141): per output, an
// exact integer block dot, scaled by the weight then the activation scale,
// added in block order with one fp32 rounding per operation. Results are
// bit-identical to the CPU path.
//
// Both operands hold Q8_0 integers stored as fp16 (every int8 is exact in
// fp16) with one float scale per 32-block: activations as written by the
// fused quantizing row kernels, weights repacked once at load. A 32-block
// dot is two v_mfma_f32_32x32x16_f16 with a zero accumulator; its products
// (|q| <= 128) and partial sums (|sum| <= 2^19) are exact in fp32, so the
// MFMA returns the integer dot exactly. The per-block scaling then costs
// three VALU operations per output, which bounds this kernel (it cannot be
// folded into the operands without changing the rounding).
#include "eg2_device.hpp"
#include "eg2_kernels.hpp"

namespace eg2 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 32;              // one Q8_0 block per k-step
constexpr int kLdsStride = kBK + 8;  // fp16 elements per LDS row (padding against bank conflicts)

// BN x BM output tile per workgroup of WN x WM waves; each wave owns a
// (BN/WN) x (BM/WM) sub-tile of 32x32 MFMA tiles. k % 32 == 0.
template <int BN, int BM, int WN, int WM>
__global__ void __launch_bounds__(WN * WM * 64)
gemm_q8_kernel(const _Float16* __restrict__ xq, const float* __restrict__ xd,
               const _Float16* __restrict__ wq, const float* __restrict__ wd,
               float* __restrict__ y, int n, int m, int k, int ldy) {
  constexpr int NT = WN * WM * 64;
  constexpr int TN = BN / WN / 32, TM = BM / WM / 32;
  constexpr int A_LOADS = (4 * BN + NT - 1) / NT;  // 16-byte quarter-block loads
  constexpr int B_LOADS = (4 * BM + NT - 1) / NT;
  __shared__ __align__(16) _Float16 As[2][BN * kLdsStride];
  __shared__ __align__(16) _Float16 Bs[2][BM * kLdsStride];
  __shared__ __align__(16) float Ad[2][BN];
  __shared__ __align__(16) float Bd[2][BM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave / WM, wm = wave % WM;
  const int n0 = blockIdx.y * BN, m0 = blockIdx.x * BM;
  const int nb = k / kBK;

  half8 ra[A_LOADS], rb[B_LOADS];
  float sa[A_LOADS], sb[B_LOADS];

  auto load = [&](int kb) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int idx = tid + i * NT, row = idx >> 2, part = idx & 3, g = n0 + row;
      const bool ok = idx < 4 * BN && g < n;
      ra[i] = ok ? *reinterpret_cast<const half8*>(xq + (size_t)g * k + kb * kBK + part * 8) : half8{};
      sa[i] = ok ? xd[(size_t)g * nb + kb] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int idx = tid + i * NT, row = idx >> 2, part = idx & 3, g = m0 + row;
      const bool ok = idx < 4 * BM && g < m;
      rb[i] = ok ? *reinterpret_cast<const half8*>(wq + (size_t)g * k + kb * kBK + part * 8) : half8{};
      sb[i] = ok ? wd[(size_t)g * nb + kb] : 0.0f;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int idx = tid + i * NT;
      if (idx < 4 * BN) {
        *reinterpret_cast<half8*>(&As[buf][(idx >> 2) * kLdsStride + (idx & 3) * 8]) = ra[i];
        if ((idx & 3) == 0) Ad[buf][idx >> 2] = sa[i];
      }
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int idx = tid + i * NT;
      if (idx < 4 * BM) {
        *reinterpret_cast<half8*>(&Bs[buf][(idx >> 2) * kLdsStride + (idx & 3) * 8]) = rb[i];
        if ((idx & 3) == 0) Bd[buf][idx >> 2] = sb[i];
      }
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
    half8 af[TN][2], bf[TM][2];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        af[a][h] = *reinterpret_cast<const half8*>(&As[cur][(wn * TN * 32 + a * 32 + r32) * kLdsStride + h * 16 + g * 8]);
#pragma unroll
    for (int b = 0; b < TM; ++b)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        bf[b][h] = *reinterpret_cast<const half8*>(&Bs[cur][(wm * TM * 32 + b * 32 + r32) * kLdsStride + h * 16 + g * 8]);
    float dw[TM];
#pragma unroll
    for (int b = 0; b < TM; ++b) dw[b] = Bd[cur][wm * TM * 32 + b * 32 + r32];
#pragma unroll
    for (int a = 0; a < TN; ++a) {
      // Row scales of this lane's 16 outputs: rows 8*(v/4) + 4*g + (v%4).
      float dx[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 s4 = *reinterpret_cast<const float4*>(&Ad[cur][wn * TN * 32 + a * 32 + 8 * q + 4 * g]);
        dx[4 * q + 0] = s4.x;
        dx[4 * q + 1] = s4.y;
        dx[4 * q + 2] = s4.z;
        dx[4 * q + 3] = s4.w;
      }
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        floatx16 dot = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[a][0], bf[b][0], floatx16{}, 0, 0, 0);
        dot = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[a][1], bf[b][1], dot, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float t = dot[v] * dw[b];
          const float u = t * dx[v];
          acc[a][b][v] = acc[a][b][v] + u;
        }
      }
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

hipError_t launch_gemm_q8(const _Float16* xq, const float* xd, const _Float16* wq, const float* wd, float* y, int n,
                          int m, int k, int ldy, hipStream_t st) {
  if (n <= 0 || m <= 0 || k <= 0 || k % kBK != 0 || ldy < m) return hipErrorInvalidValue;
  // The kernel is bound by per-block VALU scaling, so the tile is chosen to
  // spread the waves over all 256 CUs rather than for operand reuse.
  const int tiles64 = ((m + 63) / 64) * ((n + 63) / 64);
  if (tiles64 >= 1024) {
    hipLaunchKernelGGL((gemm_q8_kernel<64, 64, 2, 2>), dim3((m + 63) / 64, (n + 63) / 64), dim3(256), 0, st, xq, xd,
                       wq, wd, y, n, m, k, ldy);
  } else {
    hipLaunchKernelGGL((gemm_q8_kernel<32, 64, 1, 2>), dim3((m + 63) / 64, (n + 31) / 32), dim3(128), 0, st, xq, xd,
                       wq, wd, y, n, m, k, ldy);
  }
  return hipGetLastError();
}

}  // namespace eg2
