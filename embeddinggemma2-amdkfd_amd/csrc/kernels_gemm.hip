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
constexpr int kXcds = 8;             // MI355X: 8 XCDs of 32 CUs, each with its own L2

// BN x BM output tile per workgroup of WN x WM waves; each wave owns a
// (BN/WN) x (BM/WM) sub-tile of 32x32 MFMA tiles. k % 32 == 0.
//
// K loop: operands of a 32-block travel HBM/L2 -> registers -> LDS (double
// buffered) -> MFMA. With a 2048-token wave there are too few waves per CU
// to hide memory latency, so each thread keeps DEPTH blocks of loads in
// flight in a register ring; the loop is unrolled by DEPTH so ring slots are
// compile-time registers.
template <int BN, int BM, int WN, int WM, int DEPTH>
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
  // XCD-aware tile order: workgroups are dealt round-robin to the 8 XCDs,
  // so workgroup b runs on XCD b % 8. Renumbering gives each XCD one
  // contiguous run of tiles in column-block-major order, i.e. a slice of
  // the weight columns plus the activations, which stay in that XCD's L2.
  const int n_tiles_n = (n + BN - 1) / BN, n_tiles = n_tiles_n * ((m + BM - 1) / BM);
  const int per_xcd = (n_tiles + kXcds - 1) / kXcds;
  const int tile = (int)(blockIdx.x % kXcds) * per_xcd + (int)(blockIdx.x / kXcds);
  if (tile >= n_tiles) return;
  const int n0 = (tile % n_tiles_n) * BN, m0 = (tile / n_tiles_n) * BM;
  const int nb = k / kBK;

  struct Stage {
    half8 a[A_LOADS], b[B_LOADS];
    float sa[A_LOADS], sb[B_LOADS];
  };
  Stage ring[DEPTH];

  // Rows past n (or m) load the last valid row instead: always in bounds,
  // never stored, and free of per-lane branches.
  auto load = [&](Stage& st, int kb) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int idx = tid + i * NT, row = (idx >> 2) % BN, part = idx & 3, g = min(n0 + row, n - 1);
      st.a[i] = *reinterpret_cast<const half8*>(xq + (size_t)g * k + kb * kBK + part * 8);
      st.sa[i] = xd[(size_t)g * nb + kb];
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int idx = tid + i * NT, row = (idx >> 2) % BM, part = idx & 3, g = min(m0 + row, m - 1);
      st.b[i] = *reinterpret_cast<const half8*>(wq + (size_t)g * k + kb * kBK + part * 8);
      st.sb[i] = wd[(size_t)g * nb + kb];
    }
  };
  auto store = [&](const Stage& st, int buf) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int idx = tid + i * NT;
      if (idx < 4 * BN) {
        *reinterpret_cast<half8*>(&As[buf][(idx >> 2) * kLdsStride + (idx & 3) * 8]) = st.a[i];
        if ((idx & 3) == 0) Ad[buf][idx >> 2] = st.sa[i];
      }
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int idx = tid + i * NT;
      if (idx < 4 * BM) {
        *reinterpret_cast<half8*>(&Bs[buf][(idx >> 2) * kLdsStride + (idx & 3) * 8]) = st.b[i];
        if ((idx & 3) == 0) Bd[buf][idx >> 2] = st.sb[i];
      }
    }
  };

  floatx16 acc[TN][TM];
#pragma unroll
  for (int a = 0; a < TN; ++a)
#pragma unroll
    for (int b = 0; b < TM; ++b) acc[a][b] = floatx16{};

  const int g = lane >> 5, r32 = lane & 31;
  auto compute = [&](int cur) {
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
    // All block dots first (independent MFMAs), then the dependent scaling.
    floatx16 dot[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
      for (int b = 0; b < TM; ++b) {
        dot[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[a][0], bf[b][0], floatx16{}, 0, 0, 0);
        dot[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[a][1], bf[b][1], dot[a][b], 0, 0, 0);
      }
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
      for (int b = 0; b < TM; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float t = dot[a][b][v] * dw[b];
          const float u = t * dx[v];
          acc[a][b][v] = acc[a][b][v] + u;
        }
    }
  };

  // Prologue: DEPTH blocks in flight, block 0 staged in LDS.
#pragma unroll
  for (int u = 0; u < DEPTH; ++u)
    if (u < nb) load(ring[u], u);
  store(ring[0], 0);
  __syncthreads();
  // Block kb sits in ring slot kb % DEPTH; it went to LDS during block kb-1,
  // so that slot is refilled with block kb + DEPTH during block kb.
  for (int kb0 = 0; kb0 < nb; kb0 += DEPTH) {
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) {
      const int kb = kb0 + u;
      if (kb < nb) {
        compute(kb & 1);
        if (kb + 1 < nb) store(ring[(u + 1) % DEPTH], (kb + 1) & 1);
        if (kb + DEPTH < nb) load(ring[u], kb + DEPTH);
        __syncthreads();
      }
    }
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

// Grid for the XCD-aware order: the tile count rounded up to whole XCD slices.
template <int BN, int BM>
dim3 gemm_grid(int n, int m) {
  const int tiles = ((n + BN - 1) / BN) * ((m + BM - 1) / BM);
  return dim3(((tiles + kXcds - 1) / kXcds) * kXcds);
}

hipError_t launch_gemm_q8(const _Float16* xq, const float* xd, const _Float16* wq, const float* wd, float* y, int n,
                          int m, int k, int ldy, hipStream_t st) {
  if (n <= 0 || m <= 0 || k <= 0 || k % kBK != 0 || ldy < m) return hipErrorInvalidValue;
  // The kernel is bound by per-block VALU scaling, so the tile is chosen to
  // spread the waves over all 256 CUs rather than for operand reuse.
  const int tiles64 = ((m + 63) / 64) * ((n + 63) / 64);
  if (tiles64 >= 1024) {
    const dim3 grid = gemm_grid<64, 64>(n, m);
    hipLaunchKernelGGL((gemm_q8_kernel<64, 64, 2, 2, 4>), grid, dim3(256), 0, st, xq, xd, wq, wd, y, n, m, k, ldy);
  } else {
    const dim3 grid = gemm_grid<32, 64>(n, m);
    hipLaunchKernelGGL((gemm_q8_kernel<32, 64, 1, 2, 4>), grid, dim3(128), 0, st, xq, xd, wq, wd, y, n, m, k, ldy);
  }
  return hipGetLastError();
}

}  // namespace eg2
