// Q8_0 x Q8_0 projection GEMM on MFMA (gfx950).
//
//   y[n][m] = sum over 32-blocks b of ((float)dot_b(n, m) * d_w[m][b]) * d_x[n][b]
//
// exactly as the reference's CPU dot (gemma2.c:120-141): per output, an
// exact integer block dot, scaled by the weight then the activation scale,
// added in block order with one fp32 rounding per operation. Results are
// bit-identical to the CPU path.
//
// Operands hold Q8_0 integers as fp16 (every int8 is exact in fp16). A
// 32-block dot is two v_mfma_f32_32x32x16_f16 with a zero accumulator; its
// products (|q| <= 128) and partial sums (|sum| <= 2^19) are exact in fp32,
// so the MFMA returns the integer dot exactly. The scaling then costs three
// VALU operations per output and block (it cannot be folded into the
// operands without changing the rounding).
//
// Data layout (chosen for this kernel):
//  * activations xq [rows][k] fp16, block scales transposed xd [k/32][ldx]
//    (the quantizing row kernels write them that way);
//  * weights in a fragment-major layout, repacked once at load:
//    wf [m/32][k/32][64 lanes][16 fp16] where lane l holds row l % 32 and
//    columns 16 * (l / 32) .. +15 of the 32-block, and their scales
//    wdf [m/32][k/32][64 lanes] (one per lane, the row's block scale).
//
// One workgroup computes a 32-row x (32 * WM)-column tile with WM waves, one
// 32x32 output tile per wave. The 32 activation rows of each block go from
// global memory straight into an LDS ring (global_load_lds_dwordx4, one
// 1 KB instruction per 16 rows, XOR-swizzled 16-byte chunks so the fragment
// reads are free of bank conflicts) shared by the WM waves; each wave reads
// its weight fragments from global memory into a register ring, fully
// coalesced thanks to the fragment-major layout. LDS read bandwidth
// (~64 B/clk per CU on this part) is the scarce resource: this split moves
// only the shared operand through LDS. The activation scales of all blocks
// are preloaded into LDS once per workgroup.
//
// In the MFMA 32x32 output layout a lane holds one weight column and 16
// token rows; each row's activation scale reaches the lane through a DPP
// row broadcast folded into the multiply (v_mul_f32_dpp row_newbcast), so
// the per-block scale traffic is one float per lane.
#include <utility>

#include "eg2_device.hpp"
#include "eg2_kernels.hpp"

namespace eg2 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 32;   // one Q8_0 block per k-step
constexpr int kXcds = 8;  // MI355X: 8 XCDs of 32 CUs, each with its own L2

extern __shared__ __align__(16) unsigned char gemm_lds[];

// 4 / 16 bytes per lane from global memory straight into LDS at
// lds + 4 * lane / lds + 16 * lane (the LDS base is wave-uniform).
__device__ __forceinline__ void dma4(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
}
__device__ __forceinline__ void dma16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// Waits until at most N vector-memory operations of this wave are in
// flight, then joins the workgroup barrier. The LDS ring is filled by DMA,
// which the compiler does not track, so the wait is explicit; the memory
// clobber keeps LDS reads from moving across it.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Chunk swizzle of a 64-byte LDS row: 16-byte chunk c of row r is stored at
// c ^ swz(r). The MFMA fragment reads (lane i of each half-wave reads row i)
// then spread every 8- and 16-lane group over distinct banks.
__device__ __forceinline__ int swz(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }

// Broadcast of lane V of each 16-lane row to the whole row.
template <int V>
__device__ __forceinline__ float row_bcast(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x150 + V, 0xf, 0xf, true));
}

// acc[v] += (dot[v] * dw) * dx(row v): the lane's 16 output rows take their
// activation scales from lanes 0..15 of its 16-lane row.
template <int... V>
__device__ __forceinline__ void scale_accumulate(floatx16& acc, const floatx16& dot, float dw, float dxv,
                                                 std::integer_sequence<int, V...>) {
  ((acc[V] = acc[V] + (dot[V] * dw) * row_bcast<V>(dxv)), ...);
}

template <int WM, int D>
__global__ void __launch_bounds__(WM * 64)
gemm_q8_kernel(const _Float16* __restrict__ xq, const float* __restrict__ xd, int ldx,
               const _Float16* __restrict__ wf, const float* __restrict__ wdf, float* __restrict__ y, int n, int m,
               int k, int ldy) {
  constexpr int S = 2 * D;        // LDS ring stages
  constexpr int STAGE = 32 * 64;  // 32 rows x 64 bytes
  constexpr int QA = 2;           // 1 KB DMA instructions per stage
  static_assert(QA % WM == 0 || WM % QA == 0, "DMA split");
  constexpr int QAW = QA >= WM ? QA / WM : 1;  // per issuing wave
  constexpr int QB = 3;                        // weight loads per block
  static_assert((D & (D - 1)) == 0, "D must be a power of two");

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_tiles_n = (n + 31) / 32, mt_count = (m + 31) / 32;
  const int n_tiles = n_tiles_n * ((mt_count + WM - 1) / WM);
  // XCD-aware order: workgroup b runs on XCD b % 8; each XCD takes one
  // contiguous run of tiles (column-group major), so the weight columns it
  // needs stay in its own L2.
  const int per_xcd = (n_tiles + kXcds - 1) / kXcds;
  const int tile = (int)(blockIdx.x % kXcds) * per_xcd + (int)(blockIdx.x / kXcds);
  if (tile >= n_tiles) return;
  const int n0 = (tile % n_tiles_n) * 32;
  const int mt_raw = (tile / n_tiles_n) * WM + wave, mt = min(mt_raw, mt_count - 1);
  const int nb = k / kBK;
  unsigned char* smem = gemm_lds;
  float* sA = reinterpret_cast<float*>(smem + S * STAGE);  // [nb rounded up to 2][32]

  // Activation scales of all blocks: two blocks (2 x 32 rows) per instruction.
  for (int b0 = 2 * wave; b0 < nb; b0 += 2 * WM) {
    const int b = min(b0 + (lane >> 5), nb - 1);
    dma4(xd + (size_t)b * ldx + min(n0 + (lane & 31), n - 1), sA + b0 * 32);
  }
  // Activation DMA: instruction q fills stage rows 16q..16q+15; lane L takes
  // (row 16q + L/4, stored chunk L%4) = global chunk (L%4) ^ swz(row).
  const bool dma_wave = wave < QA;
  const _Float16* asrc[QAW];
  int aoff[QAW];
#pragma unroll
  for (int t = 0; t < QAW; ++t) {
    const int q = min(wave * QAW + t, QA - 1), row = 16 * q + (lane >> 2), c = (lane & 3) ^ swz(row);
    asrc[t] = xq + (size_t)min(n0 + row, n - 1) * k + 8 * c;
    aoff[t] = 1024 * q;
  }
  auto issue_a = [&](int slot, int kb) {
    if (!dma_wave) return;
    unsigned char* base = smem + (slot & (S - 1)) * STAGE;
#pragma unroll
    for (int t = 0; t < QAW; ++t) dma16(asrc[t] + kb * kBK, base + aoff[t]);
  };
  // Weight fragments, D blocks ahead in registers.
  const _Float16* bsrc = wf + ((size_t)mt * nb * 64 + lane) * 16;
  const float* dsrc = wdf + (size_t)mt * nb * 64 + lane;
  struct BStage {
    half8 b0, b1;
    float dw;
  };
  BStage ring[D];
  auto load_b = [&](BStage& r, int kb) {
    const half8* p = reinterpret_cast<const half8*>(bsrc + (size_t)kb * 64 * 16);
    r.b0 = p[0];
    r.b1 = p[1];
    r.dw = dsrc[kb * 64];
  };

  floatx16 acc = floatx16{};
  const int g = lane >> 5, r32 = lane & 31;
  // Row whose scale this lane supplies to the DPP broadcast: lane 16r + v
  // carries the scale of output register v for the lanes of 16-lane row r.
  const int srow = 8 * ((lane & 15) >> 2) + 4 * g + (lane & 3);
  const int af = swz(r32);

#pragma unroll
  for (int u = 0; u < D; ++u) {
    issue_a(u, min(u, nb - 1));
    load_b(ring[u], min(u, nb - 1));
  }
  // Block kb: its DMA and weight loads were issued D blocks earlier; the
  // stage it refills, (kb + D) % S, was last read in block kb - D.
  for (int kb0 = 0; kb0 < nb; kb0 += D) {
    const unsigned char* st0 = smem + (kb0 & D) * STAGE;
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const int kb = kb0 + u;
      if (dma_wave) wait_vm_barrier<(D - 1) * (QAW + QB)>();
      else wait_vm_barrier<(D - 1) * QB>();
      const unsigned char* st = st0 + u * STAGE;
      const half8 a0 = *reinterpret_cast<const half8*>(st + r32 * 64 + 16 * ((2 * g) ^ af));
      const half8 a1 = *reinterpret_cast<const half8*>(st + r32 * 64 + 16 * ((2 * g + 1) ^ af));
      const float dx = sA[kb * 32 + srow];
      floatx16 dot = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, ring[u].b0, floatx16{}, 0, 0, 0);
      dot = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, ring[u].b1, dot, 0, 0, 0);
      issue_a(kb + D, min(kb + D, nb - 1));
      scale_accumulate(acc, dot, ring[u].dw, dx, std::make_integer_sequence<int, 16>{});
      load_b(ring[u], min(kb + D, nb - 1));
    }
  }
  // The ring's last refills are redundant; they must land before the
  // workgroup's LDS is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (mt_raw >= mt_count) return;
  const int col = mt * 32 + r32;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int row = n0 + 8 * (v >> 2) + 4 * g + (v & 3);
    if (row < n && col < m) y[(size_t)row * ldy + col] = acc[v];
  }
}

template <int WM, int D>
static hipError_t launch_gemm(const _Float16* xq, const float* xd, int ldx, const _Float16* wf, const float* wdf,
                              float* y, int n, int m, int k, int ldy, hipStream_t st) {
  const int tiles = ((n + 31) / 32) * (((m + 31) / 32 + WM - 1) / WM);
  const dim3 grid(((tiles + kXcds - 1) / kXcds) * kXcds);
  const int nb = k / kBK;
  const size_t lds = (size_t)(2 * D) * 32 * 64 + (size_t)((nb + 1) / 2 * 2) * 32 * 4;
  hipLaunchKernelGGL((gemm_q8_kernel<WM, D>), grid, dim3(WM * 64), lds, st, xq, xd, ldx, wf, wdf, y, n, m, k, ldy);
  return hipGetLastError();
}

size_t gemm_q8_max_k() {
  // LDS: 4 stages of 2 KB plus 128 bytes of scales per block, within 64 KB.
  return (65536 - 4 * 2048) / 128 * 32;
}

hipError_t launch_gemm_q8(const _Float16* xq, const float* xd, int ldx, const _Float16* wf, const float* wdf,
                          float* y, int n, int m, int k, int ldy, hipStream_t st) {
  if (n <= 0 || m <= 0 || k <= 0 || k % kBK != 0 || ldy < m || ldx < n || (size_t)k > gemm_q8_max_k())
    return hipErrorInvalidValue;
  // Two waves per 32 x 64 tile, weight fragments two blocks ahead.
  if ((k / kBK) % 2 == 0) return launch_gemm<2, 2>(xq, xd, ldx, wf, wdf, y, n, m, k, ldy, st);
  return launch_gemm<2, 1>(xq, xd, ldx, wf, wdf, y, n, m, k, ldy, st);
}

}  // namespace eg2
