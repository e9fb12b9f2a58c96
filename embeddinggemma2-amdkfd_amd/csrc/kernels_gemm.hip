// Q8_0 x Q8_0 projection GEMM on int8 MFMA (gfx950).
//
//   y[n][m] = sum over 32-blocks b of ((float)dot_b(n, m) * d_w[m][b]) * d_x[n][b]
//
// exactly as the reference's CPU dot (gemma2.c:120-141): per output, an
// exact integer block dot, scaled by the weight then the activation scale,
// added in block order with one fp32 rounding per operation. Results are
// bit-identical to the CPU path.
//
// Exactness. A 32-block dot is one v_mfma_i32_32x32x32_i8 (exact int32).
// Its accumulator input is the integer 0x4B400000, the bit pattern of the
// float 1.5 * 2^23; |dot| <= 32 * 128 * 128 = 2^19 keeps the result's bits a
// float in [2^23, 2^24), where every float is an integer, and that float is
// exactly 12582912 + dot. fma(it, d_w, -12582912 * d_w) is then dot * d_w
// rounded once -- the reference's (float)dot * d_w -- since 12582912 * d_w
// is exact (d_w is the value of an fp16: at most 11 significant bits). The
// int-to-float conversion thus costs nothing, and a block costs three VALU
// operations per output (fma, multiply, add); they cannot be merged
// without changing the rounding, and they, not the MFMA, bound the kernel.
//
// Operand layout ("row tiles"; the quantizing kernels write activations in
// it, eg2_q8_weight_tiles writes weights): int8 [rows/32][k/32][2][32][16],
// so each 32-row x 32-value block is 1 KB in the register order of the
// MFMA operand (lane 32h + r holds row r, values 16h .. 16h + 15): one
// 16-byte load per lane at 16 lane moves it into the operand registers.
// Block scales are stored transposed, [k/32][ld], one float per row.
//
// Work: a workgroup of 4 waves computes a 64 x 64 output tile, wave w the
// 32 x 32 quarter at rows 32 (w >> 1), columns 32 (w & 1). Each wave loads
// its own activation and weight blocks and their scales straight into
// registers by buffer loads, three blocks ahead (93 VGPRs, five waves per
// SIMD: the 4,608 waves of gate|up all resident), with no LDS and no barrier
// (an LDS ring shared by the four waves, with a barrier per block, was no
// faster: the loop is bound by each wave's instruction stream, 24 or 36
// blocks of one MFMA and 48 VALU operations, not by its loads). Per block:
// block kb's two multiply phases, the MFMA of block kb + 1, block kb's
// adds, then the refill of kb's registers with block kb + 3. In the MFMA
// 32x32 output layout a lane holds one column and 16 rows; each row's
// activation scale reaches it through a DPP row broadcast folded into the
// multiply.
#include <algorithm>
#include <utility>

#include "eg2_device.hpp"
#include "eg2_kernels.hpp"

namespace eg2 {

typedef int intx4 __attribute__((ext_vector_type(4)));
typedef int intx16 __attribute__((ext_vector_type(16)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kXcds = 8;     // MI355X: 8 XCDs of 32 CUs, each with its own L2
constexpr int kDepth = 3;    // blocks in flight per wave in gemm_q8_kernel (93 VGPRs: five waves per SIMD)
constexpr int kUnroll = 6;   // its loop's unrolling: slots rotate mod kDepth, MFMA results mod 2
constexpr int kTile = 1024;  // one 32 x 32 int8 operand block
constexpr float kMagic = 12582912.0f;         // 1.5 * 2^23
constexpr int kMagicBits = 0x4B400000;

extern __shared__ __align__(16) unsigned char gemm_lds[];

// Broadcast of lane V of each 16-lane row to the whole row (row_newbcast).
template <int V>
__device__ __forceinline__ float row_bcast(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x150 + V, 0xf, 0xf, true));
}

// t[v] = (dot[v] * d_w) * d_x(row v) from the biased MFMA result; the
// lane's 16 output rows take their activation scales from lanes 0..15 of
// its 16-lane row. The two phases are kept apart so 16 independent
// operations separate each dependent pair; accumulate_products then adds
// t to acc (the third phase), after the next block's MFMA is issued.
template <int... V>
__device__ __forceinline__ floatx16 scale_products(const intx16& biased, float dw, float dxv,
                                                   std::integer_sequence<int, V...>) {
  const float bias = dw * -kMagic;
  const floatx16 f = __builtin_bit_cast(floatx16, biased);
  floatx16 t;
  ((t[V] = __builtin_fmaf(f[V], dw, bias)), ...);
  __builtin_amdgcn_sched_barrier(0);
  ((t[V] = t[V] * row_bcast<V>(dxv)), ...);
  return t;
}
template <int... V>
__device__ __forceinline__ void accumulate_products(floatx16& acc, const floatx16& t, std::integer_sequence<int, V...>) {
  ((acc[V] = acc[V] + t[V]), ...);
}

// The output tiles split into 8 regions, one per XCD: the row tiles in
// rparts parts and the column tiles in 8 / rparts, rparts chosen so that the
// fullest region holds the fewest tiles (the kernel lasts as long as its
// busiest XCD), ties going to 2 row parts, then 4, 8, 1. With 2 row parts an
// XCD's L2 fetches half of the activation rows and a quarter of the weight
// columns instead of all rows and an eighth of the columns (11 MB instead
// of 16 MB for gate|up at 2048 rows); the Q|K|V projection's 5 head columns
// split evenly only over 8 row parts (40 tiles per XCD at 2048 rows, where
// 2 row parts would give two XCDs nothing and two half the others' 64).
// rows_first (the O and down projections, whose output the residual kernel
// reads row by row) breaks ties toward 8 row parts instead: each XCD then
// computes whole rows, 256 of 2048, and the residual kernel's workgroups on
// that XCD take the same rows from its L2.
struct XcdRegions {
  int cparts, rows, cols;  // column parts; row and column tiles per region
};
__host__ __device__ inline XcdRegions xcd_split(int tr_count, int tc_count, bool rows_first = false) {
  XcdRegions best{0, 0, 0};
  const int order[2][4] = {{2, 4, 8, 1}, {8, 4, 2, 1}};
  for (int rparts : order[rows_first ? 1 : 0]) {
    const int cparts = kXcds / rparts;
    const XcdRegions r{cparts, (tr_count + rparts - 1) / rparts, (tc_count + cparts - 1) / cparts};
    if (best.cparts == 0 || r.rows * r.cols < best.rows * best.cols) best = r;
  }
  return best;
}
__host__ __device__ inline XcdRegions xcd_regions(int n, int m, bool rows_first = false) {
  return xcd_split((n + 63) / 64, (m + 63) / 64, rows_first);
}
__host__ inline dim3 gemm_grid(int n, int m, bool rows_first = false) {
  const XcdRegions reg = xcd_regions(n, m, rows_first);
  return dim3(kXcds * reg.rows * reg.cols);
}

// Floats per row of the GeGLU epilogue's transposed tile: odd, so that the
// 32 lanes of a half-wave reading one dword each of their row's 8-value
// part (8 rows x 4 parts) hit 32 distinct banks (row r at bank offset r,
// part p at 8 p). The reads are 4-byte (the compiler splits wider ones
// anyway), so nothing needs 16-byte alignment. Bank-conflict cycles per
// launch at 2048 x 2304: 1.03 M with a pitch of 40, 0.44 M with 36, 0 now.
constexpr int kGPitch = 33;

// GeGLU epilogue (kernels.c:367-391, engine.c's gelu(gate) * up then the
// Q8_0 quantization of the down projection's input). The weight rows are
// interleaved in 32-row groups (gate group j, then up group j), so output
// tile tc holds gate columns 32 tc .. 32 tc + 31 in its waves wc = 0 and
// the matching up columns in its waves wc = 1, and its 32 GeGLU outputs per
// row are exactly Q8_0 block tc. The two waves of a row pair write their
// tiles to LDS row-major and read them back transposed (the gate wave
// finishes rows 0-15 of the pair, the up wave rows 16-31), four lanes
// holding one row's block, and run the standalone GeGLU kernel's code
// (geglu_quantize_part4): the int8 values go to gq in the row-tile layout
// (nbf blocks per row), the scales to gd[tc * ldg + row].
// Minimum over each aligned quad of lanes, on every lane of it (all 64 lanes
// active).
__device__ __forceinline__ uint32_t quad_min_u32(uint32_t m) {
  m = min(m, (uint32_t)__builtin_amdgcn_mov_dpp((int)m, 0xB1, 0xf, 0xf, true));
  return min(m, (uint32_t)__builtin_amdgcn_mov_dpp((int)m, 0x4E, 0xf, 0xf, true));
}

// The exact GeGLU values of the workgroup's block-maximum candidates
// (geglu_quantize_part4, step 2) in one pass of one wave instead of one per
// wave: the workgroup's 4 waves hold 64 blocks (a quad of lanes each), and
// each block's first candidate -- the lowest one of the quad's lowest lane
// that has any; every block has one -- goes to LDS slot 16 w + quad; wave 0
// evaluates slot `lane` with gelu_mul, and the owner takes the value back
// into a[]. A block's other candidates (values within their bounds of its
// largest: rare) take the per-wave passes, which run only when some lane
// has one. All 256 threads must call it.
__device__ __forceinline__ void geglu_block_candidates(const float (&g)[8], const float (&u)[8], uint32_t cand,
                                                       float (&a)[8]) {
  __shared__ float slot_g[64], slot_u[64], slot_x[64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t own = cand ? ((uint32_t)(lane & 3) << 3) | (uint32_t)__builtin_ctz(cand) : 0xffu;
  const uint32_t key = quad_min_u32(own);
  const bool owner = (int)(key >> 3) == (lane & 3);
  const int k = (int)(key & 7), s = 16 * w + (lane >> 2);
  if (owner) {
    float gk = g[0], uk = u[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) {
      gk = k == i ? g[i] : gk;
      uk = k == i ? u[i] : uk;
    }
    slot_g[s] = gk;
    slot_u[s] = uk;
  }
  __syncthreads();
  if (w == 0) slot_x[lane] = gelu_mul(slot_g[lane], slot_u[lane]);
  __syncthreads();
  if (owner) {
    const float x = slot_x[s];
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = k == i ? x : a[i];
  }
  int32_t unused[8];
  geglu_exact_passes<false>(g, u, owner ? cand & ~(1u << k) : cand, 0.0f, a, unused);
}

__device__ __forceinline__ void geglu_epilogue(const floatx16& acc, int tr, int tc, int wr, int wc, int n, int nbf,
                                               int8_t* __restrict__ gq, float* __restrict__ gd, int ldg) {
  const int lane = threadIdx.x & 63, g = lane >> 5;
  // Wave (wr, wc) writes its 32 x 32 tile -- gate for wc = 0, up for wc = 1
  // -- into its matrix's transposed tile (register v: row 8 (v >> 2) + 4 g
  // + (v & 3), column lane & 31); the block loop leaves the LDS unused.
  float* tg = reinterpret_cast<float*>(gemm_lds) + wr * 2 * 32 * kGPitch;  // [32][kGPitch] gate, then up
  float* tu = tg + 32 * kGPitch;
  float* mine = wc == 0 ? tg : tu;
  const int trow = 4 * g * kGPitch + (lane & 31);
#pragma unroll
  for (int v = 0; v < 16; ++v) mine[trow + (8 * (v >> 2) + (v & 3)) * kGPitch] = acc[v];
  __syncthreads();
  const int rr = 16 * wc + (lane >> 2), part = lane & 3;
  float gs[8], us[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    gs[i] = tg[rr * kGPitch + 8 * part + i];
    us[i] = tu[rr * kGPitch + 8 * part + i];
  }
  const int t = 64 * tr + 32 * wr + rr;
  float a[8], bound[8];
  const uint32_t cand = geglu_approx_part4(gs, us, a, bound);
  geglu_block_candidates(gs, us, cand, a);  // a[] now exact for the candidates
  geglu_decide_part4(gs, us, bound, cand, a, t < n, gq + q8_tile_offset(t, 32 * tc + 8 * part, nbf),
                     gd + (size_t)tc * ldg + t);
}

// The block loop of one wave's 32 x 32 output tile, shared by the
// projection kernels: the activation block tile atile (1 KB per block, nb
// blocks) and its scales xd[kb * ldx + xoff / 4] (n rows), the weight block
// tile btile and its scales wd[kb * ldw + woff / 4] (m rows), xoff being
// the row whose scale this lane feeds to the DPP broadcast (srow) and woff
// the lane's column. Operands go straight to registers (the row-tile
// layout is the MFMA's register order: lane L's 16 bytes of a block are
// one load at 16 L) by buffer loads with a scalar offset per block, kDepth
// blocks ahead, with no LDS and no barrier: the waves of a workgroup never
// wait for each other. Each scale array is read through one descriptor,
// block kb's row at the scalar offset 4 kb ld (the launchers keep both
// arrays below 4 GiB: scales_fit), so a block's scale loads cost one
// scalar multiply each rather than a new 64-bit base and descriptor (12
// scalar instructions fewer per block and wave). Returns the tile in the
// 32x32 MFMA output layout.
template <bool TAIL>
__device__ __forceinline__ floatx16 q8_block_loop(const int8_t* atile, const float* __restrict__ xd, int ldx, int n,
                                                  uint32_t xoff, const int8_t* btile, const float* __restrict__ wd,
                                                  int ldw, int m, uint32_t woff, int nb, int lane) {
  // Buffer loads: the per-block advance is a scalar offset, so no vector
  // address is kept per block in flight.
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(atile, (uint32_t)nb * kTile);
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(btile, (uint32_t)nb * kTile);
  const __amdgpu_buffer_rsrc_t rx = buffer_rsrc(xd, 4u * ((uint32_t)(nb - 1) * (uint32_t)ldx + (uint32_t)n));
  const __amdgpu_buffer_rsrc_t rw = buffer_rsrc(wd, 4u * ((uint32_t)(nb - 1) * (uint32_t)ldw + (uint32_t)m));
  const uint32_t ldx4 = 4u * (uint32_t)ldx, ldw4 = 4u * (uint32_t)ldw;
  struct Frag {
    intx4 a, b;
    float dx, dw;
  };
  auto load = [&](Frag& f, int kb) {
    kb = min(kb, nb - 1);
    f.a = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(ra, 16u * lane, kb * kTile, 0));
    f.b = __builtin_bit_cast(intx4, __builtin_amdgcn_raw_buffer_load_b128(rb, 16u * lane, kb * kTile, 0));
    f.dx = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rx, xoff, (uint32_t)kb * ldx4, 0));
    f.dw = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rw, woff, (uint32_t)kb * ldw4, 0));
  };
  intx16 magic = (intx16)(kMagicBits);
  asm volatile("" : "+v"(magic));  // one register copy, not rebuilt per MFMA
  // Loads stay in block order (a, b, dx, dw per block; the scheduling
  // barriers keep the compiler from regrouping them), so that each wait
  // the compiler derives covers only the block it needs, here and across
  // the loop's back edge.
  Frag f[kDepth];
#pragma unroll
  for (int s = 0; s < kDepth; ++s) {
    load(f[s], s);
    __builtin_amdgcn_sched_barrier(0);
  }
  intx16 d[2];
  d[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[0].a, f[0].b, magic, 0, 0, 0);
  floatx16 acc = floatx16{};
  // One block: j = kb % kUnroll (a constant after unrolling, so the
  // fragment slot j % kDepth and the MFMA result register j % 2 are fixed
  // registers). Block kb's scaling, the MFMA of block kb + 1, block kb's
  // adds, then the slot refilled with block kb + kDepth.
  auto step = [&](int j, int kb) {
    const int cur = j & 1, nxt = cur ^ 1, slot = j % kDepth;
    const floatx16 t = scale_products(d[cur], f[slot].dw, f[slot].dx, std::make_integer_sequence<int, 16>{});
    __builtin_amdgcn_sched_barrier(0);
    d[nxt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[(j + 1) % kDepth].a, f[(j + 1) % kDepth].b, magic, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    accumulate_products(acc, t, std::make_integer_sequence<int, 16>{});
    __builtin_amdgcn_sched_barrier(0);
    load(f[slot], kb + kDepth);
    __builtin_amdgcn_sched_barrier(0);
  };
  int kb0 = 0;
  if constexpr (!TAIL) {
    // nb is a positive multiple of kUnroll: a loop without the entry test,
    // so the loads above stay in front of it in their order.
    do {
#pragma unroll
      for (int j = 0; j < kUnroll; ++j) step(j, kb0 + j);
      kb0 += kUnroll;
    } while (kb0 < nb);
  } else {
    for (; kb0 + kUnroll <= nb; kb0 += kUnroll) {
#pragma unroll
      for (int j = 0; j < kUnroll; ++j) step(j, kb0 + j);
    }
    // The last nb % kUnroll blocks (the branch stays out of the main loop,
    // whose straight-line body lets the DPP broadcasts fold into the multiplies).
#pragma unroll
    for (int j = 0; j < kUnroll - 1; ++j)
      if (kb0 + j < nb) step(j, kb0 + j);
  }
  return acc;
}

// TAIL: nb % kUnroll != 0 (a separate instantiation: the tail code costs
// registers, and every projection of the model has nb % 4 == 0). GEGLU:
// the epilogue above replaces the fp32 store (y and ldy unused; m = 2 ff).
template <bool TAIL, bool GEGLU>
__global__ void __launch_bounds__(256)
gemm_q8_kernel(const int8_t* __restrict__ xq, const float* __restrict__ xd, int ldx, const int8_t* __restrict__ wq,
               const float* __restrict__ wd, int ldw, float* __restrict__ y, int n, int m, int nb, int ldy,
               int8_t* __restrict__ gq, float* __restrict__ gd) {
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Issue priority 1: above the attention kernels (0), below the short
  // latency-bound row kernels (3), when other streams share the SIMDs.
  __builtin_amdgcn_s_setprio(1);
  // XCD-aware order: workgroup b runs on XCD b % 8, which takes one region
  // of the tile grid (column-group major inside it).
  const XcdRegions reg = xcd_regions(n, m, !GEGLU);
  const int x = (int)(blockIdx.x % kXcds), i = (int)(blockIdx.x / kXcds);
  const int r0 = (x / reg.cparts) * reg.rows, c0 = (x % reg.cparts) * reg.cols;
  const int rows_here = min(reg.rows, (n + 63) / 64 - r0), cols_here = min(reg.cols, (m + 63) / 64 - c0);
  if (rows_here <= 0 || cols_here <= 0 || i >= rows_here * cols_here) return;
  const int tr = r0 + i % rows_here, tc = c0 + i / rows_here;

  // Wave (wr, wc): activation rows 64 tr + 32 wr (clamped to the last
  // tile), weight columns 64 tc + 32 wc; scales clamped to the last row
  // and column.
  const int wr = w >> 1, wc = w & 1, g = lane >> 5;
  // Row whose scale this lane supplies to the DPP broadcast: lane 16r + v
  // carries the scale of output register v for the lanes of 16-lane row r.
  const int srow = 8 * ((lane & 15) >> 2) + 4 * g + (lane & 3);
  const floatx16 acc = q8_block_loop<TAIL>(
      xq + (size_t)min(2 * tr + wr, (n + 31) / 32 - 1) * nb * kTile, xd, ldx, n,
      4u * (uint32_t)min(64 * tr + 32 * wr + srow, n - 1),
      wq + (size_t)min(2 * tc + wc, (m + 31) / 32 - 1) * nb * kTile, wd, ldw, m,
      4u * (uint32_t)min(64 * tc + 32 * wc + (lane & 31), m - 1), nb, lane);
  if constexpr (GEGLU) {
    geglu_epilogue(acc, tr, tc, wr, wc, n, m / 64, gq, gd, ldy);
  } else {
    const int col = 64 * tc + 32 * wc + (lane & 31);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int row = 64 * tr + 32 * wr + 8 * (v >> 2) + 4 * g + (v & 3);
      if (row < n && col < m) y[(size_t)row * ldy + col] = acc[v];
    }
  }
}

// The kernel for nb blocks (TAIL: nb is not a multiple of kUnroll).
template <bool GEGLU>
static hipError_t launch_gemm_kernel(dim3 grid, size_t lds, hipStream_t st, const int8_t* xq, const float* xd,
                                     int ldx, const int8_t* wq, const float* wd, int ldw, float* y, int n, int m,
                                     int nb, int ldy, int8_t* gq, float* gd) {
  if (nb % kUnroll == 0)
    hipLaunchKernelGGL((gemm_q8_kernel<false, GEGLU>), grid, dim3(256), lds, st, xq, xd, ldx, wq, wd, ldw, y, n, m, nb,
                       ldy, gq, gd);
  else
    hipLaunchKernelGGL((gemm_q8_kernel<true, GEGLU>), grid, dim3(256), lds, st, xq, xd, ldx, wq, wd, ldw, y, n, m, nb,
                       ldy, gq, gd);
  return hipGetLastError();
}

// The block loop's scale descriptors: k / 32 rows of ld floats in at most
// 4 GiB - 1 bytes (the executor's arrays take a few hundred KB).
inline bool scales_fit(int k, int ld) { return (uint64_t)(k / kQK) * (uint64_t)ld * 4u <= 0xFFFFFFFFull; }

hipError_t launch_gemm_q8(const int8_t* xq, const float* xd, int ldx, const int8_t* wq, const float* wd, int ldw,
                          float* y, int n, int m, int k, int ldy, hipStream_t st) {
  if (n <= 0 || m <= 0 || k <= 0 || k % kQK != 0 || ldy < m || ldx < n || ldw < m) return hipErrorInvalidValue;
  if (!scales_fit(k, ldx) || !scales_fit(k, ldw)) return hipErrorInvalidValue;
  return launch_gemm_kernel<false>(gemm_grid(n, m, true), 0, st, xq, xd, ldx, wq, wd, ldw, y, n, m, k / kQK, ldy,
                                   nullptr, nullptr);
}

hipError_t launch_gemm_q8_geglu(const int8_t* xq, const float* xd, int ldx, const int8_t* wq, const float* wd, int ldw,
                                int8_t* gq, float* gd, int ldg, int n, int ff, int k, hipStream_t st) {
  const int m = 2 * ff;
  if (n <= 0 || ff <= 0 || ff % kQK != 0 || k <= 0 || k % kQK != 0 || ldx < n || ldw < m || ldg < n)
    return hipErrorInvalidValue;
  if (!scales_fit(k, ldx) || !scales_fit(k, ldw)) return hipErrorInvalidValue;
  // LDS: the epilogue's gate and up tiles
  constexpr size_t lds = 2 * 2 * 32 * kGPitch * sizeof(float);
  return launch_gemm_kernel<true>(gemm_grid(n, m), lds, st, xq, xd, ldx, wq, wd, ldw, nullptr, n, m, k / kQK, ldg, gq,
                                  gd);
}

// ---------------------------------------------------------------------------
// The Q|K|V projection with the QK-norm / RoPE epilogue (kernels.c:233-264 on
// each token of the projection's output): a workgroup of 8 waves computes 32
// token rows x one 256-wide head (head hc of [q0 q1 q2 | k | v]), wave w the
// 32 x 32 piece at columns 32 w, with the block loop of gemm_q8_kernel (so
// the projection's fp32 values are bit-identical to it). The epilogue puts
// the tile in LDS 16 rows at a time and, for q and k heads, runs each row's
// SSE2-order sum of squares (waves 0-1, 8 lanes per row), then (x*w)*inv, the NeoX rotation of
// pairs (d, d+128) with the host cos/sin row of the token's position, the
// 1/16 scale of q -- the operations and order of the standalone
// qk_norm_rope kernel -- and writes the rows [q0 q1 q2 | k | v] attention
// reads; the v head is the projection itself. The unnormalised projection
// never reaches HBM.
constexpr int kRowPitch = kHeadDim + 8;  // floats per token row of the epilogue tile (8 banks apart)
constexpr int kQkvHeads = kQKVCols / kHeadDim;  // 5

template <bool TAIL>
__global__ void __launch_bounds__(512)
gemm_q8_qkv_rope_kernel(const int8_t* __restrict__ xq, const float* __restrict__ xd, int ldx,
                        const int8_t* __restrict__ wq, const float* __restrict__ wd, int ldw, int n, int nb,
                        const float* __restrict__ q_w, const float* __restrict__ k_w, const float* __restrict__ rope,
                        const int32_t* __restrict__ pos, float eps, float* __restrict__ out) {
  __shared__ float invs[32];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Issue priority 1: above the attention kernels (0), below the short
  // latency-bound row kernels (3), when other streams share the SIMDs.
  __builtin_amdgcn_s_setprio(1);
  const XcdRegions reg = xcd_split((n + 31) / 32, kQkvHeads);
  const int x = (int)(blockIdx.x % kXcds), i = (int)(blockIdx.x / kXcds);
  const int r0 = (x / reg.cparts) * reg.rows, c0 = (x % reg.cparts) * reg.cols;
  const int rows_here = min(reg.rows, (n + 31) / 32 - r0), cols_here = min(reg.cols, kQkvHeads - c0);
  if (rows_here <= 0 || cols_here <= 0 || i >= rows_here * cols_here) return;
  const int tr = r0 + i % rows_here, hc = c0 + i / rows_here;

  // Wave w: the activation rows of tile tr and weight columns 32 w of head
  // hc, through the projection kernels' block loop (no LDS ring, no
  // barrier).
  const int g = lane >> 5;
  const int srow = 8 * ((lane & 15) >> 2) + 4 * g + (lane & 3);
  const floatx16 acc = q8_block_loop<TAIL>(
      xq + (size_t)tr * nb * kTile, xd, ldx, n, 4u * (uint32_t)min(32 * tr + srow, n - 1),
      wq + (size_t)(8 * hc + w) * nb * kTile, wd, ldw, kQKVCols,
      4u * (uint32_t)(kHeadDim * hc + 32 * w + (lane & 31)), nb, lane);
  // The epilogue runs on the tile in two halves of 16 token rows through a
  // 16-row LDS tile (17 KB per workgroup, not 34 KB). Its global inputs go
  // out now, so their latency overlaps the tile's trip through LDS and the
  // sums of squares: the norm weights, and the cos/sin of this wave's two
  // rows of each half (rows 16 hf + 2 w + rr).
  constexpr int half = kHeadDim / 2;
  const bool is_v = hc == kHeads + 1;
  const float* wgt = hc < kHeads ? q_w : k_w;
  float cs_r[2][2][4], w_r[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    w_r[2 * j] = wgt[lane + 64 * j];
    w_r[2 * j + 1] = wgt[lane + 64 * j + half];
  }
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int t = min(32 * tr + 16 * hf + 2 * w + rr, n - 1);
      const float* cs = rope + (size_t)pos[t] * kHeadDim;  // [cos 0..127 | sin 0..127]
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        cs_r[hf][rr][2 * j] = cs[lane + 64 * j];
        cs_r[hf][rr][2 * j + 1] = cs[half + lane + 64 * j];
      }
    }
  float* tile = reinterpret_cast<float*>(gemm_lds);  // [16][kRowPitch]
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    if (hf) __syncthreads();  // the first half's tile is no longer read
    // Register v holds row 8 (v >> 2) + 4 g + (v & 3): rows 0-15 are
    // v = 0..7, rows 16-31 v = 8..15.
#pragma unroll
    for (int v = 8 * hf; v < 8 * hf + 8; ++v)
      tile[(8 * (v >> 2) + 4 * g + (v & 3) - 16 * hf) * kRowPitch + 32 * w + (lane & 31)] = acc[v];
    __syncthreads();
    if (is_v) {
      // v: the projection as it is; wave w copies rows 2w, 2w + 1 of the half.
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const int row = 2 * w + rr, t = 32 * tr + 16 * hf + row;
        if (t >= n) break;
        float* vrow = out + (size_t)t * kQKVCols + kHeads * kHeadDim + kHeadDim;
        *reinterpret_cast<float4*>(vrow + 4 * lane) =
            *reinterpret_cast<const float4*>(tile + row * kRowPitch + 4 * lane);
      }
      continue;
    }
    // kernels.c:233-264 for q head hc (hc < 3) or k (hc == 3): waves 0-1
    // run the half's 16 rows' SSE2 sums of squares, 8 lanes per row.
    if (w < 2) {
      const int row = 8 * w + (lane >> 3);
      const float ss = sse2_combine(sse2_chain<kHeadDim>(tile + row * kRowPitch, lane & 7));
      if ((lane & 7) == 0) invs[16 * hf + row] = rms_inverse(ss, kHeadDim, eps);
    }
    __syncthreads();
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int row = 2 * w + rr, t = 32 * tr + 16 * hf + row;
      if (t >= n) break;
      const float inv = invs[16 * hf + row];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int dd = lane + 64 * j;
        const float c = cs_r[hf][rr][2 * j], s = cs_r[hf][rr][2 * j + 1];
        const float x0 = tile[row * kRowPitch + dd] * w_r[2 * j] * inv;
        const float x1 = tile[row * kRowPitch + dd + half] * w_r[2 * j + 1] * inv;
        const float a0 = x0 * c, a1 = x1 * s;
        const float b0 = x0 * s, b1 = x1 * c;
        float lo = a0 - a1, hi = b0 + b1;
        if (hc < kHeads) {
          lo = lo * 0.0625f;
          hi = hi * 0.0625f;
        }
        float* orow = out + (size_t)t * kQKVCols + hc * kHeadDim;
        orow[dd] = lo;
        orow[dd + half] = hi;
      }
    }
  }
}

hipError_t launch_gemm_q8_qkv_rope(const int8_t* xq, const float* xd, int ldx, const int8_t* wq, const float* wd,
                                   int ldw, int n, int k, const float* q_w, const float* k_w, const float* rope,
                                   const int32_t* pos, float eps, float* out, hipStream_t st) {
  if (n <= 0 || k <= 0 || k % kQK != 0 || ldx < n || ldw < kQKVCols) return hipErrorInvalidValue;
  if (!scales_fit(k, ldx) || !scales_fit(k, ldw)) return hipErrorInvalidValue;
  const XcdRegions reg = xcd_split((n + 31) / 32, kQkvHeads);
  const dim3 grid(kXcds * reg.rows * reg.cols);
  const int nb = k / kQK;
  constexpr size_t lds = 16 * kRowPitch * sizeof(float);  // the epilogue's 16-row tile
  if (nb % kUnroll == 0)
    hipLaunchKernelGGL(gemm_q8_qkv_rope_kernel<false>, grid, dim3(512), lds, st, xq, xd, ldx, wq, wd, ldw, n, nb, q_w,
                       k_w, rope, pos, eps, out);
  else
    hipLaunchKernelGGL(gemm_q8_qkv_rope_kernel<true>, grid, dim3(512), lds, st, xq, xd, ldx, wq, wd, ldw, n, nb, q_w,
                       k_w, rope, pos, eps, out);
  return hipGetLastError();
}

}  // namespace eg2
