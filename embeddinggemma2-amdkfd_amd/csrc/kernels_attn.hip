// Packed variable-length bidirectional GQA attention (3 query heads, 1 KV
// head, head_dim 256) on MFMA, for a wave of sequences packed back to back.
//
// Reference semantics (kernels.c:324-360 per segment, engine.c:850-873): a
// query token attends to every key of its own sequence (window == 0) or to
// keys with |q - k| <= window/2 inside it; softmax(q.k) with q already
// scaled by 1/16; the context row is then quantized to Q8_0 for the output
// projection (engine.c:644-648), which this kernel does in its epilogue.
//
// Precision: q, k, v arrive as fp32 values split into fp16 pairs
// (hi = fp16(x), lo = fp16(x - hi); q pre-multiplied by 16 to stay clear of
// fp16 subnormals), and the probabilities are split the same way, so every
// product is formed as hi*hi + hi*lo + lo*hi on v_mfma_f32_16x16x32_f16 with
// fp32 accumulation: about 2^-21 relative error per product, i.e. fp32-level
// attention. Softmax runs in fp32 (online, one pass over 32-key tiles) in
// log2 units with the hardware exp2.
//
// Work: query tiles of up to 32 tokens of ONE sequence (host-built list:
// first query, end, sequence start, sequence end, key chunk, partial slot);
// the query and key tiles of a sequence start at its first token, so a
// query's arithmetic depends only on its own sequence and packed and
// single-sequence calls give bit-identical results. One workgroup of six
// waves per query tile: wave w computes head w % 3 for the 16-query block
// w / 3; all six share each 32-key tile of K and V^T in LDS, so a K/V byte
// brought in serves 32 queries of 3 heads. The waves of a second block that
// a short tile does not have only move data.
//
// Data movement: K rows ([hi 256 | lo 256] fp16 per token) and V^T rows
// (V transposed by the QK-norm/RoPE kernel into [hi|lo][256 dims][column],
// each sequence starting at a 32-aligned column, so a key tile is 64
// contiguous bytes per dimension) go from global memory straight into a
// double-buffered LDS ring by DMA (global_load_lds_dwordx4), the next tile
// in flight while the current one is used. 16-byte chunks are XOR-swizzled
// so the MFMA fragment reads hit distinct banks.
//
// Scores are computed transposed, S^T = K . Q^T, as two 16-key x 16-query
// blocks, so each lane owns one query (lane & 15) and 8 of the tile's keys
// and the softmax reductions stay in the lane plus exchanges with lanes 16
// and 32 away. The K rows are fed to the score MFMA in a permuted order
// chosen so that lane group j (lanes 16j..16j+15) ends up holding the
// probabilities of keys 8j..8j+7: exactly the k-slots it supplies to the
// P.V MFMA, whose V^T operand is then one aligned 16-byte chunk per lane.
#include <algorithm>
#include <cfloat>
#include <type_traits>

#include "eg2_device.hpp"
#include "eg2_kernels.hpp"

namespace eg2 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kQBlock = 16;           // queries per wave (one 16x16x32 MFMA column block)
constexpr int kQTile = 2 * kQBlock;    // queries per work tile (workgroup)
constexpr int kKvTile = 32;  // keys per LDS stage (one 32-deep MFMA reduction)
constexpr int kKStage = kKvTile * 2 * kHeadDim * 2;  // [key][hi|lo][256] fp16 = 32 KB
constexpr int kVStage = 2 * kHeadDim * kKvTile * 2;  // [hi|lo][dim][32 keys] fp16 = 32 KB
constexpr int kStage = kKStage + kVStage;
constexpr float kLog2e = 1.4426950408889634f;
// A workgroup runs 6 waves, 3 heads x 2 query blocks. All six issue the
// K/V DMA: its throughput grows with the number of waves issuing it
// (measured on this part: 5.1, 9.5 and 14.4 TB/s for 3, 6 and 12 waves
// streaming 64 KB tiles, one workgroup per CU), and the 64 DMA instructions
// of a tile are spread over all six.
constexpr int kWaves = 2 * kHeads;
constexpr int kDmaPerWave = (kKvTile + kWaves - 1) / kWaves;  // 6 K and 6 V instructions
constexpr uint32_t kNoSlot = 0xFFFFFFFFu;           // item writes the final context
constexpr int kPartFloats = 16 * 64 * 4 + 64 * 2;   // per (slot, block, head): acc in lane order, then (m, l)
constexpr uint32_t kSplitLen = 256;  // longer sequences split their keys into chunks ...
constexpr uint32_t kMaxChunks = 4;   // ... of at least kSplitLen keys, at most this many

__device__ __forceinline__ floatx4 mfma(const half8& a, const half8& b, const floatx4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// LDS DMA from a wave-uniform global base (SGPR pair) plus a per-lane byte
// offset, 16 bytes per lane, to the wave-uniform LDS address `lds` (+16
// bytes per lane), which the instruction takes from M0 (this kernel has no
// other M0 user). The saddr form keeps one 32-bit offset per lane instead
// of a 64-bit address.
__device__ __forceinline__ void dma16(const void* base, unsigned off, unsigned lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
               : "memory", "m0");
}

// Key fed to row i of key block kb of the score MFMA. Output row r = 4j + v
// of a 16x16 block lands in lane group j (lanes 16j..16j+15) as register v,
// so this order gives lane group j the keys 8j..8j+7 -- the k-slots it
// supplies to the P.V MFMA.
__host__ __device__ constexpr int score_key(int kb, int i) { return 8 * (i >> 2) + 4 * kb + (i & 3); }
// Chunk swizzles. K rows (32 chunks of 16 bytes per half): XOR with a key
// hash that is distinct over the 16 keys one score block reads. V^T rows
// (4 chunks of a 64-byte row): XOR with (row >> 1) & 3. Both were chosen by
// measurement (SQ_LDS_BANK_CONFLICT over the fragment read patterns on
// this part): the V^T pattern must differ between rows 2i and 2i + 1 --
// an XOR of ((row >> 1) ^ (row >> 3)) & 3, distinct over every 4 rows 64
// bytes apart, still cost 4 conflict cycles per ds_read_b128.
__host__ __device__ constexpr int kswz(int key) { return (key & 3) | ((key >> 3) << 2); }
__host__ __device__ constexpr int vswz(int d) { return (d >> 1) & 3; }
// What the kernel's precomputed fragment offsets rely on: the second score
// block's key is the first's + 4 with the same K swizzle (below 16), and
// the V^T swizzle of dim row 16 d + q depends on d only through d & 1.
constexpr bool fragment_offsets_hold() {
  for (int q = 0; q < 16; ++q) {
    if (score_key(1, q) != score_key(0, q) + 4 || kswz(score_key(1, q)) != kswz(score_key(0, q)) ||
        kswz(score_key(0, q)) >= 16)
      return false;
    for (int d = 0; d < 16; ++d)
      if (vswz(16 * d + q) != vswz(16 * (d & 1) + q)) return false;
  }
  return true;
}
static_assert(fragment_offsets_hold(), "attention fragment offsets");

// Final context of NB Q8_0 blocks of one wave (16 queries x one head):
// context = acc / l, then Q8_0 per 32 dims (quants.c:97-177). f[2j] and
// f[2j+1] are the 16-dim MFMA blocks 2(b0+j) and 2(b0+j)+1: lane group grp
// holds dims 32b + 4grp + v and 32b + 16 + 4grp + v of query t, so a Q8_0
// block spans the four lane groups. The int8 values go to the row-tile
// layout of the projection GEMM (4 bytes per lane and half-block), the
// scales transposed ([block][row]). The blocks run phase by phase so their
// latencies overlap.
template <int NB>
__device__ __forceinline__ void store_blocks(const floatx4 (&f)[2 * NB], float l_run, uint32_t t, bool active,
                                             int head, int grp, int rows, int b0, int8_t* __restrict__ cq,
                                             float* __restrict__ cd) {
  const float inv_l = 1.0f / l_run;
  float vals[NB][8], amax[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    amax[b] = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      vals[b][v] = f[2 * b][v] * inv_l;
      vals[b][4 + v] = f[2 * b + 1][v] * inv_l;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) amax[b] = fmaxf(amax[b], fabsf(vals[b][i]));
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) amax[b] = rows4_max(amax[b]);
  // Row t of the row tiles: 32-row tile t/32, row t%32; this head's
  // blocks are 8 head .. 8 head + 7 of the row's 24.
  int8_t* qrow_out = cq + (size_t)(t >> 5) * (kEmbd / kQK) * 1024 + (size_t)(head * 8 + b0) * 1024 + (t & 31) * 16 +
                     4 * grp;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const float d = div127(amax[b]);
    const float id = amax[b] == 0.0f ? 0.0f : 1.0f / d;
    int32_t qv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) qv[i] = q8_round(vals[b][i] * id);  // id = 0 for an all-zero block
    if (active) {
      *reinterpret_cast<uint32_t*>(qrow_out + b * 1024) = pack_i8x4(qv[0], qv[1], qv[2], qv[3]);
      *reinterpret_cast<uint32_t*>(qrow_out + b * 1024 + 512) = pack_i8x4(qv[4], qv[5], qv[6], qv[7]);
      if (grp == 0) cd[(size_t)(head * 8 + b0 + b) * rows + t] = fp16_bits_to_fp32(fp32_to_fp16_bits(d));
    }
  }
}

__global__ void __launch_bounds__(64 * kWaves)
attention_kernel(const _Float16* __restrict__ qs, const _Float16* __restrict__ ks, const _Float16* __restrict__ vt,
                 int ldv, const uint4* __restrict__ items,
                 const uint32_t* __restrict__ item_count, int window, int rows, int8_t* __restrict__ cq,
                 float* __restrict__ cd, float* __restrict__ partials) {
  __shared__ __align__(16) unsigned char lds[2 * kStage];

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int head = w % kHeads, qb = w / kHeads;
  const int qi = lane & 15, grp = lane >> 4;
  const uint32_t count = *item_count;
  const unsigned lds0 = (unsigned)(uintptr_t)lds;
  for (uint32_t item = blockIdx.x; item < count; item += gridDim.x) {
    // Item fields are clamped to the wave so a malformed list can never
    // address outside the rows (an empty key range yields a non-finite row).
    const uint4 tl = items[2 * item], kc = items[2 * item + 1];
    const uint32_t seg_hi = min(tl.w, (uint32_t)rows);
    const uint32_t seg_lo = min(tl.z, seg_hi);
    const uint32_t q_end = min(tl.y, (uint32_t)rows);
    const uint32_t q0 = tl.x;
    // Key chunk of this item ([seg_lo, seg_hi) when unsplit; chunk starts
    // sit a multiple of 32 keys after seg_lo) and its partial-result slot.
    const uint32_t c_hi = min(kc.y, seg_hi), c_lo = min(max(kc.x, seg_lo), c_hi);
    const uint32_t slot = kc.z;
    // This wave's 16 queries; a block past the tile's end only moves data.
    const uint32_t qw = q0 + kQBlock * qb;
    const bool compute = qw < q_end;
    const bool active = qw + qi < q_end;
    const uint32_t t = active ? qw + qi : (q_end > 0 ? q_end - 1 : 0);

    // Key range of query u (kernels.c:330-336 in packed coordinates); both
    // ends are nondecreasing in u.
    const uint32_t half = (uint32_t)(window / 2);
    auto range_lo = [&](uint32_t u) { return window > 0 && u > half && u - half > seg_lo ? u - half : seg_lo; };
    auto range_hi = [&](uint32_t u) { return window > 0 && u + half + 1 < seg_hi ? u + half + 1 : seg_hi; };
    uint32_t lo = range_lo(t), hi = range_hi(t);
    // Union and intersection of the key ranges of the tile's queries
    // q0 .. q_end - 1 (the same for all six waves); without a window both
    // are the sequence.
    const uint32_t q_last = q_end > q0 ? q_end - 1 : q0;
    uint32_t kv_lo = range_lo(q0), kv_hi = range_hi(q_last), in_lo = range_lo(q_last), in_hi = range_hi(q0);
    kv_lo = __builtin_amdgcn_readfirstlane(max(kv_lo, c_lo));
    kv_hi = __builtin_amdgcn_readfirstlane(min(kv_hi, c_hi));
    in_lo = __builtin_amdgcn_readfirstlane(max(in_lo, c_lo));
    in_hi = __builtin_amdgcn_readfirstlane(min(in_hi, c_hi));
    lo = max(lo, c_lo);
    hi = min(hi, c_hi);
    // Key tiles are aligned to the sequence start; so are the V^T columns.
    const uint32_t k_first = kv_lo >= kv_hi ? kv_hi : seg_lo + ((kv_lo - seg_lo) & ~31u);
    // V^T column of key u: the sequence's first column (from the item, so
    // the first V DMA does not wait on a second dependent load) + u - seg_lo.
    const int col_base = (int)kc.w - (int)seg_lo;

    // DMA of key tile k0 into stage s, 64 instructions of 1 KB split over
    // the six waves: wave w issues K instruction q and V instruction q for
    // q = min(w + 6j, 31), j = 0..5 (the clamped repeats write the same
    // bytes to the same place). Issued unconditionally -- no branch splits
    // the MFMA loops -- with key rows clamped to the wave.
    // K: row of key q; lane L takes half L/32, stored chunk L%32 = global
    // chunk (L%32) ^ kswz(q). V: V^T rows 16(q%16)..+15 of half q/16; lane L
    // takes dim row L/4, stored chunk L%4 = global chunk (L%4) ^ vswz(row).
    auto dma_k = [&](uint32_t k0, int s, int j) {
      const int q = min(w + kWaves * j, kKvTile - 1);
      const uint32_t key = min(k0 + q, (uint32_t)rows - 1);
      const unsigned off = 2u * ((lane >> 5) * kHeadDim + 8 * ((lane & 31) ^ kswz(q)));
      dma16(ks + (size_t)key * (2 * kHeadDim), off, __builtin_amdgcn_readfirstlane(lds0 + s * kStage + q * 1024));
    };
    auto dma_v = [&](uint32_t k0, int s, int j) {
      const int q = min(w + kWaves * j, kKvTile - 1);
      const int hl = q >> 4, d = 16 * (q & 15) + (lane >> 2), c = (lane & 3) ^ vswz(d);
      const int col = max(0, min(col_base + (int)k0, ldv - kKvTile));  // the refill past a sequence stays inside vt
      const unsigned off = 2u * (unsigned)(((hl * kHeadDim + d) * ldv) + col + 8 * c);
      dma16(vt, off, __builtin_amdgcn_readfirstlane(lds0 + s * kStage + kKStage + q * 1024));
    };

    // Every wave has finished with both stages (previous tile of the grid
    // stride), and every DMA it issued -- including the refill of the idle
    // stage on its last key tile -- has landed, before the first DMA of
    // this tile overwrites them: each wave drains its own DMA, then issues
    // its query loads, then meets the others at a plain s_barrier (no
    // memory wait, so the query loads fly across it).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // Q^T operand of the score MFMA: lane holds query t, dims 32s + 8grp .. +7
    // for s = 0..7. Rows of qs are [hi 768 | lo 768].
    half8 qh[8], ql[8];
    if (compute) {
      const _Float16* qrow = qs + (size_t)t * (2 * kEmbd) + head * kHeadDim;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        qh[s] = *reinterpret_cast<const half8*>(qrow + 32 * s + 8 * grp);
        ql[s] = *reinterpret_cast<const half8*>(qrow + kEmbd + 32 * s + 8 * grp);
      }
    }
    __builtin_amdgcn_s_barrier();
    if (k_first < kv_hi) {
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j) {
        dma_k(k_first, 0, j);
        dma_v(k_first, 0, j);
      }
    }

    floatx4 acc[16];
#pragma unroll
    for (int db = 0; db < 16; ++db) acc[db] = floatx4{};
    // Running max in log2 units; -FLT_MAX (not -inf) until a key is in
    // range, so exp2 of a masked score (-inf) minus it is 0 and exp2 of it
    // minus a real maximum is 0, with no test.
    float m_run = -FLT_MAX, l_run = 0.0f;

    // Lane-varying LDS byte offsets of the fragment reads, fixed for the
    // item; the stage and the MFMA step only add immediates. K: key row
    // key0 (key1 = key0 + 4 has the same swizzle, 4 KB further), chunk
    // (4 st + grp) ^ kf = 4 (st ^ (kf >> 2)) + (grp ^ (kf & 3)), and
    // st ^ (kf >> 2) = (st & 4) + ((st & 3) ^ (kf >> 2)) for kf < 16.
    // V^T: dim row e = 16 d + qi, chunk grp ^ vswz(e), where vswz(e)
    // depends on d only through d & 1.
    const int key0 = score_key(0, qi), kf = kswz(key0);
    int kofs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) kofs[j] = key0 * 1024 + 64 * (j ^ (kf >> 2)) + 16 * (grp ^ (kf & 3));
    int vofs[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) vofs[p] = kKStage + 64 * qi + 16 * (grp ^ vswz(16 * p + qi));

    // One 32-key tile in LDS stage S (a compile-time constant, so every
    // fragment address is a per-item register plus an immediate).
    auto key_tile = [&](uint32_t k0, auto stage_tag) {
      constexpr int S = decltype(stage_tag)::value;
      // This tile's DMA (and the queries) have landed for every wave, and
      // every wave is done with the other stage, which the next tile's DMA
      // now refills (on the last tile: a harmless refill of the idle stage).
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      const uint32_t k1 = k0 + kKvTile;
      if (!compute) {
#pragma unroll
        for (int j = 0; j < kDmaPerWave; ++j) {
          dma_k(k1, S ^ 1, j);
          dma_v(k1, S ^ 1, j);
        }
        return;
      }
      const unsigned char* st_base = lds + S * kStage;

      // Fragment reads run one MFMA step ahead of their use (two register
      // sets), so the LDS latency overlaps the previous step's MFMAs.
      struct KFrag {
        half8 ah, al, bh, bl;  // key rows key0 / key0 + 4, hi and lo halves
      };
      auto kfrag = [&](int st) {
        const unsigned char* krow = st_base + kofs[st & 3] + 256 * (st >> 2);
        KFrag f;
        f.ah = *reinterpret_cast<const half8*>(krow);
        f.al = *reinterpret_cast<const half8*>(krow + 512);
        f.bh = *reinterpret_cast<const half8*>(krow + 4096);
        f.bl = *reinterpret_cast<const half8*>(krow + 4096 + 512);
        return f;
      };
      struct VFrag {
        half8 h0, l0, h1, l1;  // V^T rows of 16-dim blocks 2 pr and 2 pr + 1
      };
      auto vfrag = [&](int pr) {
        const unsigned char* v0 = st_base + vofs[0] + 1024 * (2 * pr);
        const unsigned char* v1 = st_base + vofs[1] + 1024 * (2 * pr + 1);
        VFrag f;
        f.h0 = *reinterpret_cast<const half8*>(v0);
        f.l0 = *reinterpret_cast<const half8*>(v0 + kHeadDim * 64);
        f.h1 = *reinterpret_cast<const half8*>(v1);
        f.l1 = *reinterpret_cast<const half8*>(v1 + kHeadDim * 64);
        return f;
      };

      // S^T = K . Q^T, two 16-key blocks; this wave's share of the next
      // tile's K rows goes out between the MFMAs.
      floatx4 s0 = floatx4{}, s1 = floatx4{};
      KFrag kfr[2];
      kfr[0] = kfrag(0);
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        if (st + 1 < 8) kfr[(st + 1) & 1] = kfrag(st + 1);
        __builtin_amdgcn_sched_barrier(0);  // keep the prefetch above this step's MFMAs
        const KFrag& f = kfr[st & 1];
        s0 = mfma(f.ah, qh[st], s0);
        s1 = mfma(f.bh, qh[st], s1);
        s0 = mfma(f.ah, ql[st], s0);
        s1 = mfma(f.bh, ql[st], s1);
        s0 = mfma(f.al, qh[st], s0);
        s1 = mfma(f.bl, qh[st], s1);
        if (st < kDmaPerWave) dma_k(k1, S ^ 1, st);
      }
      // The first V^T fragments go out before the softmax.
      VFrag vfr[2];
      vfr[0] = vfrag(0);
      __builtin_amdgcn_sched_barrier(0);
      // sc[4kb + v] = 16 x the score of key k0 + 8grp + 4kb + v, taken to
      // log2 units: exp(x) = exp2(x * log2e).
      float sc[8];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        sc[v] = s0[v] * (0.0625f * kLog2e);
        sc[4 + v] = s1[v] * (0.0625f * kLog2e);
      }
      // Masking only where some key of the tile is outside some query's range.
      if (k0 < in_lo || k0 + kKvTile > in_hi) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t key = k0 + 8 * grp + i;
          if (key < lo || key >= hi) sc[i] = -INFINITY;
        }
      }
      float mt = sc[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) mt = fmaxf(mt, sc[i]);
      const float m_new = fmaxf(m_run, rows4_max(mt));
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      float psum = 0.0f;
      half8 ph, pl;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p = __builtin_amdgcn_exp2f(sc[i] - m_new);
        psum += p;
        const _Float16 h = (_Float16)p;
        ph[i] = h;
        pl[i] = (_Float16)(p - (float)h);
      }
      l_run = l_run * alpha + rows4_sum(psum);
      m_run = m_new;
      // alpha is exactly 1 in every lane whose maximum did not grow; skip
      // the rescale when that holds for the whole wave (most tiles), and on
      // the first tile, where acc is still zero.
      if (k0 != k_first && __builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int db = 0; db < 16; ++db) acc[db] *= alpha;
      }

      // O^T += V^T . P^T: lane group grp supplies keys 8grp..8grp+7, V^T chunk
      // grp; each accumulator's three MFMAs (hi.hi, hi.lo, lo.hi, in that
      // order) alternate with the next block's. This wave's share of the
      // next tile's V^T rows goes out between them.
#pragma unroll
      for (int pr = 0; pr < 8; ++pr) {
        const int d0 = 2 * pr, d1 = 2 * pr + 1;
        if (pr + 1 < 8) vfr[(pr + 1) & 1] = vfrag(pr + 1);
        __builtin_amdgcn_sched_barrier(0);
        const VFrag& f = vfr[pr & 1];
        acc[d0] = mfma(f.h0, ph, acc[d0]);
        acc[d1] = mfma(f.h1, ph, acc[d1]);
        acc[d0] = mfma(f.h0, pl, acc[d0]);
        acc[d1] = mfma(f.h1, pl, acc[d1]);
        acc[d0] = mfma(f.l0, ph, acc[d0]);
        acc[d1] = mfma(f.l1, ph, acc[d1]);
        if (pr < kDmaPerWave) dma_v(k1, S ^ 1, pr);
      }
    };
    // Key tiles alternate between the two stages, starting in stage 0.
    for (uint32_t k0 = k_first; k0 < kv_hi;) {
      key_tile(k0, std::integral_constant<int, 0>{});
      if ((k0 += kKvTile) >= kv_hi) break;
      key_tile(k0, std::integral_constant<int, 1>{});
      k0 += kKvTile;
    }
    if (!compute) continue;

    if (slot == kNoSlot) {
      store_blocks<8>(acc, l_run, t, active, head, grp, rows, 0, cq, cd);
    } else {
      // Partial result of this key chunk: the unnormalised context and the
      // running max / sum, in the lane order of the MFMA layout (16-byte
      // stores, fully coalesced); attention_merge_kernel combines the parts.
      float* part = partials + (((size_t)slot * 2 + qb) * kHeads + head) * kPartFloats;
#pragma unroll
      for (int db = 0; db < 16; ++db) reinterpret_cast<floatx4*>(part)[db * 64 + lane] = acc[db];
      reinterpret_cast<float2*>(part + 16 * 64 * 4)[lane] = make_float2(m_run, l_run);
    }
  }
  // Drain any DMA still in flight before the workgroup's LDS is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Merges the key-chunk partials of split query tiles. One workgroup per
// (query tile, 16-query block, quarter of the head dimension), one wave per
// head, lanes in the attention kernel's MFMA layout; a quarter is 4 of the 16 16-dim
// blocks, i.e. 2 whole Q8_0 blocks, so it quantizes on its own. With m =
// max over parts of the running maxima (log2 units), l = sum_p l_p
// 2^(m_p - m) and acc = sum_p acc_p 2^(m_p - m), in part order (a
// deterministic order that depends only on the sequence), then the same
// epilogue as an unsplit tile. Every load of a wave is issued before its
// first use: the (m, l) pairs of all parts, then all parts' 4 x 16 bytes.
constexpr int kMaxParts = kMaxChunks;
__global__ void __launch_bounds__(192)
attention_merge_kernel(const uint4* __restrict__ merges, const uint32_t* __restrict__ merge_count,
                       const float* __restrict__ partials, int rows, int8_t* __restrict__ cq,
                       float* __restrict__ cd) {
  const int lane = threadIdx.x & 63, head = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qi = lane & 15, grp = lane >> 4;
  const uint32_t count = 8 * *merge_count;
  for (uint32_t wi = blockIdx.x; wi < count; wi += gridDim.x) {
    const uint4 mg = merges[wi >> 3];
    const int quarter = (int)(wi & 3), qb = (int)((wi >> 2) & 1);
    const uint32_t q_end = min(mg.y, (uint32_t)rows), qw = mg.x + kQBlock * qb, first = mg.z;
    if (qw >= q_end) continue;  // a tile with a single 16-query block
    const uint32_t parts = min(mg.w, (uint32_t)kMaxParts);
    const bool active = qw + qi < q_end;
    const uint32_t t = active ? qw + qi : q_end - 1;
    const float* base = partials + (((size_t)first * 2 + qb) * kHeads + head) * kPartFloats;
    const size_t stride = (size_t)2 * kHeads * kPartFloats;  // next part
    float2 ml[kMaxParts];
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p)
      ml[p] = p < (int)parts ? reinterpret_cast<const float2*>(base + p * stride + 16 * 64 * 4)[lane]
                             : make_float2(-INFINITY, 0.0f);
    floatx4 a[kMaxParts][4];
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[p][i] = p < (int)parts ? reinterpret_cast<const floatx4*>(base + p * stride)[(4 * quarter + i) * 64 + lane]
                                 : floatx4{};
    float m = -INFINITY;
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p) m = fmaxf(m, ml[p].x);
    floatx4 acc[4] = {floatx4{}, floatx4{}, floatx4{}, floatx4{}};
    float l = 0.0f;
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p) {
      if (p >= (int)parts) break;
      const float w = ml[p].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml[p].x - m);
      l = l + ml[p].y * w;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][v] = acc[i][v] + a[p][i][v] * w;
    }
    store_blocks<2>(acc, l, t, active, head, grp, rows, 2 * quarter, cq, cd);
  }
}

// Key chunks of a sequence of length n: one when n <= kSplitLen, else
// min(ceil(n / kSplitLen), kMaxChunks) chunks of chunk_keys(n) keys (a
// multiple of 32, so key tiles stay aligned to the sequence start; the last
// chunk takes the rest). Both depend only on n, so a sequence is computed
// the same way wherever it sits in a wave.
static size_t key_chunks(size_t n) {
  return n <= kSplitLen ? 1 : std::min<size_t>((n + kSplitLen - 1) / kSplitLen, kMaxChunks);
}
static size_t chunk_keys(size_t n) {
  const size_t c = key_chunks(n), per = (n + c - 1) / c;
  return (per + kKvTile - 1) / kKvTile * kKvTile;
}

AttentionCounts build_attention_items(const size_t* offsets, size_t batch, uint32_t* items, uint32_t* merges) {
  AttentionCounts c{0, 0, 0};
  size_t col = 0;  // first V^T column of sequence s, as build_vt_columns lays them out
  for (size_t s = 0; s < batch; ++s) {
    const size_t lo = offsets[s], hi = offsets[s + 1], chunks = key_chunks(hi - lo), ck = chunk_keys(hi - lo);
    for (size_t q = lo; q < hi; q += kQTile) {
      const size_t e = q + kQTile < hi ? q + kQTile : hi;
      if (chunks > 1) {
        uint32_t* m = merges + 4 * c.merges++;
        m[0] = (uint32_t)q;
        m[1] = (uint32_t)e;
        m[2] = c.slots;
        m[3] = (uint32_t)chunks;
      }
      for (size_t k = 0; k < chunks; ++k) {
        uint32_t* it = items + 8 * c.items++;
        it[0] = (uint32_t)q;
        it[1] = (uint32_t)e;
        it[2] = (uint32_t)lo;
        it[3] = (uint32_t)hi;
        it[4] = (uint32_t)(chunks > 1 ? lo + k * ck : lo);
        it[5] = (uint32_t)(chunks > 1 ? std::min(hi, lo + (k + 1) * ck) : hi);
        it[6] = chunks > 1 ? c.slots++ : kNoSlot;
        it[7] = (uint32_t)col;
      }
    }
    col += (hi - lo + 31) / 32 * 32;
  }
  return c;
}

AttentionCounts attention_capacity(size_t tokens, size_t batch) {
  // Items: ceil(n/32) c(n) <= n per sequence (c(n) <= 4 chunks, and n > 256
  // when c(n) > 1), so at most `tokens`; `batch` more keeps room for
  // rounding. Merges: one per query tile of a split sequence; tiles round
  // up per sequence, so at most ceil(tokens/32) + (the number of sequences
  // longer than kSplitLen that fit); slots: at most kMaxChunks per merge.
  const size_t split_seqs = tokens / (kSplitLen + 1);
  const size_t tiles = (tokens + kQTile - 1) / kQTile + split_seqs;
  AttentionCounts c;
  c.items = (unsigned)(tokens + batch);
  c.merges = (unsigned)(split_seqs ? tiles : 0);
  c.slots = (unsigned)(split_seqs ? tiles * key_chunks(tokens) : 0);
  return c;
}

size_t build_vt_columns(const size_t* offsets, size_t batch, int32_t* vcol) {
  size_t base = 0;
  for (size_t s = 0; s < batch; ++s) {
    for (size_t t = offsets[s]; t < offsets[s + 1]; ++t) vcol[t] = (int32_t)(base + (t - offsets[s]));
    base += (offsets[s + 1] - offsets[s] + 31) / 32 * 32;
  }
  return base;
}

hipError_t launch_attention(const _Float16* qs, const _Float16* ks, const _Float16* vt, int ldv, const uint32_t* items,
                            const uint32_t* item_count, int grid, int window, int rows, int8_t* cq, float* cd, float* partials, hipStream_t st) {
  if (rows <= 0 || grid <= 0 || ldv <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_kernel, dim3(grid), dim3(64 * kWaves), 0, st, qs, ks, vt, ldv,
                     reinterpret_cast<const uint4*>(items), item_count, window, rows, cq, cd, partials);
  return hipGetLastError();
}

hipError_t launch_attention_merge(const uint32_t* merges, const uint32_t* merge_count, int grid, const float* partials,
                                  int rows, int8_t* cq, float* cd, hipStream_t st) {
  if (rows <= 0 || grid <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_merge_kernel, dim3(grid), dim3(192), 0, st, reinterpret_cast<const uint4*>(merges),
                     merge_count, partials, rows, cq, cd);
  return hipGetLastError();
}

}  // namespace eg2
