// Operator-level C ABI (include/eg2_hip.h): argument checks and launches of
// the gfx950 kernels, plus the host helpers shared with the executor.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>

#include "eg2_hip.h"
#include "eg2_kernels.hpp"

namespace {
hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
_Float16* h16(uint16_t* p) { return reinterpret_cast<_Float16*>(p); }
const _Float16* h16(const uint16_t* p) { return reinterpret_cast<const _Float16*>(p); }

// IEEE fp16 bit pattern of an int8 value (exact: |q| <= 128 < 2^11).
uint16_t int8_to_fp16_bits(int8_t q) {
  if (q == 0) return 0;
  const uint32_t sign = q < 0 ? 0x8000u : 0u;
  uint32_t mag = (uint32_t)(q < 0 ? -(int)q : (int)q);
  int e = 0;
  while ((mag >> e) > 1) ++e;  // mag in [2^e, 2^(e+1))
  const uint32_t mant = (mag << (10 - e)) & 0x3FFu;
  return (uint16_t)(sign | ((uint32_t)(e + 15) << 10) | mant);
}
int code(hipError_t e) { return (int)e; }
constexpr int kInvalid = (int)hipErrorInvalidValue;

float fp16_to_fp32_host(uint16_t h) {
  // common.h:17-40
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  uint32_t bits;
  if (e == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      int sh = 0;
      uint32_t m = man;
      while (!(m & 0x400u)) {
        m <<= 1;
        ++sh;
      }
      bits = sign | ((uint32_t)(127 - 14 - sh) << 23) | ((m & 0x3FFu) << 13);
    }
  } else if (e == 0x1F) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((e - 15 + 127) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}
}  // namespace

extern "C" {

int eg2_hip_embed_norm_quant(const void* table_q8, const int32_t* ids, unsigned rows, float embed_scale,
                             const float* norm_w, float eps, float* x, uint16_t* xq, float* xd, void* stream) {
  if (!table_q8 || !ids || !norm_w || !x || !xq || !xd || rows == 0) return kInvalid;
  return code(eg2::launch_embed_norm_quant(static_cast<const uint8_t*>(table_q8), ids, (int)rows, embed_scale,
                                           norm_w, eps, x, h16(xq), xd, as_stream(stream)));
}

int eg2_hip_residual_norm_quant(float* x, const float* h, const float* post_w, const float* next_w, float eps,
                                uint16_t* xq, float* xd, unsigned rows, void* stream) {
  if (!x || !h || !post_w || rows == 0 || (next_w && (!xq || !xd))) return kInvalid;
  return code(
      eg2::launch_residual_norm_quant(x, h, post_w, next_w, eps, h16(xq), xd, (int)rows, as_stream(stream)));
}

int eg2_hip_qk_norm_rope(const float* qkv, const float* q_w, const float* k_w, const float* rope_table,
                         const int32_t* pos, const int32_t* vcol, float eps, uint16_t* qs, uint16_t* ks, uint16_t* vt,
                         unsigned ldv, unsigned rows, void* stream) {
  if (!qkv || !q_w || !k_w || !rope_table || !pos || !vcol || !qs || !ks || !vt || rows == 0 || ldv == 0 ||
      ldv % 32 != 0 || ldv > (1u << 20))
    return kInvalid;
  return code(eg2::launch_qk_norm_rope(qkv, q_w, k_w, rope_table, pos, vcol, eps, h16(qs), h16(ks), h16(vt),
                                       (int)ldv, (int)rows, as_stream(stream)));
}

int eg2_hip_attention(const uint16_t* qs, const uint16_t* ks, const uint16_t* vt, unsigned ldv, const int32_t* vcol,
                      const uint32_t* tiles, const uint32_t* tile_count, unsigned grid, unsigned window,
                      unsigned rows, uint16_t* cq, float* cd, void* stream) {
  if (!qs || !ks || !vt || !vcol || !tiles || !tile_count || !cq || !cd || rows == 0 || grid == 0 ||
      grid > 65536 || window > 4096u || ldv == 0 || ldv % 32 != 0 || ldv > (1u << 20))
    return kInvalid;
  return code(eg2::launch_attention(h16(qs), h16(ks), h16(vt), (int)ldv, vcol, tiles, tile_count, (int)grid,
                                    (int)window, (int)rows, h16(cq), cd, as_stream(stream)));
}

unsigned eg2_attention_tiles(const size_t* offsets, size_t batch, uint32_t* tiles) {
  if (!offsets || !tiles) return 0;
  return eg2::build_attention_tiles(offsets, batch, tiles);
}

size_t eg2_attention_vt_columns(const size_t* offsets, size_t batch, int32_t* vcol) {
  if (!offsets || !vcol) return 0;
  return eg2::build_vt_columns(offsets, batch, vcol);
}

int eg2_hip_gelu_quant(const float* gate_up, uint16_t* gq, float* gd, unsigned rows, void* stream) {
  if (!gate_up || !gq || !gd || rows == 0) return kInvalid;
  return code(eg2::launch_gelu_quant(gate_up, h16(gq), gd, (int)rows, as_stream(stream)));
}

int eg2_hip_quantize_rows(const float* x, unsigned k, uint16_t* q, float* d, unsigned rows, void* stream) {
  if (!x || !q || !d || rows == 0 || k == 0 || k % 64 != 0) return kInvalid;
  return code(eg2::launch_quantize_rows(x, (int)k, h16(q), d, (int)rows, as_stream(stream)));
}

int eg2_hip_rms_norm_rows(float* x, const float* w, float eps, unsigned rows, void* stream) {
  if (!x || !w || rows == 0) return kInvalid;
  return code(eg2::launch_rms_norm_rows(x, w, eps, (int)rows, as_stream(stream)));
}

int eg2_hip_pool_l2(const float* x, const uint32_t* offsets, float* out, unsigned batch, void* stream) {
  if (!x || !offsets || !out || batch == 0) return kInvalid;
  return code(eg2::launch_pool_l2(x, offsets, out, (int)batch, as_stream(stream)));
}

int eg2_hip_l2_prefix(float* x, unsigned width, unsigned dims, unsigned rows, void* stream) {
  if (!x || rows == 0 || dims == 0 || dims > width || dims % 8 != 0 || dims > 8192) return kInvalid;
  return code(eg2::launch_l2_prefix(x, (int)width, (int)dims, (int)rows, as_stream(stream)));
}

int eg2_hip_gemm_q8(const uint16_t* xq, const float* xd, unsigned ldx, const uint16_t* wf, const float* wdf,
                    float* y, unsigned n, unsigned m, unsigned k, unsigned ldy, void* stream) {
  if (!xq || !xd || !wf || !wdf || !y || n == 0 || m == 0 || k == 0 || k % 32 != 0 || ldy < m || ldx < n ||
      k > eg2::gemm_q8_max_k())
    return kInvalid;
  return code(eg2::launch_gemm_q8(h16(xq), xd, (int)ldx, h16(wf), wdf, y, (int)n, (int)m, (int)k, (int)ldy,
                                  as_stream(stream)));
}

const char* eg2_hip_error_string(int c) { return hipGetErrorString((hipError_t)c); }

int eg2_hip_device_check(char* err, size_t len) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
    if (err && len) std::snprintf(err, len, "no HIP device");
    return -1;
  }
  int dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
    if (err && len) std::snprintf(err, len, "cannot query the HIP device");
    return -1;
  }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    if (err && len) std::snprintf(err, len, "device %s is not gfx950", prop.gcnArchName);
    return -1;
  }
  return 0;
}

void eg2_q8_split(const void* blocks, size_t rows, unsigned k, uint16_t* q, float* d) {
  const uint8_t* src = static_cast<const uint8_t*>(blocks);
  const size_t nb = k / 32;
  for (size_t r = 0; r < rows; ++r)
    for (size_t b = 0; b < nb; ++b) {
      const uint8_t* blk = src + (r * nb + b) * 34;
      d[r * nb + b] = fp16_to_fp32_host((uint16_t)(blk[0] | (blk[1] << 8)));
      for (int i = 0; i < 32; ++i) q[r * k + b * 32 + i] = int8_to_fp16_bits((int8_t)blk[2 + i]);
    }
}

void eg2_q8_fragments(const void* blocks, size_t rows, unsigned k, uint16_t* wf, float* wdf) {
  const uint8_t* src = static_cast<const uint8_t*>(blocks);
  const size_t nb = k / 32, tiles = (rows + 31) / 32;
  for (size_t mt = 0; mt < tiles; ++mt)
    for (size_t b = 0; b < nb; ++b)
      for (unsigned lane = 0; lane < 64; ++lane) {
        const size_t r = mt * 32 + lane % 32, f = (mt * nb + b) * 64 + lane;
        const uint8_t* blk = r < rows ? src + (r * nb + b) * 34 : nullptr;
        wdf[f] = blk ? fp16_to_fp32_host((uint16_t)(blk[0] | (blk[1] << 8))) : 0.0f;
        for (unsigned i = 0; i < 16; ++i)
          wf[f * 16 + i] = blk ? int8_to_fp16_bits((int8_t)blk[2 + 16 * (lane / 32) + i]) : 0;
      }
}

size_t eg2_q8_fragment_halves(size_t rows, unsigned k) { return (rows + 31) / 32 * (k / 32) * 64 * 16; }

void eg2_rope_table(float base, unsigned n_pos, float* table) {
  for (unsigned p = 0; p < n_pos; ++p)
    for (int dim = 0; dim < 128; ++dim) {
      const float theta = (float)(int)p * powf(base, -2.0f * (float)dim / 256.0f);
      table[(size_t)p * 256 + dim] = cosf(theta);
      table[(size_t)p * 256 + 128 + dim] = sinf(theta);
    }
}

}  // extern "C"
