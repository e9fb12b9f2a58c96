// Operator-level C ABI (include/eg2_hip.h): argument checks and launches of
// the gfx950 kernels, plus the host helpers shared with the executor.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>

#include "eg2_hip.h"
#include "eg2_device.hpp"
#include "eg2_kernels.hpp"

namespace {
hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

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
                             const float* norm_w, float eps, float* x, int8_t* xq, float* xd, void* stream) {
  if (!table_q8 || !ids || !norm_w || !x || !xq || !xd || rows == 0) return kInvalid;
  return code(eg2::launch_embed_norm_quant(static_cast<const uint8_t*>(table_q8), ids, (int)rows, embed_scale,
                                           norm_w, eps, x, xq, xd, as_stream(stream)));
}

int eg2_hip_residual_norm_quant(float* x, const float* h, const float* post_w, const float* next_w, float eps,
                                int8_t* xq, float* xd, unsigned rows, void* stream) {
  if (!x || !h || !post_w || rows == 0 || (next_w && (!xq || !xd))) return kInvalid;
  return code(eg2::launch_residual_norm_quant(x, h, post_w, next_w, eps, xq, xd, (int)rows, as_stream(stream)));
}

int eg2_hip_qk_norm_rope(const float* qkv, const float* q_w, const float* k_w, const float* rope_table,
                         const int32_t* pos, float eps, float* out, unsigned rows, void* stream) {
  if (!qkv || !q_w || !k_w || !rope_table || !pos || !out || rows == 0) return kInvalid;
  return code(eg2::launch_qk_norm_rope(qkv, q_w, k_w, rope_table, pos, eps, out, (int)rows, as_stream(stream)));
}

int eg2_hip_attention(const float* qkv, const uint32_t* items, const uint32_t* item_count, unsigned grid,
                      const uint32_t* tok, unsigned window, unsigned rows, unsigned longest, float* scores, int8_t* cq,
                      float* cd, void* stream) {
  if (!qkv || !items || !item_count || !tok || !scores || !cq || !cd || rows == 0 || rows % 4 != 0 ||
      rows > (1u << 24) || grid == 0 || grid > 65536 || window > 4096u || longest > rows)
    return kInvalid;
  return code(eg2::launch_attention(qkv, items, item_count, (int)grid, tok, (int)window, (int)rows, (int)longest,
                                    scores, cq, cd, as_stream(stream)));
}

int eg2_hip_attention_scores(const float* qkv, const uint32_t* items, const uint32_t* item_count, unsigned grid,
                             unsigned window, unsigned rows, float* scores, void* stream) {
  if (!qkv || !items || !item_count || !scores || rows == 0 || rows % 4 != 0 || rows > (1u << 24) || grid == 0 ||
      grid > 65536 || window > 4096u)
    return kInvalid;
  return code(eg2::launch_attention_scores(qkv, items, item_count, (int)grid, (int)window, (int)rows, scores,
                                           as_stream(stream)));
}

int eg2_hip_attention_softmax(const uint32_t* tok, unsigned window, unsigned rows, unsigned longest, float* scores,
                              void* stream) {
  if (!tok || !scores || rows == 0 || rows % 4 != 0 || rows > (1u << 24) || window > 4096u || longest > rows)
    return kInvalid;
  return code(eg2::launch_attention_softmax(tok, (int)window, (int)rows, (int)longest, scores, as_stream(stream)));
}

int eg2_hip_attention_context(const float* qkv, const uint32_t* items, const uint32_t* item_count, unsigned grid,
                              unsigned window, unsigned rows, const float* scores, int8_t* cq, float* cd,
                              void* stream) {
  if (!qkv || !items || !item_count || !scores || !cq || !cd || rows == 0 || rows % 4 != 0 || rows > (1u << 24) ||
      grid == 0 || grid > 65536 || window > 4096u)
    return kInvalid;
  return code(eg2::launch_attention_context(qkv, items, item_count, (int)grid, (int)window, (int)rows, scores, cq, cd,
                                            as_stream(stream)));
}

int eg2_hip_attention_static(const float* qkv, const uint32_t* offsets, unsigned batch, unsigned window,
                             unsigned rows, int8_t* cq, float* cd, void* stream) {
  if (!qkv || !offsets || !cq || !cd || rows == 0 || rows % 4 != 0 || rows > EG2_ATTENTION_STATIC_ROWS ||
      batch == 0 || batch > EG2_ATTENTION_STATIC_BATCH || window > 4096u)
    return kInvalid;
  return code(eg2::launch_attention_static(qkv, offsets, (int)batch, (int)window, (int)rows, cq, cd,
                                           as_stream(stream)));
}

int eg2_attention_plan(const size_t* offsets, size_t batch, size_t items_cap, size_t scores_cap, uint32_t* items,
                       uint32_t* tok, size_t* counts) {
  if (!offsets || !items || !tok || !counts) return -1;
  for (size_t s = 0; s < batch; ++s)
    if (offsets[s + 1] < offsets[s] || offsets[s + 1] > (1u << 24)) return -1;
  eg2::AttentionCounts used{0, 0, 0};
  const bool ok = eg2::build_attention_plan(offsets, batch, eg2::AttentionCounts{items_cap, scores_cap, 0}, items,
                                            tok, &used);
  counts[0] = used.items;
  counts[1] = used.score_floats;
  counts[2] = used.score_items;
  return ok ? 0 : -1;
}

void eg2_attention_capacity(size_t tokens, size_t batch, size_t* counts) {
  if (!counts) return;
  const eg2::AttentionCounts c = eg2::attention_capacity(tokens, batch);
  counts[0] = c.items;
  counts[1] = c.score_floats;
}

int eg2_hip_libm_eval(const float* x, unsigned n, float* expf_out, float* tanhf_out, void* stream) {
  if (!x || !expf_out || !tanhf_out || n == 0) return kInvalid;
  return code(eg2::launch_libm_eval(x, n, expf_out, tanhf_out, as_stream(stream)));
}

int eg2_hip_tanh_approx_error(uint32_t* out, void* stream) {
  if (!out) return kInvalid;
  return code(eg2::launch_tanh_approx_error(out, as_stream(stream)));
}

int eg2_hip_gelu_quant(const float* gate_up, int8_t* gq, float* gd, unsigned rows, void* stream) {
  if (!gate_up || !gq || !gd || rows == 0) return kInvalid;
  return code(eg2::launch_gelu_quant(gate_up, gq, gd, (int)rows, as_stream(stream)));
}

int eg2_hip_quantize_rows(const float* x, unsigned k, int8_t* q, float* d, unsigned rows, void* stream) {
  if (!x || !q || !d || rows == 0 || k == 0 || k % 64 != 0) return kInvalid;
  return code(eg2::launch_quantize_rows(x, (int)k, q, d, (int)rows, as_stream(stream)));
}

int eg2_hip_rms_norm_rows(float* x, const float* w, float eps, unsigned rows, void* stream) {
  if (!x || !w || rows == 0) return kInvalid;
  return code(eg2::launch_rms_norm_rows(x, w, eps, (int)rows, as_stream(stream)));
}

int eg2_hip_pool_l2(const float* x, const uint32_t* offsets, float* out, unsigned batch, void* stream) {
  if (!x || !offsets || !out || batch == 0) return kInvalid;
  return code(eg2::launch_pool_l2(x, offsets, out, (int)batch, as_stream(stream)));
}

int eg2_hip_pool_mean(const float* x, const uint32_t* offsets, float* out, unsigned batch, void* stream) {
  if (!x || !offsets || !out || batch == 0 || batch > 65535) return kInvalid;
  return code(eg2::launch_pool_mean(x, offsets, out, (int)batch, as_stream(stream)));
}

int eg2_hip_l2_prefix(float* x, unsigned width, unsigned dims, unsigned rows, void* stream) {
  if (!x || rows == 0 || dims == 0 || dims > width || dims % 8 != 0 || dims > 8192) return kInvalid;
  return code(eg2::launch_l2_prefix(x, (int)width, (int)dims, (int)rows, as_stream(stream)));
}

int eg2_hip_gemm_q8(const int8_t* xq, const float* xd, unsigned ldx, const int8_t* wq, const float* wd, unsigned ldw,
                    float* y, unsigned n, unsigned m, unsigned k, unsigned ldy, void* stream) {
  constexpr unsigned kMax = 1u << 24;  // keeps every index inside 32-bit arithmetic
  if (!xq || !xd || !wq || !wd || !y || n == 0 || m == 0 || k == 0 || k % 32 != 0 || ldy < m || ldx < n ||
      ldw < m || n > kMax || m > kMax || k > kMax || ldx > kMax || ldw > kMax || ldy > kMax)
    return kInvalid;
  return code(eg2::launch_gemm_q8(xq, xd, (int)ldx, wq, wd, (int)ldw, y, (int)n, (int)m, (int)k, (int)ldy,
                                  as_stream(stream)));
}

int eg2_hip_gemm_q8_qkv_rope(const int8_t* xq, const float* xd, unsigned ldx, const int8_t* wq, const float* wd,
                             unsigned ldw, unsigned n, unsigned k, const float* q_w, const float* k_w,
                             const float* rope_table, const int32_t* pos, float eps, float* out, void* stream) {
  constexpr unsigned kMax = 1u << 24;
  if (!xq || !xd || !wq || !wd || !q_w || !k_w || !rope_table || !pos || !out || n == 0 || k == 0 || k % 32 != 0 ||
      ldx < n || ldw < 1280 || n > kMax || k > kMax || ldx > kMax || ldw > kMax)
    return kInvalid;
  return code(eg2::launch_gemm_q8_qkv_rope(xq, xd, (int)ldx, wq, wd, (int)ldw, (int)n, (int)k, q_w, k_w, rope_table,
                                           pos, eps, out, as_stream(stream)));
}

int eg2_hip_gemm_q8_geglu(const int8_t* xq, const float* xd, unsigned ldx, const int8_t* wq, const float* wd,
                          unsigned ldw, int8_t* gq, float* gd, unsigned ldg, unsigned n, unsigned ff, unsigned k,
                          void* stream) {
  constexpr unsigned kMax = 1u << 24;
  if (!xq || !xd || !wq || !wd || !gq || !gd || n == 0 || ff == 0 || ff % 32 != 0 || k == 0 || k % 32 != 0 ||
      ldx < n || ldg < n || n > kMax || ff > kMax / 2 || ldw < 2 * ff || k > kMax || ldx > kMax || ldw > kMax ||
      ldg > kMax)
    return kInvalid;
  return code(eg2::launch_gemm_q8_geglu(xq, xd, (int)ldx, wq, wd, (int)ldw, gq, gd, (int)ldg, (int)n, (int)ff, (int)k,
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

size_t eg2_q8_tile_bytes(size_t rows, unsigned k) { return (rows + 31) / 32 * (k / 32) * 1024; }

void eg2_q8_pack_rows(const int8_t* q, size_t rows, unsigned k, int8_t* tiles) {
  const size_t padded = (rows + 31) / 32 * 32;
  for (size_t r = 0; r < padded; ++r)
    for (unsigned e = 0; e < k; ++e) tiles[eg2::q8_tile_offset(r, e, k / 32)] = r < rows ? q[r * k + e] : 0;
}

void eg2_q8_unpack_rows(const int8_t* tiles, size_t rows, unsigned k, int8_t* q) {
  for (size_t r = 0; r < rows; ++r)
    for (unsigned e = 0; e < k; ++e) q[r * k + e] = tiles[eg2::q8_tile_offset(r, e, k / 32)];
}

void eg2_q8_weight_tiles(const void* blocks, size_t rows, unsigned k, int8_t* wq, float* wd) {
  const uint8_t* src = static_cast<const uint8_t*>(blocks);
  const unsigned nb = k / 32;
  const size_t ld = (rows + 31) / 32 * 32;
  for (size_t r = 0; r < ld; ++r)
    for (unsigned b = 0; b < nb; ++b) {
      const uint8_t* blk = r < rows ? src + (r * nb + b) * 34 : nullptr;
      wd[(size_t)b * ld + r] = blk ? fp16_to_fp32_host((uint16_t)(blk[0] | (blk[1] << 8))) : 0.0f;
      for (unsigned i = 0; i < 32; ++i)
        wq[eg2::q8_tile_offset(r, 32 * b + i, nb)] = blk ? (int8_t)blk[2 + i] : 0;
    }
}

int eg2_q8_geglu_weight_tiles(const void* gate, const void* up, size_t ff, unsigned k, int8_t* wq, float* wd) {
  if (!gate || !up || !wq || !wd || ff == 0 || ff % 32 != 0 || k == 0 || k % 32 != 0) return -1;
  const size_t row_bytes = (size_t)(k / 32) * 34, group = 32 * row_bytes;
  std::vector<uint8_t> rows(2 * ff * row_bytes);
  for (size_t j = 0; j < ff / 32; ++j) {
    std::memcpy(rows.data() + (2 * j) * group, static_cast<const uint8_t*>(gate) + j * group, group);
    std::memcpy(rows.data() + (2 * j + 1) * group, static_cast<const uint8_t*>(up) + j * group, group);
  }
  eg2_q8_weight_tiles(rows.data(), 2 * ff, k, wq, wd);
  return 0;
}

void eg2_rope_table(float base, unsigned n_pos, float* table) {
  for (unsigned p = 0; p < n_pos; ++p)
    for (int dim = 0; dim < 128; ++dim) {
      const float theta = (float)(int)p * powf(base, -2.0f * (float)dim / 256.0f);
      table[(size_t)p * 256 + dim] = cosf(theta);
      table[(size_t)p * 256 + 128 + dim] = sinf(theta);
    }
}

}  // extern "C"
