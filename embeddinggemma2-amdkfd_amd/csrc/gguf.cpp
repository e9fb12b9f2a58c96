// GGUF v3 reader into the engine's ei_gguf layout, and a writer of synthetic
// `gemma-embedding` models with Q8_0 matrices (include/eg2_hip.h).
//
// Reader semantics follow gguf.c:119-196: little-endian header, KV scalars
// normalised into the union (unsigned -> u64, signed -> i64, floats -> f64,
// bool -> b), STRING arrays indexed as ei_str, general.alignment (default
// 32, power of two), data section at the aligned end of the header, tensor
// offsets aligned and inside the file.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "eg2_hip.h"

namespace {

struct Cursor {
  const uint8_t* p;
  const uint8_t* end;
  const uint8_t* take(uint64_t n) {
    if ((uint64_t)(end - p) < n) throw std::runtime_error("truncated file");
    const uint8_t* r = p;
    p += n;
    return r;
  }
  uint32_t u32() {
    uint32_t v;
    std::memcpy(&v, take(4), 4);
    return v;
  }
  uint64_t u64() {
    uint64_t v;
    std::memcpy(&v, take(8), 8);
    return v;
  }
  ei_str str() {
    ei_str s;
    s.len = u64();
    s.str = reinterpret_cast<const char*>(take(s.len));
    return s;
  }
};

uint64_t scalar_size(uint32_t type) {
  switch (type) {
    case EI_GGUF_U8: case EI_GGUF_I8: case EI_GGUF_BOOL: return 1;
    case EI_GGUF_U16: case EI_GGUF_I16: return 2;
    case EI_GGUF_U32: case EI_GGUF_I32: case EI_GGUF_F32: return 4;
    case EI_GGUF_U64: case EI_GGUF_I64: case EI_GGUF_F64: return 8;
    default: throw std::runtime_error("unsupported kv scalar type " + std::to_string(type));
  }
}

void read_scalar(ei_kv* kv, uint32_t type, const uint8_t* p) {
  switch (type) {
    case EI_GGUF_U8: kv->v.u64 = *p; break;
    case EI_GGUF_I8: kv->v.i64 = *reinterpret_cast<const int8_t*>(p); break;
    case EI_GGUF_U16: { uint16_t v; std::memcpy(&v, p, 2); kv->v.u64 = v; } break;
    case EI_GGUF_I16: { int16_t v; std::memcpy(&v, p, 2); kv->v.i64 = v; } break;
    case EI_GGUF_U32: { uint32_t v; std::memcpy(&v, p, 4); kv->v.u64 = v; } break;
    case EI_GGUF_I32: { int32_t v; std::memcpy(&v, p, 4); kv->v.i64 = v; } break;
    case EI_GGUF_F32: { float v; std::memcpy(&v, p, 4); kv->v.f64 = v; } break;
    case EI_GGUF_U64: { uint64_t v; std::memcpy(&v, p, 8); kv->v.u64 = v; } break;
    case EI_GGUF_I64: { int64_t v; std::memcpy(&v, p, 8); kv->v.i64 = v; } break;
    case EI_GGUF_F64: { double v; std::memcpy(&v, p, 8); kv->v.f64 = v; } break;
    case EI_GGUF_BOOL: kv->v.b = *p != 0; break;
    default: break;
  }
}

uint64_t tensor_bytes(const ei_tensor* t) {
  uint64_t n = 1;
  for (uint32_t i = 0; i < t->n_dims; ++i) n *= t->ne[i];
  switch (t->type) {
    case EI_T_F32: return n * 4;
    case EI_T_F16: case EI_T_BF16: return n * 2;
    case EI_T_Q4_0:
    case EI_T_Q8_0:
      if (t->ne[0] % 32 != 0) throw std::runtime_error("quantized row length not a multiple of 32");
      return n / 32 * (t->type == EI_T_Q8_0 ? 34 : 18);
    default: throw std::runtime_error("unsupported ggml type " + std::to_string(t->type));
  }
}

void parse(ei_gguf* g) {
  Cursor c{g->map, g->map + g->map_len};
  if (c.u32() != 0x46554747u) throw std::runtime_error("not a GGUF file");
  g->version = c.u32();
  if (g->version != 3) throw std::runtime_error("GGUF version " + std::to_string(g->version) + " (only v3)");
  g->n_tensors = c.u64();
  g->n_kv = c.u64();
  if (g->n_tensors > (1u << 24) || g->n_kv > (1u << 24)) throw std::runtime_error("implausible GGUF counts");
  g->kv = static_cast<ei_kv*>(std::calloc(g->n_kv ? g->n_kv : 1, sizeof(ei_kv)));
  g->tensors = static_cast<ei_tensor*>(std::calloc(g->n_tensors ? g->n_tensors : 1, sizeof(ei_tensor)));
  if (!g->kv || !g->tensors) throw std::runtime_error("out of memory");
  g->alignment = 32;
  for (uint64_t i = 0; i < g->n_kv; ++i) {
    ei_kv* kv = &g->kv[i];
    kv->key = c.str();
    kv->type = c.u32();
    if (kv->type == EI_GGUF_ARRAY) {
      kv->arr_type = c.u32();
      kv->arr_n = c.u64();
      if (kv->arr_type == EI_GGUF_STRING) {
        if (kv->arr_n > (uint64_t)(c.end - c.p) / 8) throw std::runtime_error("truncated string array");
        ei_str* idx = static_cast<ei_str*>(std::malloc(sizeof(ei_str) * (kv->arr_n ? kv->arr_n : 1)));
        if (!idx) throw std::runtime_error("out of memory");
        kv->arr_data = idx;
        for (uint64_t k = 0; k < kv->arr_n; ++k) idx[k] = c.str();
      } else if (kv->arr_type == EI_GGUF_ARRAY) {
        throw std::runtime_error("nested arrays are not supported");
      } else {
        const uint64_t sz = scalar_size(kv->arr_type);
        if (kv->arr_n > (uint64_t)(c.end - c.p) / sz) throw std::runtime_error("truncated array");
        kv->arr_data = c.take(sz * kv->arr_n);
      }
    } else if (kv->type == EI_GGUF_STRING) {
      kv->v.s = c.str();
    } else {
      read_scalar(kv, kv->type, c.take(scalar_size(kv->type)));
    }
  }
  for (uint64_t i = 0; i < g->n_kv; ++i) {
    const ei_kv& kv = g->kv[i];
    if (kv.key.len == 17 && std::memcmp(kv.key.str, "general.alignment", 17) == 0) g->alignment = kv.v.u64;
  }
  if (g->alignment == 0 || (g->alignment & (g->alignment - 1)) != 0) throw std::runtime_error("bad alignment");
  for (uint64_t i = 0; i < g->n_tensors; ++i) {
    ei_tensor* t = &g->tensors[i];
    t->name = c.str();
    t->n_dims = c.u32();
    if (t->n_dims == 0 || t->n_dims > 4) throw std::runtime_error("tensor with bad rank");
    for (int d = 0; d < 4; ++d) t->ne[d] = 1;
    for (uint32_t d = 0; d < t->n_dims; ++d) t->ne[d] = c.u64();
    t->type = c.u32();
    t->offset = c.u64();
  }
  const uint64_t off = (uint64_t)(c.p - g->map);
  g->data_off = (off + g->alignment - 1) & ~(g->alignment - 1);
  for (uint64_t i = 0; i < g->n_tensors; ++i) {
    ei_tensor* t = &g->tensors[i];
    t->n_bytes = tensor_bytes(t);
    if (t->offset % g->alignment != 0) throw std::runtime_error("misaligned tensor offset");
    const uint64_t abs = g->data_off + t->offset;
    if (abs > g->map_len || t->n_bytes > g->map_len - abs) throw std::runtime_error("tensor extends past end of file");
    t->data = g->map + abs;
  }
}

// ------------------------------------------------------------------ writer

// Counter-based normal generator: splitmix64 stream seeded per (tensor, row)
// and the Box-Muller transform in double precision.
struct Normal {
  uint64_t state;
  bool has_spare = false;
  double spare = 0;
  explicit Normal(uint64_t seed) : state(seed) {}
  uint64_t next() {
    uint64_t z = (state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  double uniform() { return ((next() >> 11) + 1) * (1.0 / 9007199254740993.0); }  // (0, 1]
  double operator()() {
    if (has_spare) {
      has_spare = false;
      return spare;
    }
    const double r = std::sqrt(-2.0 * std::log(uniform()));
    const double a = 6.283185307179586 * uniform();
    spare = r * std::sin(a);
    has_spare = true;
    return r * std::cos(a);
  }
};

uint64_t row_seed(uint64_t seed, uint64_t tensor, uint64_t row) {
  Normal mix(seed ^ (tensor * 0xD1B54A32D192ED03ull) ^ (row * 0x8CB92BA72F3D8DD7ull));
  return mix.next();
}

uint16_t fp32_to_fp16_host(float f) {
  // Same rounding as the reference quantizer's scale store (quants.c:13-37).
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t mant = x & 0x007FFFFFu;
  const int32_t e = (int32_t)((x >> 23) & 0xFFu) - 127 + 15;
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    mant |= 0x00800000u;
    const uint32_t shift = (uint32_t)(14 - e);
    uint32_t h = sign | (mant >> shift);
    if ((mant >> (shift - 1u)) & 1u) h++;
    return (uint16_t)h;
  }
  if (e >= 31) return (uint16_t)(sign | 0x7C00u | (mant ? ((mant >> 13) | 1u) : 0u));
  uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13);
  if (mant & 0x00001000u) h++;
  return (uint16_t)h;
}

// One Q8_0 row from n floats (quants.c:97-177 scalar rules).
void quantize_row(const float* x, int n, uint8_t* out) {
  for (int b = 0; b < n / 32; ++b) {
    const float* xb = x + b * 32;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = std::fabs(xb[j]) > amax ? std::fabs(xb[j]) : amax;
    const float d = amax / 127.0f;
    const uint16_t h = fp32_to_fp16_host(d);
    uint8_t* blk = out + b * 34;
    blk[0] = (uint8_t)(h & 0xFF);
    blk[1] = (uint8_t)(h >> 8);
    if (amax == 0.0f) {
      std::memset(blk + 2, 0, 32);
      continue;
    }
    const float id = 1.0f / d;
    for (int j = 0; j < 32; ++j) {
      int q = (int)std::round(xb[j] * id);
      q = q < -128 ? -128 : (q > 127 ? 127 : q);
      blk[2 + j] = (uint8_t)(int8_t)q;
    }
  }
}

struct TensorSpec {
  std::string name;
  std::vector<uint64_t> ne;  // ne[0] = row length
  uint32_t type;             // EI_T_Q8_0 or EI_T_F32
  float std_dev;             // Q8_0: N(0, std); F32: 1 + std*N(0,1)
  uint64_t offset = 0, bytes = 0;
};

class Writer {
 public:
  explicit Writer(FILE* f) : f_(f) {}
  void bytes(const void* p, size_t n) {
    if (n && std::fwrite(p, 1, n, f_) != n) throw std::runtime_error("write failed");
  }
  void u32(uint32_t v) { bytes(&v, 4); }
  void u64(uint64_t v) { bytes(&v, 8); }
  void f32(float v) { bytes(&v, 4); }
  void str(const std::string& s) {
    u64(s.size());
    bytes(s.data(), s.size());
  }
  void kv_u32(const std::string& k, uint32_t v) { str(k), u32(EI_GGUF_U32), u32(v); }
  void kv_f32(const std::string& k, float v) { str(k), u32(EI_GGUF_F32), f32(v); }
  void kv_str(const std::string& k, const std::string& v) { str(k), u32(EI_GGUF_STRING), str(v); }
  void pad(uint64_t pos, uint64_t align) {
    static const uint8_t zeros[64] = {0};
    const uint64_t p = (align - pos % align) % align;
    bytes(zeros, p);
  }

 private:
  FILE* f_;
};

void fill_tensor(const TensorSpec& t, uint64_t seed, uint64_t tensor_index, unsigned threads, std::vector<uint8_t>& out) {
  const uint64_t k = t.ne[0];
  const uint64_t rows = t.ne.size() > 1 ? t.ne[1] : 1;
  out.assign(t.bytes, 0);
  const uint64_t row_bytes = t.type == EI_T_Q8_0 ? k / 32 * 34 : k * 4;
  auto work = [&](uint64_t r0, uint64_t r1) {
    std::vector<float> buf(k);
    for (uint64_t r = r0; r < r1; ++r) {
      Normal rng(row_seed(seed, tensor_index, r));
      if (t.type == EI_T_Q8_0) {
        for (uint64_t i = 0; i < k; ++i) buf[i] = (float)(rng() * t.std_dev);
        quantize_row(buf.data(), (int)k, out.data() + r * row_bytes);
      } else {
        for (uint64_t i = 0; i < k; ++i) buf[i] = (float)(1.0 + rng() * t.std_dev);
        std::memcpy(out.data() + r * row_bytes, buf.data(), k * 4);
      }
    }
  };
  unsigned nt = threads ? threads : 1;
  if (rows < 1024) nt = 1;
  std::vector<std::thread> pool;
  for (unsigned i = 0; i < nt; ++i) pool.emplace_back(work, rows * i / nt, rows * (i + 1) / nt);
  for (auto& th : pool) th.join();
}

}  // namespace

extern "C" int eg2_gguf_open(const char* path, ei_gguf* g, char* err, size_t len) {
  if (!g) return -1;
  std::memset(g, 0, sizeof *g);
  try {
    if (!path) throw std::runtime_error("no path");
    const int fd = open(path, O_RDONLY);
    if (fd < 0) throw std::runtime_error("cannot open");
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
      close(fd);
      throw std::runtime_error("cannot stat");
    }
    g->map_len = (size_t)st.st_size;
    void* m = mmap(nullptr, g->map_len, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) throw std::runtime_error("mmap failed");
    g->map = static_cast<const uint8_t*>(m);
    parse(g);
    return 0;
  } catch (const std::exception& e) {
    if (err && len) std::snprintf(err, len, "%s: %s", path ? path : "(null)", e.what());
    eg2_gguf_close(g);
    return -1;
  }
}

extern "C" void eg2_gguf_close(ei_gguf* g) {
  if (!g) return;
  if (g->kv)
    for (uint64_t i = 0; i < g->n_kv; ++i)
      if (g->kv[i].type == EI_GGUF_ARRAY && g->kv[i].arr_type == EI_GGUF_STRING)
        std::free(const_cast<void*>(g->kv[i].arr_data));
  std::free(g->kv);
  std::free(g->tensors);
  if (g->map) munmap(const_cast<uint8_t*>(g->map), g->map_len);
  std::memset(g, 0, sizeof *g);
}

extern "C" int eg2_synth_write_gguf(const char* path, const eg2_synth_config* cfg, char* err, size_t len) {
  FILE* f = nullptr;
  try {
    if (!path || !cfg) throw std::runtime_error("missing path or config");
    if (cfg->n_layer < 1 || cfg->n_layer > 64) throw std::runtime_error("n_layer must be 1..64");
    std::vector<TensorSpec> ts;
    const float ws = cfg->weight_std, ns = cfg->norm_std;
    ts.push_back({"token_embd.weight", {768, 262144}, EI_T_Q8_0, cfg->embed_std});
    ts.push_back({"output_norm.weight", {768}, EI_T_F32, ns});
    for (unsigned l = 0; l < cfg->n_layer; ++l) {
      const std::string p = "blk." + std::to_string(l) + ".";
      ts.push_back({p + "attn_q.weight", {768, 768}, EI_T_Q8_0, ws});
      ts.push_back({p + "attn_k.weight", {768, 256}, EI_T_Q8_0, ws});
      ts.push_back({p + "attn_v.weight", {768, 256}, EI_T_Q8_0, ws});
      ts.push_back({p + "attn_output.weight", {768, 768}, EI_T_Q8_0, ws});
      ts.push_back({p + "ffn_up.weight", {768, 1152}, EI_T_Q8_0, ws});
      ts.push_back({p + "ffn_gate.weight", {768, 1152}, EI_T_Q8_0, ws});
      ts.push_back({p + "ffn_down.weight", {1152, 768}, EI_T_Q8_0, ws});
      ts.push_back({p + "attn_norm.weight", {768}, EI_T_F32, ns});
      ts.push_back({p + "attn_q_norm.weight", {256}, EI_T_F32, ns});
      ts.push_back({p + "attn_k_norm.weight", {256}, EI_T_F32, ns});
      ts.push_back({p + "post_attention_norm.weight", {768}, EI_T_F32, ns});
      ts.push_back({p + "ffn_norm.weight", {768}, EI_T_F32, ns});
      ts.push_back({p + "post_ffw_norm.weight", {768}, EI_T_F32, ns});
    }
    if (cfg->dense_head) {
      ts.push_back({"dense_2.weight", {768, 3072}, EI_T_Q8_0, ws});
      ts.push_back({"dense_3.weight", {3072, 768}, EI_T_Q8_0, ws});
    }
    constexpr uint64_t align = 32;
    uint64_t off = 0;
    for (auto& t : ts) {
      uint64_t n = 1;
      for (auto e : t.ne) n *= e;
      t.bytes = t.type == EI_T_Q8_0 ? n / 32 * 34 : n * 4;
      t.offset = off;
      off = (off + t.bytes + align - 1) / align * align;
    }
    f = std::fopen(path, "wb");
    if (!f) throw std::runtime_error("cannot create file");
    Writer w(f);
    w.u32(0x46554747u);
    w.u32(3);
    w.u64(ts.size());
    const uint64_t n_kv = 16;
    w.u64(n_kv);
    w.kv_str("general.architecture", "gemma-embedding");
    w.kv_u32("general.alignment", (uint32_t)align);
    w.kv_u32("gemma-embedding.block_count", cfg->n_layer);
    w.kv_u32("gemma-embedding.embedding_length", 768);
    w.kv_u32("gemma-embedding.feed_forward_length", 1152);
    w.kv_u32("gemma-embedding.attention.head_count", 3);
    w.kv_u32("gemma-embedding.attention.head_count_kv", 1);
    w.kv_u32("gemma-embedding.attention.key_length", 256);
    w.kv_u32("gemma-embedding.attention.value_length", 256);
    w.kv_u32("gemma-embedding.context_length", 2048);
    w.kv_f32("gemma-embedding.attention.layer_norm_rms_epsilon", 1e-6f);
    w.kv_f32("gemma-embedding.rope.freq_base", cfg->rope_base_full);
    w.kv_f32("gemma-embedding.rope.freq_base_swa", cfg->rope_base_swa);
    w.kv_u32("gemma-embedding.attention.sliding_window", cfg->sliding_window);
    w.kv_u32("gemma-embedding.attention.sliding_window_pattern", cfg->sliding_window_pattern);
    w.kv_str("tokenizer.ggml.model", "llama");
    for (auto& t : ts) {
      w.str(t.name);
      w.u32((uint32_t)t.ne.size());
      for (auto e : t.ne) w.u64(e);
      w.u32(t.type);
      w.u64(t.offset);
    }
    const long header = std::ftell(f);
    if (header < 0) throw std::runtime_error("ftell failed");
    w.pad((uint64_t)header, align);
    std::vector<uint8_t> data;
    uint64_t pos = 0;
    for (size_t i = 0; i < ts.size(); ++i) {
      fill_tensor(ts[i], cfg->seed, i, cfg->threads, data);
      w.bytes(data.data(), data.size());
      pos += data.size();
      w.pad(pos, align);
      pos = (pos + align - 1) / align * align;
    }
    if (std::fclose(f) != 0) {
      f = nullptr;
      throw std::runtime_error("close failed");
    }
    return 0;
  } catch (const std::exception& e) {
    if (f) std::fclose(f);
    if (err && len) std::snprintf(err, len, "%s", e.what());
    return -1;
  }
}
