// Packed-wave executor on one MI355X: the HIP replacement of the reference's
// /dev/kfd executor (src/gemma2_kfd.cpp), behind the same three C symbols.
//
// Create (src/gemma2_kfd.cpp:86-155): select the gfx950 device, read the
// `gemma-embedding` hyper-parameters and tensors from the caller's ei_gguf
// (model.c:61-105 names, Q8_0 matrices), repack every matrix once into the
// projection GEMM's operand layout (the int8 values as row tiles + the
// block scales transposed, see eg2_q8_weight_tiles), fuse Q|K|V into one
// projection and gate|up (interleaved in 32-row groups) into the operand of
// the fused gate|up + GeGLU GEMM, upload the raw Q8_0
// embedding table, build the RoPE tables on the host, and allocate a
// 2048-token workspace.
//
// Batch (src/gemma2_kfd.cpp:268-353): validate, build per-token metadata
// (sequence bounds, positions), pad the wave to a multiple of 32 rows with a
// dummy sequence, run the layer stack -- captured once per padded wave size
// as a hipGraph -- then pooling, the optional dense head and L2, and copy the
// [batch][768] embeddings back. Every call is serialised; a device failure
// poisons the context (src/gemma2_kfd.cpp:190-191, 214-215, 270).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "eg2_hip.h"
#include "eg2_kernels.hpp"
#include "gemma2_kfd.h"

namespace {

constexpr unsigned kCap = 2048;  // packed tokens per wave (src/gemma2_kfd.cpp:20)
// Transposed-v columns: every sequence (and the padding sequence) starts at
// a multiple of 32, so at most kCap + 31 * (kCap + 1) columns, rounded to 32.
constexpr unsigned kVtCols = (kCap + 31 * (kCap + 1) + 31) / 32 * 32;
constexpr int kEmbd = 768, kFF = 1152, kHeadDim = 256, kQKV = 768 + 2 * 256, kDenseFF = 3072;
constexpr int kVocab = 262144;
constexpr double kTimeoutSeconds = 30.0;  // src/gemma2_kfd.cpp:21

void check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

bool str_eq(const ei_str& s, const char* z) {
  const size_t n = std::strlen(z);
  return s.len == n && std::memcmp(s.str, z, n) == 0;
}

// Environment flag that must be "0" or "1" when set (src/gemma2_kfd.cpp:118-122).
bool env_flag(const char* name, bool dflt) {
  const char* v = std::getenv(name);
  if (!v) return dflt;
  if (std::strcmp(v, "0") && std::strcmp(v, "1")) throw std::runtime_error(std::string(name) + " must be 0 or 1");
  return v[0] == '1';
}

struct DevMat {
  int8_t* q = nullptr;  // row tiles
  float* d = nullptr;   // block scales [k/32][ld]
  int m = 0, k = 0, ld = 0;
};

struct Layer {
  DevMat qkv, o, gu, down;
  const float *attn_norm, *q_norm, *k_norm, *post_attn, *ffn_norm, *post_ffw;
  const float* rope;
  int window;
};

class Backend {
 public:
  explicit Backend(const ei_gguf* g);
  ~Backend();
  void batch(const int32_t* ids, const size_t* offsets, size_t batch, float* out);
  // The three phases of batch(), exposed for measurement: upload one wave's
  // ids and metadata, enqueue its forward (device-resident, no host copies),
  // and wait + copy the embeddings back.
  void stage(const int32_t* ids, const size_t* offsets, size_t batch);
  void launch_staged(unsigned repeats);
  void collect(float* out);
  std::mutex& mutex() { return mutex_; }

 private:
  const ei_gguf* model_;
  hipStream_t stream_ = nullptr;
  std::vector<void*> dev_allocs_;
  std::vector<void*> host_allocs_;
  std::mutex mutex_;
  bool poisoned_ = false;
  bool use_graph_ = true;
  bool profile_ = false;

  float eps_ = 1e-6f;
  std::vector<Layer> layers_;
  const uint8_t* token_embd_ = nullptr;
  const float* output_norm_ = nullptr;
  DevMat dense2_, dense3_;
  bool dense_ = false;

  // Workspace for kCap tokens.
  float *x_, *h_, *qkv_, *xd_, *cd_, *pooled_, *mid_, *mid_d_;
  int8_t *xq_, *cq_, *mid_q_;
  _Float16 *qs_, *ks_, *vt_;
  int32_t *ids_d_, *pos_d_, *vcol_d_;
  // Attention work lists (items, merges) and their counts {items, merges};
  // partial results of split sequences.
  uint32_t *items_d_, *merges_d_, *counts_d_, *off_d_;
  float* partials_;
  // Pinned staging.
  int32_t *ids_h_, *pos_h_, *vcol_h_;
  uint32_t *items_h_, *merges_h_, *counts_h_, *off_h_;
  eg2::AttentionCounts attn_cap_{};
  bool staged_merge_ = false;
  float* out_h_;

  std::map<unsigned, hipGraphExec_t> graphs_;  // key: 2 * padded rows + (wave has split sequences)
  unsigned staged_tokens_ = 0, staged_rows_ = 0;
  size_t staged_batch_ = 0;
  std::map<std::string, double> timings_;

  template <class T>
  T* dalloc(size_t n) {
    void* p = nullptr;
    check(hipMalloc(&p, n * sizeof(T) + 256), "hipMalloc");
    dev_allocs_.push_back(p);
    return static_cast<T*>(p);
  }
  template <class T>
  T* halloc(size_t n) {
    void* p = nullptr;
    check(hipHostMalloc(&p, n * sizeof(T) + 256, hipHostMallocDefault), "hipHostMalloc");
    host_allocs_.push_back(p);
    return static_cast<T*>(p);
  }
  const ei_tensor* tensor(const std::string& name, bool required = true) const;
  const ei_kv* kv(const char* key) const;
  double kv_f64(const char* key, double dflt) const;
  uint64_t kv_u64(const char* key, uint64_t dflt) const;
  const float* upload_vector(const std::string& name, int n);
  std::vector<uint8_t> q8_rows(const std::string& name, int k, int m) const;
  DevMat upload_q8(const std::vector<const std::vector<uint8_t>*>& parts, int k);
  DevMat upload_q8_geglu(const std::vector<uint8_t>& gate, const std::vector<uint8_t>& up, int k);
  void launch(const char* name, hipError_t e);
  void record_layers(unsigned rows, bool merge);
  void gemm(const char* name, const int8_t* xq, const float* xd, const DevMat& w, float* y, int n, int ldy,
            hipStream_t s);
  void wait(const char* what);
};

const ei_tensor* Backend::tensor(const std::string& name, bool required) const {
  for (uint64_t i = 0; i < model_->n_tensors; ++i)
    if (str_eq(model_->tensors[i].name, name.c_str())) return &model_->tensors[i];
  if (required) throw std::runtime_error("missing tensor: " + name);
  return nullptr;
}

const ei_kv* Backend::kv(const char* key) const {
  for (uint64_t i = 0; i < model_->n_kv; ++i)
    if (str_eq(model_->kv[i].key, key)) return &model_->kv[i];
  return nullptr;
}

// model.c:71-77 read these through ei_gguf_kv_f64/_u64, which take the
// normalised union member (gguf.c:46-61); an integer-typed key read as a
// float (or the reverse) is converted here instead of reinterpreted.
double Backend::kv_f64(const char* key, double dflt) const {
  const ei_kv* k = kv(key);
  if (!k) return dflt;
  switch (k->type) {
    case EI_GGUF_F32:
    case EI_GGUF_F64: return k->v.f64;
    case EI_GGUF_I8: case EI_GGUF_I16: case EI_GGUF_I32: case EI_GGUF_I64: return (double)k->v.i64;
    case EI_GGUF_U8: case EI_GGUF_U16: case EI_GGUF_U32: case EI_GGUF_U64: return (double)k->v.u64;
    default: throw std::runtime_error(std::string("GGUF key is not numeric: ") + key);
  }
}

uint64_t Backend::kv_u64(const char* key, uint64_t dflt) const {
  const ei_kv* k = kv(key);
  if (!k) return dflt;
  switch (k->type) {
    case EI_GGUF_U8: case EI_GGUF_U16: case EI_GGUF_U32: case EI_GGUF_U64: return k->v.u64;
    case EI_GGUF_I8: case EI_GGUF_I16: case EI_GGUF_I32: case EI_GGUF_I64:
      if (k->v.i64 < 0) throw std::runtime_error(std::string("negative GGUF key: ") + key);
      return (uint64_t)k->v.i64;
    default: throw std::runtime_error(std::string("GGUF key is not an integer: ") + key);
  }
}

const float* Backend::upload_vector(const std::string& name, int n) {
  const ei_tensor* t = tensor(name);
  if (t->type != EI_T_F32 || t->ne[0] != (uint64_t)n || t->ne[1] != 1)
    throw std::runtime_error("norm requires F32[" + std::to_string(n) + "]: " + name);
  float* d = dalloc<float>(n);
  check(hipMemcpy(d, t->data, n * sizeof(float), hipMemcpyHostToDevice), "upload");
  return d;
}

// Raw Q8_0 rows of a [k, m] (ne[0] = k) matrix, validated (model.c:93-99 with Q8_0).
std::vector<uint8_t> Backend::q8_rows(const std::string& name, int k, int m) const {
  const ei_tensor* t = tensor(name);
  if (t->type != EI_T_Q8_0) throw std::runtime_error("matrix must be Q8_0: " + name);
  if (t->ne[0] != (uint64_t)k || t->ne[1] != (uint64_t)m || t->ne[2] != 1 || t->ne[3] != 1)
    throw std::runtime_error("unexpected shape: " + name);
  const size_t bytes = (size_t)m * (k / 32) * 34;
  const uint8_t* p = static_cast<const uint8_t*>(t->data);
  return std::vector<uint8_t>(p, p + bytes);
}

// Concatenates matrices along the output dimension and uploads them in the
// GEMM's operand layout (row tiles + transposed block scales).
DevMat Backend::upload_q8(const std::vector<const std::vector<uint8_t>*>& parts, int k) {
  std::vector<uint8_t> rows_q8;
  for (auto* p : parts) rows_q8.insert(rows_q8.end(), p->begin(), p->end());
  const size_t rows = rows_q8.size() / ((size_t)(k / 32) * 34);
  DevMat mat;
  mat.m = (int)rows;
  mat.k = k;
  mat.ld = (int)((rows + 31) / 32 * 32);
  std::vector<int8_t> q(eg2_q8_tile_bytes(rows, (unsigned)k));
  std::vector<float> d((size_t)(k / 32) * mat.ld);
  eg2_q8_weight_tiles(rows_q8.data(), rows, (unsigned)k, q.data(), d.data());
  mat.q = dalloc<int8_t>(q.size());
  mat.d = dalloc<float>(d.size());
  check(hipMemcpy(mat.q, q.data(), q.size(), hipMemcpyHostToDevice), "upload");
  check(hipMemcpy(mat.d, d.data(), d.size() * sizeof(float), hipMemcpyHostToDevice), "upload");
  return mat;
}

// The gate and up matrices interleaved in 32-row groups, the operand of
// the fused gate|up + GeGLU GEMM.
DevMat Backend::upload_q8_geglu(const std::vector<uint8_t>& gate, const std::vector<uint8_t>& up, int k) {
  const size_t ff = gate.size() / ((size_t)(k / 32) * 34);
  DevMat mat;
  mat.m = (int)(2 * ff);
  mat.k = k;
  mat.ld = mat.m;
  std::vector<int8_t> q(eg2_q8_tile_bytes(2 * ff, (unsigned)k));
  std::vector<float> d((size_t)(k / 32) * mat.ld);
  if (up.size() != gate.size() || eg2_q8_geglu_weight_tiles(gate.data(), up.data(), ff, (unsigned)k, q.data(), d.data()))
    throw std::runtime_error("ffn_gate / ffn_up shapes");
  mat.q = dalloc<int8_t>(q.size());
  mat.d = dalloc<float>(d.size());
  check(hipMemcpy(mat.q, q.data(), q.size(), hipMemcpyHostToDevice), "upload");
  check(hipMemcpy(mat.d, d.data(), d.size() * sizeof(float), hipMemcpyHostToDevice), "upload");
  return mat;
}

Backend::Backend(const ei_gguf* g) : model_(g) {
  if (!g || !g->tensors) throw std::runtime_error("empty GGUF");
  char why[256];
  if (eg2_hip_device_check(why, sizeof why) != 0)
    throw std::runtime_error(std::string("supported HIP device not found (gfx950): ") + why);
  use_graph_ = env_flag("EG2_HIP_GRAPH", true);
  profile_ = env_flag("EG2_HIP_PROFILE", false);

  const ei_kv* arch = kv("general.architecture");
  if (!arch || arch->type != EI_GGUF_STRING || !str_eq(arch->v.s, "gemma-embedding"))
    throw std::runtime_error("expected a gemma-embedding GGUF");
  auto hp = [&](const char* key, uint64_t want) {
    if (kv_u64(key, 0) != want) throw std::runtime_error(std::string("unsupported hyper-parameter ") + key);
  };
  hp("gemma-embedding.embedding_length", kEmbd);
  hp("gemma-embedding.feed_forward_length", kFF);
  hp("gemma-embedding.attention.head_count", 3);
  hp("gemma-embedding.attention.head_count_kv", 1);
  hp("gemma-embedding.attention.key_length", kHeadDim);
  hp("gemma-embedding.attention.value_length", kHeadDim);
  const uint64_t n_layer = kv_u64("gemma-embedding.block_count", 0);
  if (n_layer < 1 || n_layer > 64) throw std::runtime_error("block_count must be 1..64");
  eps_ = (float)kv_f64("gemma-embedding.attention.layer_norm_rms_epsilon", 1e-6);
  const float base_full = (float)kv_f64("gemma-embedding.rope.freq_base", 1000000.0);
  const float base_swa = (float)kv_f64("gemma-embedding.rope.freq_base_swa", 10000.0);
  const uint64_t swa_window = kv_u64("gemma-embedding.attention.sliding_window", 512);
  const uint64_t swa_period = kv_u64("gemma-embedding.attention.sliding_window_pattern", 6);
  if (swa_period == 0) throw std::runtime_error("sliding_window_pattern must be positive");
  if (swa_window > 2 * kCap) throw std::runtime_error("sliding_window too large");

  check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");

  // RoPE tables, one per distinct base (kernels.c:245-249 values).
  std::vector<float> table((size_t)kCap * kHeadDim);
  std::map<float, const float*> ropes;
  for (float base : {base_full, base_swa}) {
    if (ropes.count(base)) continue;
    eg2_rope_table(base, kCap, table.data());
    float* d = dalloc<float>(table.size());
    check(hipMemcpy(d, table.data(), table.size() * sizeof(float), hipMemcpyHostToDevice), "upload");
    ropes[base] = d;
  }

  const ei_tensor* emb = tensor("token_embd.weight");
  if (emb->type != EI_T_Q8_0 || emb->ne[0] != (uint64_t)kEmbd || emb->ne[1] != (uint64_t)kVocab)
    throw std::runtime_error("token_embd.weight must be Q8_0 [768, 262144]");
  if (reinterpret_cast<uintptr_t>(emb->data) % 2 != 0) throw std::runtime_error("token_embd.weight misaligned");
  {
    uint8_t* d = dalloc<uint8_t>(emb->n_bytes);
    check(hipMemcpy(d, emb->data, emb->n_bytes, hipMemcpyHostToDevice), "upload");
    token_embd_ = d;
  }
  output_norm_ = upload_vector("output_norm.weight", kEmbd);

  for (uint64_t il = 0; il < n_layer; ++il) {
    const std::string p = "blk." + std::to_string(il) + ".";
    Layer L{};
    auto wq = q8_rows(p + "attn_q.weight", kEmbd, 768), wk = q8_rows(p + "attn_k.weight", kEmbd, 256),
         wv = q8_rows(p + "attn_v.weight", kEmbd, 256);
    L.qkv = upload_q8({&wq, &wk, &wv}, kEmbd);
    auto wo = q8_rows(p + "attn_output.weight", 768, kEmbd);
    L.o = upload_q8({&wo}, 768);
    auto wg = q8_rows(p + "ffn_gate.weight", kEmbd, kFF), wu = q8_rows(p + "ffn_up.weight", kEmbd, kFF);
    L.gu = upload_q8_geglu(wg, wu, kEmbd);
    auto wd = q8_rows(p + "ffn_down.weight", kFF, kEmbd);
    L.down = upload_q8({&wd}, kFF);
    L.attn_norm = upload_vector(p + "attn_norm.weight", kEmbd);
    L.q_norm = upload_vector(p + "attn_q_norm.weight", kHeadDim);
    L.k_norm = upload_vector(p + "attn_k_norm.weight", kHeadDim);
    L.post_attn = upload_vector(p + "post_attention_norm.weight", kEmbd);
    L.ffn_norm = upload_vector(p + "ffn_norm.weight", kEmbd);
    L.post_ffw = upload_vector(p + "post_ffw_norm.weight", kEmbd);
    // model.c:123-127: in each period the last layer is full attention.
    const bool swa = (il % swa_period) < (swa_period - 1);
    L.rope = ropes[swa ? base_swa : base_full];
    L.window = swa ? (int)swa_window : 0;
    layers_.push_back(L);
  }
  // Optional dense head (EXTRACTION.md:178-181: dense_2 {768, 3072}, dense_3 {3072, 768}).
  const ei_tensor* d2 = tensor("dense_2.weight", false);
  const ei_tensor* d3 = tensor("dense_3.weight", false);
  if ((d2 == nullptr) != (d3 == nullptr)) throw std::runtime_error("dense_2/dense_3 must be both present or absent");
  if (d2) {
    auto a = q8_rows("dense_2.weight", kEmbd, kDenseFF), b = q8_rows("dense_3.weight", kDenseFF, kEmbd);
    dense2_ = upload_q8({&a}, kEmbd);
    dense3_ = upload_q8({&b}, kDenseFF);
    dense_ = true;
  }

  x_ = dalloc<float>((size_t)kCap * kEmbd);
  h_ = dalloc<float>((size_t)kCap * kEmbd);
  qkv_ = dalloc<float>((size_t)kCap * kQKV);
  xq_ = dalloc<int8_t>(eg2_q8_tile_bytes(kCap, kFF));
  xd_ = dalloc<float>((size_t)kCap * (kFF / 32));
  cq_ = dalloc<int8_t>(eg2_q8_tile_bytes(kCap, kEmbd));
  cd_ = dalloc<float>((size_t)kCap * (kEmbd / 32));
  qs_ = dalloc<_Float16>((size_t)kCap * 2 * kEmbd);
  ks_ = dalloc<_Float16>((size_t)kCap * 2 * kHeadDim);
  // Columns no token writes are read (masked) by the attention kernel and
  // must hold finite values: zero the buffer once.
  vt_ = dalloc<_Float16>((size_t)2 * kHeadDim * kVtCols);
  check(hipMemset(vt_, 0, (size_t)2 * kHeadDim * kVtCols * sizeof(_Float16)), "hipMemset");
  ids_d_ = dalloc<int32_t>(kCap);
  pos_d_ = dalloc<int32_t>(kCap);
  vcol_d_ = dalloc<int32_t>(kCap);
  // Capacity for the wave cap plus the padding sequence (rows rounded to 32).
  attn_cap_ = eg2::attention_capacity(kCap + 32, kCap + 1);
  items_d_ = dalloc<uint32_t>(8 * (size_t)attn_cap_.items);
  merges_d_ = dalloc<uint32_t>(4 * (size_t)std::max(1u, attn_cap_.merges));
  counts_d_ = dalloc<uint32_t>(2);
  partials_ = dalloc<float>(eg2::kAttentionPartialFloats * std::max(1u, attn_cap_.slots));
  off_d_ = dalloc<uint32_t>(kCap + 1);
  pooled_ = dalloc<float>((size_t)kCap * kEmbd);
  mid_ = dalloc<float>((size_t)kCap * kDenseFF);
  mid_q_ = dalloc<int8_t>(eg2_q8_tile_bytes(kCap, kDenseFF));
  mid_d_ = dalloc<float>((size_t)kCap * (kDenseFF / 32));
  ids_h_ = halloc<int32_t>(kCap);
  pos_h_ = halloc<int32_t>(kCap);
  vcol_h_ = halloc<int32_t>(kCap);
  items_h_ = halloc<uint32_t>(8 * (size_t)attn_cap_.items);
  merges_h_ = halloc<uint32_t>(4 * (size_t)std::max(1u, attn_cap_.merges));
  counts_h_ = halloc<uint32_t>(2);
  off_h_ = halloc<uint32_t>(kCap + 1);
  out_h_ = halloc<float>((size_t)kCap * kEmbd);
  check(hipDeviceSynchronize(), "upload");

  size_t bytes = 0;
  for (auto& L : layers_)
    for (const DevMat* w : {&L.qkv, &L.o, &L.gu, &L.down})
      bytes += eg2_q8_tile_bytes(w->m, w->k) + (size_t)(w->k / 32) * w->ld * sizeof(float);
  std::fprintf(stderr, "HIP: gfx950, %zu layers, Q8_0 layer weights %.1f MiB (int8 row tiles + scales), embedding table %.1f MiB, cap %u packed tokens%s\n",
               layers_.size(), bytes / 1048576.0, emb->n_bytes / 1048576.0, kCap, dense_ ? ", dense head" : "");
}

Backend::~Backend() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (auto& kvp : graphs_) (void)hipGraphExecDestroy(kvp.second);
  if (stream_) (void)hipStreamDestroy(stream_);
  for (void* p : dev_allocs_) (void)hipFree(p);
  for (void* p : host_allocs_) (void)hipHostFree(p);
}

void Backend::launch(const char* name, hipError_t e) {
  if (e != hipSuccess) throw std::runtime_error(std::string(name) + ": " + hipGetErrorString(e));
}

// y[n][w.m] (row stride ldy) = activations (row tiles xq, scales xd
// [k/32][n]) times the weights w.
void Backend::gemm(const char* name, const int8_t* xq, const float* xd, const DevMat& w, float* y, int n, int ldy,
                   hipStream_t s) {
  launch(name, eg2::launch_gemm_q8(xq, xd, n, w.q, w.d, w.ld, y, n, w.m, w.k, ldy, s));
}

// The per-wave layer stack for `rows` (padded) token rows: embedding + norm,
// then per layer (engine.c:1115-1127 order) QKV GEMM, QK-norm/RoPE,
// attention (+Q8_0; with `merge`, the merge of split sequences' key-chunk
// partials), O GEMM, residual + ffn_norm (+Q8_0), gate|up GEMM with the
// GeGLU (+Q8_0) in its epilogue, down GEMM, residual + next attn_norm
// (+Q8_0); finally the
// output_norm per token (the first half of kernels.c:417-427).
void Backend::record_layers(unsigned rows, bool merge) {
  hipStream_t s = stream_;
  const int n = (int)rows;
  launch("embed", eg2::launch_embed_norm_quant(token_embd_, ids_d_, n, std::sqrt((float)kEmbd), layers_[0].attn_norm,
                                               eps_, x_, xq_, xd_, s));
  for (size_t il = 0; il < layers_.size(); ++il) {
    const Layer& L = layers_[il];
    gemm("gemm_qkv", xq_, xd_, L.qkv, qkv_, n, kQKV, s);
    launch("qk_norm_rope", eg2::launch_qk_norm_rope(qkv_, L.q_norm, L.k_norm, L.rope, pos_d_, vcol_d_, eps_, qs_, ks_,
                                                    vt_, kVtCols, n, s));
    launch("attention", eg2::launch_attention(qs_, ks_, vt_, kVtCols, vcol_d_, items_d_, counts_d_, (n + 7) / 8,
                                              L.window, n, cq_, cd_, partials_, s));
    if (merge)
      launch("attention_merge",
             eg2::launch_attention_merge(merges_d_, counts_d_ + 1, (n + 3) / 4, partials_, n, cq_, cd_, s));
    gemm("gemm_o", cq_, cd_, L.o, h_, n, kEmbd, s);
    // The FFN input goes to the attention context's buffers (free after the
    // O GEMM), so the fused gate|up + GeGLU kernel reads them and writes xq.
    launch("residual", eg2::launch_residual_norm_quant(x_, h_, L.post_attn, L.ffn_norm, eps_, cq_, cd_, n, s));
    launch("gemm_gate_up_geglu", eg2::launch_gemm_q8_geglu(cq_, cd_, n, L.gu.q, L.gu.d, L.gu.ld, xq_, xd_, n, n, kFF,
                                                            kEmbd, s));
    gemm("gemm_down", xq_, xd_, L.down, h_, n, kEmbd, s);
    const float* next = il + 1 < layers_.size() ? layers_[il + 1].attn_norm : nullptr;
    launch("residual", eg2::launch_residual_norm_quant(x_, h_, L.post_ffw, next, eps_, xq_, xd_, n, s));
  }
  launch("output_norm", eg2::launch_rms_norm_rows(x_, output_norm_, eps_, n, s));
}

void Backend::wait(const char* what) {
  const auto start = std::chrono::steady_clock::now();
  for (;;) {
    const hipError_t e = hipStreamQuery(stream_);
    if (e == hipSuccess) return;
    if (e != hipErrorNotReady) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
    if (std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count() > kTimeoutSeconds)
      throw std::runtime_error(std::string(what) + ": timed out");
    std::this_thread::yield();
  }
}

void Backend::batch(const int32_t* ids, const size_t* offsets, size_t batch, float* out) {
  std::lock_guard<std::mutex> guard(mutex_);
  const auto t0 = std::chrono::steady_clock::now();
  stage(ids, offsets, batch);
  launch_staged(1);
  collect(out);
  if (profile_) {
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    std::fprintf(stderr, "HIP_PROFILE {\"tokens\":%u,\"batch\":%zu,\"wall_ms\":%.3f,\"layers_ms\":%.3f}\n",
                 staged_tokens_, staged_batch_, ms, timings_["layers"]);
    timings_.clear();
  }
}

void Backend::stage(const int32_t* ids, const size_t* offsets, size_t batch) {
  if (poisoned_) throw std::runtime_error("HIP context failed; restart process before reuse");
  staged_batch_ = 0;
  // src/gemma2_kfd.cpp:271-278
  if (!ids || !offsets || !batch || batch > kCap || offsets[0] || offsets[batch] > kCap)
    throw std::runtime_error("HIP batch requires 1..2048 packed tokens and nonempty sequences");
  for (size_t s = 0; s < batch; ++s)
    if (offsets[s + 1] <= offsets[s]) throw std::runtime_error("invalid HIP sequence offsets");
  const unsigned n = (unsigned)offsets[batch];
  for (unsigned i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= kVocab) throw std::runtime_error("token ID out of range");

  // Metadata; rows [n, rows) form one dummy sequence that is never pooled.
  const unsigned rows = (n + 31) / 32 * 32;
  for (size_t s = 0; s < batch; ++s)
    for (size_t t = offsets[s]; t < offsets[s + 1]; ++t) {
      ids_h_[t] = ids[t];
      pos_h_[t] = (int32_t)(t - offsets[s]);
    }
  for (unsigned t = n; t < rows; ++t) {
    ids_h_[t] = 0;
    pos_h_[t] = (int32_t)(t - n);
  }
  for (size_t s = 0; s <= batch; ++s) off_h_[s] = (uint32_t)offsets[s];
  // Attention work lists; the padding rows form one more sequence.
  std::vector<size_t> all(offsets, offsets + batch + 1);
  if (rows > n) all.push_back(rows);
  const eg2::AttentionCounts ac = eg2::build_attention_items(all.data(), all.size() - 1, items_h_, merges_h_);
  if (ac.items > attn_cap_.items || ac.merges > attn_cap_.merges || ac.slots > attn_cap_.slots)
    throw std::runtime_error("attention work list exceeds its capacity");
  counts_h_[0] = ac.items;
  counts_h_[1] = ac.merges;
  const bool merge = ac.merges > 0;
  // Transposed-v columns: the padding rows form one more sequence.
  const size_t cols = eg2::build_vt_columns(offsets, batch, vcol_h_);
  for (unsigned t = n; t < rows; ++t) vcol_h_[t] = (int32_t)(cols + (t - n));

  poisoned_ = true;  // cleared only when the whole wave completed
  hipStream_t s = stream_;
  check(hipMemcpyAsync(ids_d_, ids_h_, rows * sizeof(int32_t), hipMemcpyHostToDevice, s), "copy ids");
  check(hipMemcpyAsync(pos_d_, pos_h_, rows * sizeof(int32_t), hipMemcpyHostToDevice, s), "copy positions");
  check(hipMemcpyAsync(vcol_d_, vcol_h_, rows * sizeof(int32_t), hipMemcpyHostToDevice, s), "copy columns");
  check(hipMemcpyAsync(items_d_, items_h_, 8 * (size_t)ac.items * sizeof(uint32_t), hipMemcpyHostToDevice, s),
        "copy attention items");
  if (merge)
    check(hipMemcpyAsync(merges_d_, merges_h_, 4 * (size_t)ac.merges * sizeof(uint32_t), hipMemcpyHostToDevice, s),
          "copy attention merges");
  check(hipMemcpyAsync(counts_d_, counts_h_, 2 * sizeof(uint32_t), hipMemcpyHostToDevice, s), "copy attention counts");
  check(hipMemcpyAsync(off_d_, off_h_, (batch + 1) * sizeof(uint32_t), hipMemcpyHostToDevice, s), "copy offsets");
  const unsigned key = 2 * rows + (merge ? 1 : 0);
  if (use_graph_ && !profile_ && graphs_.find(key) == graphs_.end()) {
    hipGraph_t graph = nullptr;
    check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    try {
      record_layers(rows, merge);
    } catch (...) {
      (void)hipStreamEndCapture(s, &graph);
      if (graph) (void)hipGraphDestroy(graph);
      throw;
    }
    check(hipStreamEndCapture(s, &graph), "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    const hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    check(e, "hipGraphInstantiate");
    graphs_.emplace(key, exec);
  }
  staged_merge_ = merge;
  staged_tokens_ = n;
  staged_rows_ = rows;
  staged_batch_ = batch;
}

// Layer stack (graph or eager), then kernels.c:417-427 (mean + L2 per
// sequence) and the dense head.
void Backend::launch_staged(unsigned repeats) {
  if (!staged_batch_) throw std::runtime_error("no staged wave");
  hipStream_t s = stream_;
  const int B = (int)staged_batch_;
  poisoned_ = true;
  for (unsigned r = 0; r < repeats; ++r) {
    if (use_graph_ && !profile_) {
      check(hipGraphLaunch(graphs_.at(2 * staged_rows_ + (staged_merge_ ? 1 : 0)), s), "hipGraphLaunch");
    } else if (profile_) {
      // Per-stage timing needs events around eager launches; the totals are
      // printed like the reference's KFD_PROFILE line (src/gemma2_kfd.cpp:346-352).
      hipEvent_t a, b;
      check(hipEventCreate(&a), "hipEventCreate");
      check(hipEventCreate(&b), "hipEventCreate");
      check(hipEventRecord(a, s), "hipEventRecord");
      record_layers(staged_rows_, staged_merge_);
      check(hipEventRecord(b, s), "hipEventRecord");
      check(hipEventSynchronize(b), "hipEventSynchronize");
      float ms = 0;
      (void)hipEventElapsedTime(&ms, a, b);
      timings_["layers"] += ms;
      (void)hipEventDestroy(a);
      (void)hipEventDestroy(b);
    } else {
      record_layers(staged_rows_, staged_merge_);
    }
    launch("pool", eg2::launch_pool_l2(x_, off_d_, pooled_, B, s));
    if (dense_) {
      launch("dense_quant", eg2::launch_quantize_rows(pooled_, kEmbd, cq_, cd_, B, s));
      gemm("dense_2", cq_, cd_, dense2_, mid_, B, kDenseFF, s);
      launch("dense_quant", eg2::launch_quantize_rows(mid_, kDenseFF, mid_q_, mid_d_, B, s));
      gemm("dense_3", mid_q_, mid_d_, dense3_, pooled_, B, kEmbd, s);
      launch("dense_l2", eg2::launch_l2_prefix(pooled_, kEmbd, kEmbd, B, s));
    }
  }
}

void Backend::collect(float* out) {
  if (!staged_batch_) throw std::runtime_error("no staged wave");
  if (!out) throw std::runtime_error("null output");
  const int B = (int)staged_batch_;
  check(hipMemcpyAsync(out_h_, pooled_, (size_t)B * kEmbd * sizeof(float), hipMemcpyDeviceToHost, stream_),
        "copy out");
  wait("HIP wave");
  poisoned_ = false;

  // src/gemma2_kfd.cpp:337-343 rejects non-finite or zero embeddings.
  for (int r = 0; r < B; ++r) {
    double ss = 0;
    for (int z = 0; z < kEmbd; ++z) {
      const float f = out_h_[(size_t)r * kEmbd + z];
      if (!std::isfinite(f)) throw std::runtime_error("nonfinite GPU output");
      ss += (double)f * f;
    }
    if (ss <= 0) throw std::runtime_error("zero GPU embedding");
  }
  std::memcpy(out, out_h_, (size_t)B * kEmbd * sizeof(float));
}

}  // namespace

extern "C" void* ei_gemma2_kfd_create(const ei_gguf* g, char* err, size_t len) {
  try {
    return new Backend(g);
  } catch (const std::exception& e) {
    if (err && len) std::snprintf(err, len, "HIP: %s", e.what());
    return nullptr;
  }
}

extern "C" void ei_gemma2_kfd_free(void* ctx) { delete static_cast<Backend*>(ctx); }

extern "C" bool ei_gemma2_kfd_batch(void* ctx, const int32_t* ids, const size_t* offsets, size_t batch, float* out,
                                    char* err, size_t len) {
  try {
    if (!ctx) throw std::runtime_error("empty context");
    if (!out) throw std::runtime_error("HIP batch requires 1..2048 packed tokens and nonempty sequences");
    static_cast<Backend*>(ctx)->batch(ids, offsets, batch, out);
    return true;
  } catch (const std::exception& e) {
    if (err && len) std::snprintf(err, len, "HIP: %s", e.what());
    return false;
  }
}

extern "C" bool eg2_kfd_stage(void* ctx, const int32_t* ids, const size_t* offsets, size_t batch, char* err,
                              size_t len) {
  try {
    if (!ctx) throw std::runtime_error("empty context");
    Backend* b = static_cast<Backend*>(ctx);
    std::lock_guard<std::mutex> guard(b->mutex());
    b->stage(ids, offsets, batch);
    return true;
  } catch (const std::exception& e) {
    if (err && len) std::snprintf(err, len, "HIP: %s", e.what());
    return false;
  }
}

extern "C" bool eg2_kfd_launch_staged(void* ctx, unsigned repeats, char* err, size_t len) {
  try {
    if (!ctx) throw std::runtime_error("empty context");
    Backend* b = static_cast<Backend*>(ctx);
    std::lock_guard<std::mutex> guard(b->mutex());
    b->launch_staged(repeats);
    return true;
  } catch (const std::exception& e) {
    if (err && len) std::snprintf(err, len, "HIP: %s", e.what());
    return false;
  }
}

extern "C" bool eg2_kfd_collect(void* ctx, float* out, char* err, size_t len) {
  try {
    if (!ctx) throw std::runtime_error("empty context");
    Backend* b = static_cast<Backend*>(ctx);
    std::lock_guard<std::mutex> guard(b->mutex());
    b->collect(out);
    return true;
  } catch (const std::exception& e) {
    if (err && len) std::snprintf(err, len, "HIP: %s", e.what());
    return false;
  }
}
