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
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <condition_variable>
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
constexpr unsigned kPoolSplitLen = 256;  // longest sequence above which pooling spreads over columns
// The attention's softmax takes one of four equivalent kernel forms by the
// wave's longest sequence (eg2::kSoftmaxLanes16, kSoftmaxLanes32,
// kSoftmaxWave, longer); a graph is kept per padded row count and form, and
// records the form's bound as its longest.
inline unsigned softmax_form(unsigned longest) {
  return longest <= (unsigned)eg2::kSoftmaxLanes16 ? 0u
         : longest <= (unsigned)eg2::kSoftmaxLanes32 ? 1u
         : longest <= (unsigned)eg2::kSoftmaxWave ? 2u
                                                  : 3u;
}
inline unsigned attention_form(unsigned longest) {
  const unsigned bound[4] = {(unsigned)eg2::kSoftmaxLanes16, (unsigned)eg2::kSoftmaxLanes32,
                             (unsigned)eg2::kSoftmaxWave, kCap};
  return bound[softmax_form(longest)];
}
inline unsigned graph_key(unsigned rows, unsigned longest) { return 4 * rows + softmax_form(longest); }
constexpr int kEmbd = 768, kFF = 1152, kHeadDim = 256, kQKV = 768 + 2 * 256, kDenseFF = 3072;
constexpr int kVocab = 262144;
constexpr double kTimeoutSeconds = 30.0;  // src/gemma2_kfd.cpp:21

std::string fixed3(double v) {
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.3f", v);
  return buf;
}

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

const ei_tensor* find_tensor(const ei_gguf* g, const std::string& name) {
  for (uint64_t i = 0; i < g->n_tensors; ++i)
    if (str_eq(g->tensors[i].name, name.c_str())) return &g->tensors[i];
  return nullptr;
}

// A tensor of `type` with shape [ne0, ne1] (ne[2] = ne[3] = 1) whose byte
// count is exactly what that shape takes, with its data present
// (model.c:79-105 names; model.c:93-99 checks type and shape). Every tensor
// the executor uploads goes through this check first, so no upload or
// kernel reads past a tensor whose record disagrees with its shape.
const ei_tensor* checked_tensor(const ei_gguf* g, const std::string& name, uint32_t type, uint64_t ne0, uint64_t ne1,
                                bool required = true) {
  const ei_tensor* t = find_tensor(g, name);
  if (!t) {
    if (required) throw std::runtime_error("missing tensor: " + name);
    return nullptr;
  }
  const uint64_t want_bytes = type == EI_T_Q8_0 ? ne1 * (ne0 / 32) * 34 : ne0 * ne1 * 4;
  const bool ok_type = t->type == type && (type == EI_T_Q8_0 || type == EI_T_F32);
  if (!ok_type || (type == EI_T_Q8_0 && ne0 % 32 != 0))
    throw std::runtime_error("unexpected type: " + name + (type == EI_T_Q8_0 ? " (need Q8_0)" : " (need F32)"));
  if (t->n_dims < 1 || t->n_dims > 4 || t->ne[0] != ne0 || t->ne[1] != ne1 || t->ne[2] != 1 || t->ne[3] != 1)
    throw std::runtime_error("unexpected shape: " + name + " (need [" + std::to_string(ne0) + ", " +
                             std::to_string(ne1) + "])");
  if (t->n_bytes != want_bytes || !t->data) throw std::runtime_error("unexpected byte count: " + name);
  return t;
}

const ei_kv* find_kv(const ei_gguf* g, const char* key) {
  for (uint64_t i = 0; i < g->n_kv; ++i)
    if (str_eq(g->kv[i].key, key)) return &g->kv[i];
  return nullptr;
}

// model.c:71-77 read these through ei_gguf_kv_f64/_u64, which take the
// normalised union member (gguf.c:46-61); an integer-typed key read as a
// float (or the reverse) is converted here instead of reinterpreted.
double kv_f64(const ei_gguf* g, const char* key, double dflt) {
  const ei_kv* k = find_kv(g, key);
  if (!k) return dflt;
  switch (k->type) {
    case EI_GGUF_F32:
    case EI_GGUF_F64: return k->v.f64;
    case EI_GGUF_I8: case EI_GGUF_I16: case EI_GGUF_I32: case EI_GGUF_I64: return (double)k->v.i64;
    case EI_GGUF_U8: case EI_GGUF_U16: case EI_GGUF_U32: case EI_GGUF_U64: return (double)k->v.u64;
    default: throw std::runtime_error(std::string("GGUF key is not numeric: ") + key);
  }
}

uint64_t kv_u64(const ei_gguf* g, const char* key, uint64_t dflt) {
  const ei_kv* k = find_kv(g, key);
  if (!k) return dflt;
  switch (k->type) {
    case EI_GGUF_U8: case EI_GGUF_U16: case EI_GGUF_U32: case EI_GGUF_U64: return k->v.u64;
    case EI_GGUF_I8: case EI_GGUF_I16: case EI_GGUF_I32: case EI_GGUF_I64:
      if (k->v.i64 < 0) throw std::runtime_error(std::string("negative GGUF key: ") + key);
      return (uint64_t)k->v.i64;
    default: throw std::runtime_error(std::string("GGUF key is not an integer: ") + key);
  }
}

// Everything the executor reads from the model, checked on the host before
// any device call: the architecture, the hyper-parameters this build's
// kernels are specialised for (model.c:61-77), and the type, shape and byte
// count of every tensor (model.c:79-105, plus the optional dense_2 /
// dense_3 of EXTRACTION.md:178-181). Returns the layer count.
uint64_t validate_model(const ei_gguf* g) {
  if (!g || !g->tensors) throw std::runtime_error("empty GGUF");
  const ei_kv* arch = find_kv(g, "general.architecture");
  if (!arch || arch->type != EI_GGUF_STRING || !str_eq(arch->v.s, "gemma-embedding"))
    throw std::runtime_error("expected a gemma-embedding GGUF");
  auto hp = [&](const char* key, uint64_t want) {
    if (kv_u64(g, key, 0) != want) throw std::runtime_error(std::string("unsupported hyper-parameter ") + key);
  };
  hp("gemma-embedding.embedding_length", kEmbd);
  hp("gemma-embedding.feed_forward_length", kFF);
  hp("gemma-embedding.attention.head_count", 3);
  hp("gemma-embedding.attention.head_count_kv", 1);
  hp("gemma-embedding.attention.key_length", kHeadDim);
  hp("gemma-embedding.attention.value_length", kHeadDim);
  const uint64_t n_layer = kv_u64(g, "gemma-embedding.block_count", 0);
  if (n_layer < 1 || n_layer > 64) throw std::runtime_error("block_count must be 1..64");
  (void)kv_f64(g, "gemma-embedding.attention.layer_norm_rms_epsilon", 1e-6);
  (void)kv_f64(g, "gemma-embedding.rope.freq_base", 1000000.0);
  (void)kv_f64(g, "gemma-embedding.rope.freq_base_swa", 10000.0);
  if (kv_u64(g, "gemma-embedding.attention.sliding_window_pattern", 6) == 0)
    throw std::runtime_error("sliding_window_pattern must be positive");
  if (kv_u64(g, "gemma-embedding.attention.sliding_window", 512) > 2 * kCap)
    throw std::runtime_error("sliding_window too large");

  const ei_tensor* emb = checked_tensor(g, "token_embd.weight", EI_T_Q8_0, kEmbd, kVocab);
  if (reinterpret_cast<uintptr_t>(emb->data) % 2 != 0) throw std::runtime_error("token_embd.weight misaligned");
  checked_tensor(g, "output_norm.weight", EI_T_F32, kEmbd, 1);
  for (uint64_t il = 0; il < n_layer; ++il) {
    const std::string p = "blk." + std::to_string(il) + ".";
    checked_tensor(g, p + "attn_q.weight", EI_T_Q8_0, kEmbd, 768);
    checked_tensor(g, p + "attn_k.weight", EI_T_Q8_0, kEmbd, 256);
    checked_tensor(g, p + "attn_v.weight", EI_T_Q8_0, kEmbd, 256);
    checked_tensor(g, p + "attn_output.weight", EI_T_Q8_0, 768, kEmbd);
    checked_tensor(g, p + "ffn_gate.weight", EI_T_Q8_0, kEmbd, kFF);
    checked_tensor(g, p + "ffn_up.weight", EI_T_Q8_0, kEmbd, kFF);
    checked_tensor(g, p + "ffn_down.weight", EI_T_Q8_0, kFF, kEmbd);
    for (const char* v : {"attn_norm.weight", "post_attention_norm.weight", "ffn_norm.weight", "post_ffw_norm.weight"})
      checked_tensor(g, p + v, EI_T_F32, kEmbd, 1);
    checked_tensor(g, p + "attn_q_norm.weight", EI_T_F32, kHeadDim, 1);
    checked_tensor(g, p + "attn_k_norm.weight", EI_T_F32, kHeadDim, 1);
  }
  const ei_tensor* d2 = checked_tensor(g, "dense_2.weight", EI_T_Q8_0, kEmbd, kDenseFF, false);
  const ei_tensor* d3 = checked_tensor(g, "dense_3.weight", EI_T_Q8_0, kDenseFF, kEmbd, false);
  if ((d2 == nullptr) != (d3 == nullptr)) throw std::runtime_error("dense_2/dense_3 must be both present or absent");
  return n_layer;
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

// One wave in flight: a stream, the workspace of a 2048-token wave, pinned
// staging, and the hipGraphs recorded on them. Several lanes share one
// context's weights, so consecutive waves overlap on the device: one wave's
// latency-bound kernels (row kernels, attention over few sequences) run
// beside another wave's GEMMs.
struct Lane {
  unsigned index = 0;
  hipStream_t stream = nullptr;
  std::mutex mutex;
  float *x, *h, *xd, *cd, *pooled, *mid, *mid_d;
  int8_t *xq, *cq, *mid_q;
  float* qkv;     // [rows][q0 q1 q2 | k | v] after QK-norm / RoPE
  float* scores;  // attention scratch: 1/sum per (token, head), then a score row per (token, head)
  int32_t *ids_d, *pos_d;
  // Attention plan: score and context work items, their two counts, one
  // record per token.
  uint32_t *items_d, *count_d, *tok_d, *off_d;
  // Pinned staging.
  int32_t *ids_h, *pos_h;
  uint32_t *items_h, *count_h, *tok_h, *off_h;
  float* out_h;
  std::map<unsigned, hipGraphExec_t> graphs;  // key: graph_key(padded rows, longest sequence)
  unsigned staged_tokens = 0, staged_rows = 0, staged_longest = 0;
  size_t staged_batch = 0;
  // EG2_HIP_PROFILE (only then non-empty): a pool of events, one recorded
  // before the first launch of an eager forward and one after every
  // launch, the launch names, and the per-name sums in ms.
  std::vector<hipEvent_t> prof_events;
  std::vector<const char*> prof_names;
  std::map<std::string, double> timings;
};

class Backend {
 public:
  explicit Backend(const ei_gguf* g);
  ~Backend();
  // One wave through any free lane: stage, launch, collect. Calls from
  // several threads run on separate lanes at the same time.
  void batch(const int32_t* ids, const size_t* offsets, size_t batch, float* out);
  // The three phases of batch() on one lane, exposed for measurement and
  // pipelining: upload one wave's ids and metadata, enqueue its forward
  // (device-resident, no host copies), and wait + copy the embeddings back.
  // The caller holds the lane's mutex.
  void stage(Lane& L, const int32_t* ids, const size_t* offsets, size_t batch);
  void launch_staged(Lane& L, unsigned repeats);
  void collect(Lane& L, float* out);
  unsigned lanes() const { return (unsigned)lanes_.size(); }
  // The pool of lanes not held by a caller: acquire blocks until one is free.
  unsigned acquire_lane() {
    std::unique_lock<std::mutex> pool(pool_mutex_);
    pool_cv_.wait(pool, [&] { return !free_lanes_.empty(); });
    const unsigned i = free_lanes_.back();
    free_lanes_.pop_back();
    return i;
  }
  // A free lane from the pool, or -1 when every lane is taken (no wait).
  int try_acquire_lane() {
    std::lock_guard<std::mutex> pool(pool_mutex_);
    if (free_lanes_.empty()) return -1;
    const unsigned i = free_lanes_.back();
    free_lanes_.pop_back();
    return (int)i;
  }
  // Takes lane i itself from the pool, blocking until it is free.
  void acquire_lane(unsigned i) {
    if (i >= lanes_.size()) throw std::runtime_error("lane index out of range");
    std::unique_lock<std::mutex> pool(pool_mutex_);
    pool_cv_.wait(pool, [&] { return std::find(free_lanes_.begin(), free_lanes_.end(), i) != free_lanes_.end(); });
    free_lanes_.erase(std::find(free_lanes_.begin(), free_lanes_.end(), i));
  }
  void release_lane(unsigned i) {
    {
      std::lock_guard<std::mutex> pool(pool_mutex_);
      if (i >= lanes_.size() || std::find(free_lanes_.begin(), free_lanes_.end(), i) != free_lanes_.end()) return;
      free_lanes_.push_back(i);
    }
    pool_cv_.notify_one();
  }
  Lane& lane(unsigned i) {
    if (i >= lanes_.size()) throw std::runtime_error("lane index out of range");
    return *lanes_[i];
  }
  // Lane 0 taken from the pool by eg2_kfd_stage and held until
  // eg2_kfd_collect returns it, so that no concurrent batch call stages
  // over the wave in between.
  std::mutex lane0_mutex;
  bool lane0_held = false;
  // Test hook: the next device wait reports a failure as a failing HIP
  // call would, from the host, with no device fault involved.
  std::atomic<bool> inject_failure{false};

 private:
  const ei_gguf* model_;
  std::vector<void*> dev_allocs_;
  std::vector<void*> host_allocs_;
  std::vector<std::unique_ptr<Lane>> lanes_;
  std::mutex pool_mutex_;
  std::condition_variable pool_cv_;
  std::vector<unsigned> free_lanes_;
  // Set by any device-side failure (src/gemma2_kfd.cpp:190-191, 214-215,
  // 270): every later call fails.
  std::atomic<bool> failed_{false};
  bool use_graph_ = true;
  bool profile_ = false;

  float eps_ = 1e-6f;
  std::vector<Layer> layers_;
  const uint8_t* token_embd_ = nullptr;
  const float* output_norm_ = nullptr;
  DevMat dense2_, dense3_;
  bool dense_ = false;
  eg2::AttentionCounts attn_cap_{};

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
  const float* upload_vector(const std::string& name, int n);
  std::vector<uint8_t> q8_rows(const std::string& name, int k, int m) const;
  DevMat upload_q8(const std::vector<const std::vector<uint8_t>*>& parts, int k);
  DevMat upload_q8_geglu(const std::vector<uint8_t>& gate, const std::vector<uint8_t>& up, int k);
  void alloc_lane(Lane& L);
  // Checks a launch's status; while the lane is profiled, also records an
  // event after it on the lane's stream under `name`.
  void launch(Lane& L, const char* name, hipError_t e);
  void record_layers(Lane& L, unsigned rows, unsigned longest);
  void record_head(Lane& L, int batch);
  void gemm(Lane& L, const char* name, const int8_t* xq, const float* xd, const DevMat& w, float* y, int n, int ldy,
            hipStream_t s);
  void wait(Lane& L, const char* what);
  // Runs device work; any exception it throws marks the context failed.
  template <class F>
  void device_step(F&& f) {
    try {
      f();
    } catch (...) {
      failed_ = true;
      throw;
    }
  }
};

const float* Backend::upload_vector(const std::string& name, int n) {
  const ei_tensor* t = checked_tensor(model_, name, EI_T_F32, (uint64_t)n, 1);
  float* d = dalloc<float>(n);
  check(hipMemcpy(d, t->data, n * sizeof(float), hipMemcpyHostToDevice), "upload");
  return d;
}

// Raw Q8_0 rows of a [k, m] (ne[0] = k) matrix, validated (model.c:93-99 with Q8_0).
std::vector<uint8_t> Backend::q8_rows(const std::string& name, int k, int m) const {
  const ei_tensor* t = checked_tensor(model_, name, EI_T_Q8_0, (uint64_t)k, (uint64_t)m);
  const uint8_t* p = static_cast<const uint8_t*>(t->data);
  return std::vector<uint8_t>(p, p + t->n_bytes);
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
  // The whole model is checked before the first device call.
  const uint64_t n_layer = validate_model(g);
  use_graph_ = env_flag("EG2_HIP_GRAPH", true);
  profile_ = env_flag("EG2_HIP_PROFILE", false);
  char why[256];
  if (eg2_hip_device_check(why, sizeof why) != 0)
    throw std::runtime_error(std::string("supported HIP device not found (gfx950): ") + why);

  eps_ = (float)kv_f64(g, "gemma-embedding.attention.layer_norm_rms_epsilon", 1e-6);
  const float base_full = (float)kv_f64(g, "gemma-embedding.rope.freq_base", 1000000.0);
  const float base_swa = (float)kv_f64(g, "gemma-embedding.rope.freq_base_swa", 10000.0);
  const uint64_t swa_window = kv_u64(g, "gemma-embedding.attention.sliding_window", 512);
  const uint64_t swa_period = kv_u64(g, "gemma-embedding.attention.sliding_window_pattern", 6);

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

  const ei_tensor* emb = checked_tensor(g, "token_embd.weight", EI_T_Q8_0, kEmbd, kVocab);
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
  if (find_tensor(g, "dense_2.weight")) {
    auto a = q8_rows("dense_2.weight", kEmbd, kDenseFF), b = q8_rows("dense_3.weight", kDenseFF, kEmbd);
    dense2_ = upload_q8({&a}, kEmbd);
    dense3_ = upload_q8({&b}, kDenseFF);
    dense_ = true;
  }

  // Capacity for the wave cap plus the padding sequence (rows rounded to 32).
  attn_cap_ = eg2::attention_capacity(kCap + 32, kCap + 1);
  // EG2_HIP_LANES (1..8): waves in flight per context, 4 by default (more
  // lanes measured slower). Each lane's stream has a hardware queue of its
  // own whatever GPU_MAX_HW_QUEUES says (alloc_lane).
  unsigned n_lanes = 4;
  if (const char* v = std::getenv("EG2_HIP_LANES")) {
    char* end = nullptr;
    const long l = std::strtol(v, &end, 10);
    if (!*v || *end || l < 1 || l > 8) throw std::runtime_error("EG2_HIP_LANES must be 1..8");
    n_lanes = (unsigned)l;
  }
  for (unsigned i = 0; i < n_lanes; ++i) {
    lanes_.push_back(std::make_unique<Lane>());
    lanes_.back()->index = i;
    alloc_lane(*lanes_.back());
    free_lanes_.push_back(n_lanes - 1 - i);  // lane 0 is taken first
  }
  check(hipDeviceSynchronize(), "upload");

  size_t bytes = 0;
  for (auto& L : layers_)
    for (const DevMat* w : {&L.qkv, &L.o, &L.gu, &L.down})
      bytes += eg2_q8_tile_bytes(w->m, w->k) + (size_t)(w->k / 32) * w->ld * sizeof(float);
  std::fprintf(stderr, "HIP: gfx950, %zu layers, Q8_0 layer weights %.1f MiB (int8 row tiles + scales), embedding table %.1f MiB, cap %u packed tokens%s\n",
               layers_.size(), bytes / 1048576.0, emb->n_bytes / 1048576.0, kCap, dense_ ? ", dense head" : "");
}

void Backend::alloc_lane(Lane& L) {
  // The lane's stream, created with a CU mask that enables every CU: the
  // HIP runtime gives a stream with a CU mask a hardware queue of its own
  // instead of sharing one of its GPU_MAX_HW_QUEUES queues (4 unless set)
  // with other streams, which would serialise the lanes' kernels. Four
  // lanes under the default 4 queues ran like four on 8 queues (1.32 ms
  // per wave, against 1.59 with shared queues and 1.39 for three lanes).
  // Such a stream synchronises with the null stream (it has no non-blocking
  // flag); the lanes' work never uses the null stream.
  int dev = 0, ncu = 0;
  check(hipGetDevice(&dev), "hipGetDevice");
  check(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev), "CU count");
  if (ncu <= 0) throw std::runtime_error("device reports no compute units");
  std::vector<uint32_t> mask((size_t)(ncu + 31) / 32, 0u);
  for (int c = 0; c < ncu; ++c) mask[(size_t)c / 32] |= 1u << (c % 32);
  check(hipExtStreamCreateWithCUMask(&L.stream, (uint32_t)mask.size(), mask.data()), "hipExtStreamCreateWithCUMask");
  L.x = dalloc<float>((size_t)kCap * kEmbd);
  L.h = dalloc<float>((size_t)kCap * kEmbd);
  L.xq = dalloc<int8_t>(eg2_q8_tile_bytes(kCap, kFF));
  L.xd = dalloc<float>((size_t)kCap * (kFF / 32));
  L.cq = dalloc<int8_t>(eg2_q8_tile_bytes(kCap, kEmbd));
  L.cd = dalloc<float>((size_t)kCap * (kEmbd / 32));
  L.qkv = dalloc<float>((size_t)kCap * kQKV);
  L.scores = dalloc<float>(attn_cap_.score_floats);
  L.ids_d = dalloc<int32_t>(kCap);
  L.pos_d = dalloc<int32_t>(kCap);
  L.items_d = dalloc<uint32_t>(8 * attn_cap_.items);
  L.count_d = dalloc<uint32_t>(2);
  L.tok_d = dalloc<uint32_t>(4 * (size_t)kCap);
  L.off_d = dalloc<uint32_t>(kCap + 1);
  L.pooled = dalloc<float>((size_t)kCap * kEmbd);
  L.mid = dalloc<float>((size_t)kCap * kDenseFF);
  L.mid_q = dalloc<int8_t>(eg2_q8_tile_bytes(kCap, kDenseFF));
  L.mid_d = dalloc<float>((size_t)kCap * (kDenseFF / 32));
  L.ids_h = halloc<int32_t>(kCap);
  L.pos_h = halloc<int32_t>(kCap);
  L.items_h = halloc<uint32_t>(8 * attn_cap_.items);
  L.count_h = halloc<uint32_t>(2);
  L.tok_h = halloc<uint32_t>(4 * (size_t)kCap);
  L.off_h = halloc<uint32_t>(kCap + 1);
  L.out_h = halloc<float>((size_t)kCap * kEmbd);
}

Backend::~Backend() {
  for (auto& L : lanes_) {
    if (L->stream) (void)hipStreamSynchronize(L->stream);
    for (hipEvent_t ev : L->prof_events) (void)hipEventDestroy(ev);
    for (auto& kvp : L->graphs) (void)hipGraphExecDestroy(kvp.second);
    if (L->stream) (void)hipStreamDestroy(L->stream);
  }
  for (void* p : dev_allocs_) (void)hipFree(p);
  for (void* p : host_allocs_) (void)hipHostFree(p);
}

void Backend::launch(Lane& ln, const char* name, hipError_t e) {
  if (e != hipSuccess) throw std::runtime_error(std::string(name) + ": " + hipGetErrorString(e));
  if (ln.prof_events.empty()) return;  // not profiled
  const size_t i = ln.prof_names.size();
  if (i + 1 >= ln.prof_events.size()) throw std::runtime_error("profile event pool exhausted");
  check(hipEventRecord(ln.prof_events[i + 1], ln.stream), "hipEventRecord");
  ln.prof_names.push_back(name);
}

// y[n][w.m] (row stride ldy) = activations (row tiles xq, scales xd
// [k/32][n]) times the weights w.
void Backend::gemm(Lane& ln, const char* name, const int8_t* xq, const float* xd, const DevMat& w, float* y, int n,
                   int ldy, hipStream_t s) {
  launch(ln, name, eg2::launch_gemm_q8(xq, xd, n, w.q, w.d, w.ld, y, n, w.m, w.k, ldy, s));
}

// The per-wave layer stack for `rows` (padded) token rows: embedding + norm,
// then per layer (engine.c:1115-1127 order) QKV GEMM with QK-norm/RoPE,
// attention (scores, then the context and its Q8_0), O GEMM, residual +
// ffn_norm (+Q8_0), gate|up GEMM with the GeGLU (+Q8_0) in its epilogue,
// down GEMM, residual + next attn_norm (+Q8_0); finally the output_norm per
// token (the first half of kernels.c:417-427).
void Backend::record_layers(Lane& ln, unsigned rows, unsigned longest) {
  hipStream_t s = ln.stream;
  const int n = (int)rows;
  launch(ln, "embed", eg2::launch_embed_norm_quant(token_embd_, ln.ids_d, n, std::sqrt((float)kEmbd),
                                                   layers_[0].attn_norm, eps_, ln.x, ln.xq, ln.xd, s));
  for (size_t il = 0; il < layers_.size(); ++il) {
    const Layer& L = layers_[il];
    // Q|K|V projection with QK-norm / RoPE in its epilogue: the attention
    // operand rows, no unnormalised projection in HBM.
    launch(ln, "gemm_qkv_rope", eg2::launch_gemm_q8_qkv_rope(ln.xq, ln.xd, n, L.qkv.q, L.qkv.d, L.qkv.ld, n, kEmbd,
                                                             L.q_norm, L.k_norm, L.rope, ln.pos_d, eps_, ln.qkv, s));
    launch(ln, "attention_scores", eg2::launch_attention_scores(ln.qkv, ln.items_d, ln.count_d, eg2::kAttentionGrid,
                                                                L.window, n, ln.scores, s));
    launch(ln, "attention_softmax", eg2::launch_attention_softmax(ln.tok_d, L.window, n, (int)longest, ln.scores, s));
    launch(ln, "attention_context", eg2::launch_attention_context(ln.qkv, ln.items_d, ln.count_d, eg2::kAttentionGrid,
                                                                  L.window, n, ln.scores, ln.cq, ln.cd, s));
    gemm(ln, "gemm_o", ln.cq, ln.cd, L.o, ln.h, n, kEmbd, s);
    // The FFN input goes to the attention context's buffers (free after the
    // O GEMM), so the fused gate|up + GeGLU kernel reads them and writes xq.
    launch(ln, "residual",
           eg2::launch_residual_norm_quant(ln.x, ln.h, L.post_attn, L.ffn_norm, eps_, ln.cq, ln.cd, n, s));
    launch(ln, "gemm_gate_up_geglu", eg2::launch_gemm_q8_geglu(ln.cq, ln.cd, n, L.gu.q, L.gu.d, L.gu.ld, ln.xq,
                                                                ln.xd, n, n, kFF, kEmbd, s));
    gemm(ln, "gemm_down", ln.xq, ln.xd, L.down, ln.h, n, kEmbd, s);
    const float* next = il + 1 < layers_.size() ? layers_[il + 1].attn_norm : nullptr;
    launch(ln, "residual", eg2::launch_residual_norm_quant(ln.x, ln.h, L.post_ffw, next, eps_, ln.xq, ln.xd, n, s));
  }
  launch(ln, "output_norm", eg2::launch_rms_norm_rows(ln.x, output_norm_, eps_, n, s));
}

// kernels.c:417-427 (mean + L2 per sequence) and the dense head.
void Backend::record_head(Lane& ln, int B) {
  hipStream_t s = ln.stream;
  if (dense_) {
    // EXTRACTION.md:178-181: dense_2 then dense_3 on the mean pool
    // (kernels.c:417-425 without its L2), each input Q8_0-quantized,
    // then the L2 of kernels.c:393-396.
    launch(ln, "pool", eg2::launch_pool_mean(ln.x, ln.off_d, ln.pooled, B, s));
    launch(ln, "dense_quant", eg2::launch_quantize_rows(ln.pooled, kEmbd, ln.cq, ln.cd, B, s));
    gemm(ln, "dense_2", ln.cq, ln.cd, dense2_, ln.mid, B, kDenseFF, s);
    launch(ln, "dense_quant", eg2::launch_quantize_rows(ln.mid, kDenseFF, ln.mid_q, ln.mid_d, B, s));
    gemm(ln, "dense_3", ln.mid_q, ln.mid_d, dense3_, ln.pooled, B, kEmbd, s);
    launch(ln, "dense_l2", eg2::launch_l2_prefix(ln.pooled, kEmbd, kEmbd, B, s));
  } else if (ln.staged_longest > kPoolSplitLen) {
    // One workgroup per sequence reads it through one CU; past 256
    // tokens the mean spreads over 12 workgroups per sequence and the
    // L2 follows (the same result, bit for bit).
    launch(ln, "pool", eg2::launch_pool_mean(ln.x, ln.off_d, ln.pooled, B, s));
    launch(ln, "pool_l2", eg2::launch_l2_prefix(ln.pooled, kEmbd, kEmbd, B, s));
  } else {
    launch(ln, "pool", eg2::launch_pool_l2(ln.x, ln.off_d, ln.pooled, B, s));
  }
}

void Backend::wait(Lane& ln, const char* what) {
  const auto start = std::chrono::steady_clock::now();
  if (inject_failure.exchange(false)) throw std::runtime_error(std::string(what) + ": injected HIP failure");
  for (;;) {
    const hipError_t e = hipStreamQuery(ln.stream);
    if (e == hipSuccess) return;
    if (e != hipErrorNotReady) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
    if (std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count() > kTimeoutSeconds)
      throw std::runtime_error(std::string(what) + ": timed out");
    std::this_thread::yield();
  }
}

void Backend::batch(const int32_t* ids, const size_t* offsets, size_t batch, float* out) {
  const unsigned idx = acquire_lane();
  struct Release {
    Backend* b;
    unsigned i;
    ~Release() { b->release_lane(i); }
  } release{this, idx};
  Lane& ln = *lanes_[idx];
  std::lock_guard<std::mutex> guard(ln.mutex);
  const auto t0 = std::chrono::steady_clock::now();
  stage(ln, ids, offsets, batch);
  launch_staged(ln, 1);
  collect(ln, out);
  if (profile_) {
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    // src/gemma2_kfd.cpp:346-352's KFD_PROFILE line: per launch name, the
    // summed GPU time of its launches (names in sorted order).
    std::string line = "HIP_PROFILE {\"tokens\":" + std::to_string(ln.staged_tokens) +
                       ",\"batch\":" + std::to_string(ln.staged_batch) + ",\"wall_ms\":" + fixed3(ms) +
                       ",\"command_ms\":{";
    bool first = true;
    for (const auto& kv : ln.timings) {
      line += (first ? "\"" : ",\"") + kv.first + "\":" + fixed3(kv.second);
      first = false;
    }
    line += "}}\n";
    std::fputs(line.c_str(), stderr);
    ln.timings.clear();
  }
}

void Backend::stage(Lane& ln, const int32_t* ids, const size_t* offsets, size_t batch) {
  if (failed_) throw std::runtime_error("HIP context failed; restart process before reuse");
  ln.staged_batch = 0;
  // src/gemma2_kfd.cpp:271-278
  if (!ids || !offsets || !batch || batch > kCap || offsets[0] || offsets[batch] > kCap)
    throw std::runtime_error("HIP batch requires 1..2048 packed tokens and nonempty sequences");
  unsigned longest = 0;
  for (size_t s = 0; s < batch; ++s) {
    if (offsets[s + 1] <= offsets[s]) throw std::runtime_error("invalid HIP sequence offsets");
    longest = std::max(longest, (unsigned)(offsets[s + 1] - offsets[s]));
  }
  const unsigned n = (unsigned)offsets[batch];
  for (unsigned i = 0; i < n; ++i)
    if (ids[i] < 0 || ids[i] >= kVocab) throw std::runtime_error("token ID out of range");
  // The lane's pinned staging may still feed its previous wave's copies.
  device_step([&] { wait(ln, "HIP previous wave"); });

  // Metadata; rows [n, rows) form one dummy sequence that is never pooled.
  const unsigned rows = (n + 31) / 32 * 32;
  for (size_t s = 0; s < batch; ++s)
    for (size_t t = offsets[s]; t < offsets[s + 1]; ++t) {
      ln.ids_h[t] = ids[t];
      ln.pos_h[t] = (int32_t)(t - offsets[s]);
    }
  for (unsigned t = n; t < rows; ++t) {
    ln.ids_h[t] = 0;
    ln.pos_h[t] = (int32_t)(t - n);
  }
  for (size_t s = 0; s <= batch; ++s) ln.off_h[s] = (uint32_t)offsets[s];
  // The attention plan; the padding rows form one more sequence. Its counts
  // are checked against the allocation before anything is written.
  std::vector<size_t> all(offsets, offsets + batch + 1);
  if (rows > n) all.push_back(rows);
  eg2::AttentionCounts used{0, 0, 0};
  if (!eg2::build_attention_plan(all.data(), all.size() - 1, attn_cap_, ln.items_h, ln.tok_h, &used))
    throw std::runtime_error("attention work list exceeds its capacity");
  ln.count_h[0] = (uint32_t)used.score_items;
  ln.count_h[1] = (uint32_t)(used.items - used.score_items);

  device_step([&] {
    hipStream_t s = ln.stream;
    check(hipMemcpyAsync(ln.ids_d, ln.ids_h, rows * sizeof(int32_t), hipMemcpyHostToDevice, s), "copy ids");
    check(hipMemcpyAsync(ln.pos_d, ln.pos_h, rows * sizeof(int32_t), hipMemcpyHostToDevice, s), "copy positions");
    check(hipMemcpyAsync(ln.items_d, ln.items_h, 8 * used.items * sizeof(uint32_t), hipMemcpyHostToDevice, s),
          "copy attention items");
    check(hipMemcpyAsync(ln.count_d, ln.count_h, 2 * sizeof(uint32_t), hipMemcpyHostToDevice, s),
          "copy attention counts");
    check(hipMemcpyAsync(ln.tok_d, ln.tok_h, 4 * (size_t)rows * sizeof(uint32_t), hipMemcpyHostToDevice, s),
          "copy token records");
    check(hipMemcpyAsync(ln.off_d, ln.off_h, (batch + 1) * sizeof(uint32_t), hipMemcpyHostToDevice, s),
          "copy offsets");
    const unsigned key = graph_key(rows, longest);
    if (use_graph_ && !profile_ && ln.graphs.find(key) == ln.graphs.end()) {
      hipGraph_t graph = nullptr;
      check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
      try {
        record_layers(ln, rows, attention_form(longest));
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
      ln.graphs.emplace(key, exec);
    }
  });
  ln.staged_tokens = n;
  ln.staged_rows = rows;
  ln.staged_batch = batch;
  ln.staged_longest = longest;
}

// Layer stack (graph or eager), then kernels.c:417-427 (mean + L2 per
// sequence) and the dense head.
void Backend::launch_staged(Lane& ln, unsigned repeats) {
  if (failed_) throw std::runtime_error("HIP context failed; restart process before reuse");
  if (!ln.staged_batch) throw std::runtime_error("no staged wave");
  hipStream_t s = ln.stream;
  const int B = (int)ln.staged_batch;
  device_step([&] {
    for (unsigned r = 0; r < repeats; ++r) {
      if (profile_) {
        // Per-kernel timing (the reference's KFD_PROFILE, src/gemma2_kfd.cpp:
        // 173-186, 216-222): an eager forward with an event after every
        // launch, each kernel's time (from the previous event to its own)
        // summed per launch name.
        if (ln.prof_events.empty()) {
          ln.prof_events.resize(1024);
          for (auto& ev : ln.prof_events) check(hipEventCreate(&ev), "hipEventCreate");
        }
        ln.prof_names.clear();
        check(hipEventRecord(ln.prof_events[0], s), "hipEventRecord");
        record_layers(ln, ln.staged_rows, attention_form(ln.staged_longest));
        record_head(ln, B);
        const size_t k = ln.prof_names.size();
        check(hipEventSynchronize(ln.prof_events[k]), "hipEventSynchronize");
        for (size_t i = 0; i < k; ++i) {
          float ms = 0;
          check(hipEventElapsedTime(&ms, ln.prof_events[i], ln.prof_events[i + 1]), "hipEventElapsedTime");
          ln.timings[ln.prof_names[i]] += ms;
        }
        ln.prof_names.clear();
      } else if (use_graph_) {
        check(hipGraphLaunch(ln.graphs.at(graph_key(ln.staged_rows, ln.staged_longest)), s), "hipGraphLaunch");
        record_head(ln, B);
      } else {
        record_layers(ln, ln.staged_rows, attention_form(ln.staged_longest));
        record_head(ln, B);
      }
    }
  });
}

void Backend::collect(Lane& ln, float* out) {
  if (failed_) throw std::runtime_error("HIP context failed; restart process before reuse");
  if (!ln.staged_batch) throw std::runtime_error("no staged wave");
  if (!out) throw std::runtime_error("null output");
  const int B = (int)ln.staged_batch;
  device_step([&] {
    check(hipMemcpyAsync(ln.out_h, ln.pooled, (size_t)B * kEmbd * sizeof(float), hipMemcpyDeviceToHost, ln.stream),
          "copy out");
    wait(ln, "HIP wave");
  });

  // src/gemma2_kfd.cpp:337-343 rejects non-finite or zero embeddings.
  for (int r = 0; r < B; ++r) {
    double ss = 0;
    for (int z = 0; z < kEmbd; ++z) {
      const float f = ln.out_h[(size_t)r * kEmbd + z];
      if (!std::isfinite(f)) throw std::runtime_error("nonfinite GPU output");
      ss += (double)f * f;
    }
    if (ss <= 0) throw std::runtime_error("zero GPU embedding");
  }
  std::memcpy(out, ln.out_h, (size_t)B * kEmbd * sizeof(float));
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

namespace {
// Runs f on lane `lane` of ctx with the lane held; exceptions become
// "HIP: ..." messages.
template <class F>
bool on_lane(void* ctx, unsigned lane, char* err, size_t len, F&& f) {
  try {
    if (!ctx) throw std::runtime_error("empty context");
    Backend* b = static_cast<Backend*>(ctx);
    Lane& ln = b->lane(lane);
    std::lock_guard<std::mutex> guard(ln.mutex);
    f(*b, ln);
    return true;
  } catch (const std::exception& e) {
    if (err && len) std::snprintf(err, len, "HIP: %s", e.what());
    return false;
  }
}
}  // namespace

extern "C" unsigned eg2_kfd_lanes(void* ctx) { return ctx ? static_cast<Backend*>(ctx)->lanes() : 0; }

extern "C" int eg2_kfd_acquire_lane(void* ctx) { return ctx ? (int)static_cast<Backend*>(ctx)->acquire_lane() : -1; }

extern "C" int eg2_kfd_try_acquire_lane(void* ctx) {
  return ctx ? static_cast<Backend*>(ctx)->try_acquire_lane() : -1;
}

extern "C" void eg2_kfd_release_lane(void* ctx, unsigned lane) {
  if (ctx) static_cast<Backend*>(ctx)->release_lane(lane);
}

extern "C" bool eg2_kfd_stage_lane(void* ctx, unsigned lane, const int32_t* ids, const size_t* offsets, size_t batch,
                                   char* err, size_t len) {
  return on_lane(ctx, lane, err, len, [&](Backend& b, Lane& ln) { b.stage(ln, ids, offsets, batch); });
}

extern "C" bool eg2_kfd_launch_lane(void* ctx, unsigned lane, unsigned repeats, char* err, size_t len) {
  return on_lane(ctx, lane, err, len, [&](Backend& b, Lane& ln) { b.launch_staged(ln, repeats); });
}

extern "C" bool eg2_kfd_collect_lane(void* ctx, unsigned lane, float* out, char* err, size_t len) {
  return on_lane(ctx, lane, err, len, [&](Backend& b, Lane& ln) { b.collect(ln, out); });
}

extern "C" int eg2_kfd_lane_ready(void* ctx, unsigned lane, char* err, size_t len) {
  int ready = -1;
  const bool ok = on_lane(ctx, lane, err, len, [&](Backend&, Lane& ln) {
    const hipError_t e = hipStreamQuery(ln.stream);
    if (e != hipSuccess && e != hipErrorNotReady) throw std::runtime_error(std::string("HIP lane query: ") + hipGetErrorString(e));
    ready = e == hipSuccess ? 1 : 0;
  });
  return ok ? ready : -1;
}

// Lane 0 through the pool: eg2_kfd_stage takes it (unless a wave staged
// by it is still uncollected) and keeps it after a successful stage;
// eg2_kfd_collect gives it back.
extern "C" bool eg2_kfd_stage(void* ctx, const int32_t* ids, const size_t* offsets, size_t batch, char* err,
                              size_t len) {
  if (!ctx) return eg2_kfd_stage_lane(ctx, 0, ids, offsets, batch, err, len);
  Backend* b = static_cast<Backend*>(ctx);
  std::lock_guard<std::mutex> g(b->lane0_mutex);
  const bool took = !b->lane0_held;
  if (took) b->acquire_lane(0u);
  const bool ok = eg2_kfd_stage_lane(ctx, 0, ids, offsets, batch, err, len);
  if (ok) {
    b->lane0_held = true;
  } else if (took) {
    b->release_lane(0);
  }
  return ok;
}

extern "C" bool eg2_kfd_launch_staged(void* ctx, unsigned repeats, char* err, size_t len) {
  if (ctx) {
    Backend* b = static_cast<Backend*>(ctx);
    std::lock_guard<std::mutex> g(b->lane0_mutex);
    if (!b->lane0_held) {
      if (err && len) std::snprintf(err, len, "HIP: no staged wave (eg2_kfd_stage first)");
      return false;
    }
  }
  return eg2_kfd_launch_lane(ctx, 0, repeats, err, len);
}

extern "C" bool eg2_kfd_collect(void* ctx, float* out, char* err, size_t len) {
  if (!ctx) return eg2_kfd_collect_lane(ctx, 0, out, err, len);
  Backend* b = static_cast<Backend*>(ctx);
  std::lock_guard<std::mutex> g(b->lane0_mutex);
  if (!b->lane0_held) {
    if (err && len) std::snprintf(err, len, "HIP: no staged wave (eg2_kfd_stage first)");
    return false;
  }
  const bool ok = eg2_kfd_collect_lane(ctx, 0, out, err, len);
  b->lane0_held = false;
  b->release_lane(0);
  return ok;
}

extern "C" void eg2_kfd_inject_failure(void* ctx) {
  if (ctx) static_cast<Backend*>(ctx)->inject_failure = true;
}

extern "C" bool eg2_kfd_validate_gguf(const ei_gguf* g, char* err, size_t len) {
  try {
    validate_model(g);
    return true;
  } catch (const std::exception& e) {
    if (err && len) std::snprintf(err, len, "HIP: %s", e.what());
    return false;
  }
}
