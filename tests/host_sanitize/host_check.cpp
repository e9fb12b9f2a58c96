// Host-side checks of libeg2hip's host code and of the CPU oracle, built
// with AddressSanitizer + UndefinedBehaviorSanitizer (make asan) or with
// ThreadSanitizer (make tsan). No GPU call is made: the executor's model
// validation, the attention plan builder, the Q8_0 repacking, the wave
// packer, the float-text / base64 / response formatting, the tokenizer
// (single and threaded batch forms), the GGUF reader and the threaded
// synthetic-model writer run here, together with the oracle's threaded
// GEMM and one encoder layer, so that a heap overflow, use after free,
// undefined operation or data race in any of them ends the run with a
// sanitizer report.
//
//   host_check <workdir>
// workdir holds tok.gguf (a tokenizer vocabulary) and texts.bin (u64 n,
// u64 offsets[n + 1], the text bytes); ids.bin (u64 n, u64 offsets[n + 1],
// int32 ids) is written back for the caller to compare with the reference
// ids. Prints "host checks passed" and exits 0 when every check holds.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "eg2_format.h"
#include "eg2_hip.h"
#include "eg2_stream.h"
#include "eg2_tokenizer.h"
#include "gguf.h"
#include "oracle.h"

namespace {

int failures = 0;

void check(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "FAILED: %s\n", what);
    ++failures;
  }
}

std::vector<uint8_t> read_file(const std::string& path) {
  std::vector<uint8_t> buf;
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) return buf;
  std::fseek(f, 0, SEEK_END);
  buf.resize((size_t)std::ftell(f));
  std::fseek(f, 0, SEEK_SET);
  if (std::fread(buf.data(), 1, buf.size(), f) != buf.size()) buf.clear();
  std::fclose(f);
  return buf;
}

const ei_tensor* tensor(const ei_gguf& g, const char* name) {
  for (uint64_t i = 0; i < g.n_tensors; ++i)
    if (g.tensors[i].name.len == std::strlen(name) && !std::memcmp(g.tensors[i].name.str, name, g.tensors[i].name.len))
      return &g.tensors[i];
  return nullptr;
}

// The synthetic model: written with 4 threads, read back, validated, then
// validated again with corrupted tensor records (each must be rejected
// with a message naming the tensor).
void check_model(const std::string& dir, ei_gguf& g) {
  eg2_synth_config cfg{};
  cfg.seed = 7;
  cfg.n_layer = 1;
  cfg.dense_head = 1;
  cfg.weight_std = 0.02f;
  cfg.embed_std = 0.02f;
  cfg.norm_std = 0.1f;
  cfg.rope_base_full = 1e6f;
  cfg.rope_base_swa = 1e4f;
  cfg.sliding_window = 512;
  cfg.sliding_window_pattern = 6;
  cfg.threads = 4;
  char err[256] = {0};
  const std::string path = dir + "/model.gguf";
  check(eg2_synth_write_gguf(path.c_str(), &cfg, err, sizeof err) == 0, "synthetic model written");
  check(eg2_gguf_open(path.c_str(), &g, err, sizeof err) == 0, "synthetic model parsed");
  check(eg2_kfd_validate_gguf(&g, err, sizeof err), "synthetic model validates");

  ei_tensor* emb = const_cast<ei_tensor*>(tensor(g, "token_embd.weight"));
  ei_tensor* norm = const_cast<ei_tensor*>(tensor(g, "blk.0.attn_norm.weight"));
  check(emb && norm, "tensors present");
  if (!emb || !norm) return;
  const ei_tensor e0 = *emb, n0 = *norm;
  emb->n_dims = 3;
  emb->ne[2] = 0;
  emb->n_bytes = 0;
  check(!eg2_kfd_validate_gguf(&g, err, sizeof err) && std::strstr(err, "token_embd.weight"),
        "a zero-sized 3-d token_embd is rejected");
  *emb = e0;
  norm->n_bytes -= 4;
  check(!eg2_kfd_validate_gguf(&g, err, sizeof err) && std::strstr(err, "attn_norm"),
        "a short norm vector is rejected");
  *norm = n0;
  check(eg2_kfd_validate_gguf(&g, err, sizeof err), "restored records validate");

  // A file cut short must be refused by the reader, not read past its end.
  const std::vector<uint8_t> whole = read_file(path);
  for (size_t cut : {size_t(3), size_t(40), whole.size() / 2, whole.size() - 1}) {
    const std::string part = dir + "/cut.gguf";
    FILE* f = std::fopen(part.c_str(), "wb");
    std::fwrite(whole.data(), 1, cut, f);
    std::fclose(f);
    ei_gguf bad{};
    check(eg2_gguf_open(part.c_str(), &bad, err, sizeof err) != 0, "truncated file refused");
  }
}

// The attention plan for random packings: exact-size buffers (so that any
// write past the counts the planner reports is a heap overflow), every
// token record inside its sequence, and the capacity bound respected.
void check_attention_plan(std::mt19937_64& rng) {
  size_t cap[2];
  eg2_attention_capacity(2048 + 32, 2049, cap);
  for (int it = 0; it < 60; ++it) {
    std::vector<size_t> offsets{0};
    const size_t total = 1 + rng() % 2048;
    while (offsets.back() < total) offsets.push_back(std::min(total, offsets.back() + 1 + rng() % (it % 3 ? 300 : 2048)));
    const size_t batch = offsets.size() - 1;
    // A call with no capacity writes nothing and reports the counts.
    size_t counts[3];
    uint32_t none[1] = {0};
    check(eg2_attention_plan(offsets.data(), batch, 0, 0, none, none, counts) == -1, "plan sizes query");
    check(counts[0] <= cap[0] && counts[1] <= cap[1], "plan within the capacity bound");
    std::vector<uint32_t> items(8 * counts[0]), tok(4 * offsets.back());
    size_t got[3];
    check(eg2_attention_plan(offsets.data(), batch, counts[0], counts[1], items.data(), tok.data(), got) == 0,
          "plan written");
    check(got[0] == counts[0] && got[1] == counts[1] && got[2] == counts[2], "plan counts stable");
    for (size_t s = 0; s < batch; ++s)
      for (size_t t = offsets[s]; t < offsets[s + 1]; ++t)
        check(tok[4 * t] == offsets[s] && tok[4 * t + 1] == offsets[s + 1], "token record in its sequence");
  }
}

// Q8_0 repacking into row tiles: every value lands at q8_tile_offset and the
// padding stays zero.
void check_tiles(std::mt19937_64& rng) {
  const size_t rows = 45;
  const unsigned k = 96;
  std::vector<int8_t> q(rows * k);
  for (auto& v : q) v = (int8_t)(rng() % 255 - 127);
  std::vector<int8_t> tiles(eg2_q8_tile_bytes(rows, k), 99);
  eg2_q8_pack_rows(q.data(), rows, k, tiles.data());
  size_t nonzero = 0;
  for (int8_t v : tiles) nonzero += v != 0;
  size_t want = 0;
  for (int8_t v : q) want += v != 0;
  check(nonzero == want, "row tiles hold the values and zero padding");
  std::vector<uint8_t> blocks(rows * (k / 32) * 34);
  for (size_t i = 0; i < blocks.size(); ++i) blocks[i] = (uint8_t)rng();
  for (size_t b = 0; b < rows * (k / 32); ++b) {  // finite fp16 scales
    blocks[34 * b] = (uint8_t)(rng() & 0xff);
    blocks[34 * b + 1] = (uint8_t)(0x20 + rng() % 0x20);
  }
  std::vector<int8_t> wq(eg2_q8_tile_bytes(rows, k));
  std::vector<float> wd((k / 32) * ((rows + 31) / 32 * 32));
  eg2_q8_weight_tiles(blocks.data(), rows, k, wq.data(), wd.data());
  check(std::isfinite(wd[0]), "weight scales converted");
}

void check_packer(std::mt19937_64& rng) {
  eg2_batch_config cfg;
  eg2_batch_config_default(&cfg);
  for (int it = 0; it < 40; ++it) {
    const size_t n = 1 + rng() % 500;
    std::vector<size_t> len(n), order(n), wave_end(n);
    for (auto& l : len) l = 1 + (size_t)std::floor(std::exp(std::log(4.0) + (std::log(2048.0) - std::log(4.0)) *
                                                                              (double)(rng() % 1000000) / 1e6));
    cfg.lookahead = it % 2;
    const size_t waves = eg2_pack_waves(len.data(), n, &cfg, order.data(), wave_end.data());
    check(waves > 0 && wave_end[waves - 1] == n, "every sequence placed");
    std::vector<int> seen(n, 0);
    for (size_t i = 0; i < n; ++i) seen[order[i]]++;
    bool once = true;
    for (int s : seen) once = once && s == 1;
    check(once, "each sequence in exactly one wave");
  }
  std::vector<float> e(768);
  for (auto& v : e) v = (float)((double)(rng() % 2000000) / 1e6 - 1.0);
  check(eg2_normalize_prefix(e.data(), 128) && !eg2_normalize_prefix(e.data(), 100), "prefix normalisation");
}

void check_format(std::mt19937_64& rng) {
  char buf[EG2_F32_CHARS + 1];
  for (int i = 0; i < 200000; ++i) {
    const uint32_t bits = (uint32_t)rng();
    float f;
    std::memcpy(&f, &bits, 4);
    const size_t n = eg2_f32_to_chars(buf, f);
    if (!std::isfinite(f)) {
      check(n == 0, "no text for a non-finite value");
      continue;
    }
    check(n > 0 && n <= EG2_F32_CHARS, "float text length");
    buf[n] = 0;
    if (std::strtof(buf, nullptr) != f && !(f == 0.0f)) {
      check(false, "float text reads back");
      break;
    }
  }
  std::vector<float> v(768 * 3);
  for (auto& x : v) x = (float)((double)(rng() % 2000000) / 1e6 - 1.0);
  std::vector<char> b64((v.size() * 4 + 2) / 3 * 4);
  check(eg2_base64_f32(v.data(), v.size(), b64.data()) == b64.size(), "base64 length");
  for (unsigned dims : {128u, 768u})
    for (int api = 0; api < 2; ++api)
      for (int enc = 0; enc < 2; ++enc) {
        const size_t bound = eg2_embeddings_response_bound(3, dims, 9);
        std::vector<char> out(bound);
        std::vector<float> emb(v);
        const size_t n = eg2_embeddings_response(emb.data(), 3, dims, (eg2_embedding_api)api,
                                                 (eg2_embedding_encoding)enc, "model-x.q", 9, 1234, out.data(),
                                                 out.size());
        check(n > 0 && n <= bound, "response body within its bound");
      }
}

void check_tokenizer(const std::string& dir) {
  ei_gguf g{};
  char err[256] = {0};
  check(eg2_gguf_open((dir + "/tok.gguf").c_str(), &g, err, sizeof err) == 0, "tokenizer file parsed");
  eg2_tokenizer* tok = eg2_tokenizer_create(&g, err, sizeof err);
  check(tok != nullptr, "tokenizer created");
  if (!tok) return;
  const std::vector<uint8_t> raw = read_file(dir + "/texts.bin");
  uint64_t n = 0;
  std::memcpy(&n, raw.data(), 8);
  std::vector<size_t> offs(n + 1);
  for (uint64_t i = 0; i <= n; ++i) {
    uint64_t o;
    std::memcpy(&o, raw.data() + 8 + 8 * i, 8);
    offs[i] = (size_t)o;
  }
  const char* texts = reinterpret_cast<const char*>(raw.data() + 8 + 8 * (n + 1));
  // An exact-size id buffer (the single-text form counts without writing
  // when cap is 0): the batch form must not write past cap, and must refuse
  // a buffer one id short.
  size_t need = 0;
  for (uint64_t i = 0; i < n; ++i) need += eg2_tokenize(tok, texts + offs[i], offs[i + 1] - offs[i], true, true, nullptr, 0);
  std::vector<int32_t> ids(need);
  std::vector<size_t> id_offs(n + 1);
  check(eg2_tokenize_batch(tok, texts, offs.data(), n, true, true, ids.data(), ids.size(), id_offs.data(), 4) == need,
        "threaded batch tokenization");
  std::vector<size_t> short_offs(n + 1);
  check(eg2_tokenize_batch(tok, texts, offs.data(), n, true, true, ids.data(), need - 1, short_offs.data(), 4) ==
            SIZE_MAX,
        "a short id buffer is refused");
  // The single-text form agrees with the batch form.
  std::vector<int32_t> one(4096);
  bool same = true;
  for (uint64_t i = 0; i < n && same; ++i) {
    const size_t k = eg2_tokenize(tok, texts + offs[i], offs[i + 1] - offs[i], true, true, one.data(), one.size());
    same = k == id_offs[i + 1] - id_offs[i] && !std::memcmp(one.data(), ids.data() + id_offs[i], k * 4);
  }
  check(same, "batch = per text");
  FILE* f = std::fopen((dir + "/ids.bin").c_str(), "wb");
  std::fwrite(&n, 8, 1, f);
  for (uint64_t i = 0; i <= n; ++i) {
    const uint64_t o = id_offs[i];
    std::fwrite(&o, 8, 1, f);
  }
  std::fwrite(ids.data(), 4, ids.size(), f);
  std::fclose(f);
  eg2_tokenizer_free(tok);
  eg2_gguf_close(&g);
}

// The oracle: the threaded Q8_0 GEMM against its one-thread result, and
// one encoder layer of the synthetic model over a small ragged wave.
void check_oracle(const ei_gguf& g, std::mt19937_64& rng) {
  auto q8 = [&](const char* name) { return static_cast<const or_block_q8_0*>(tensor(g, name)->data); };
  auto f32 = [&](const char* name) { return static_cast<const float*>(tensor(g, name)->data); };
  const int n = 37, k = 768, m = 256;
  std::vector<float> x(n * k);
  std::normal_distribution<float> nd(0.0f, 1.0f);
  for (auto& v : x) v = nd(rng);
  std::vector<or_block_q8_0> xq(n * k / 32);
  for (int t = 0; t < n; ++t) or_quantize_row_q8_0(x.data() + t * k, xq.data() + t * k / 32, k);
  std::vector<float> y1(n * m), y4(n * m);
  or_gemm_q8_0(q8("blk.0.attn_q.weight"), xq.data(), n, k, m, y1.data(), 1);
  or_gemm_q8_0(q8("blk.0.attn_q.weight"), xq.data(), n, k, m, y4.data(), 4);
  check(!std::memcmp(y1.data(), y4.data(), y1.size() * 4), "oracle GEMM thread-count invariant");

  or_layer L{};
  L.attn_q = q8("blk.0.attn_q.weight");
  L.attn_k = q8("blk.0.attn_k.weight");
  L.attn_v = q8("blk.0.attn_v.weight");
  L.attn_output = q8("blk.0.attn_output.weight");
  L.ffn_up = q8("blk.0.ffn_up.weight");
  L.ffn_gate = q8("blk.0.ffn_gate.weight");
  L.ffn_down = q8("blk.0.ffn_down.weight");
  L.attn_norm = f32("blk.0.attn_norm.weight");
  L.attn_q_norm = f32("blk.0.attn_q_norm.weight");
  L.attn_k_norm = f32("blk.0.attn_k_norm.weight");
  L.post_attention_norm = f32("blk.0.post_attention_norm.weight");
  L.ffn_norm = f32("blk.0.ffn_norm.weight");
  L.post_ffw_norm = f32("blk.0.post_ffw_norm.weight");
  L.rope_base = 1e4f;
  L.window = 8;
  const size_t offsets[] = {0, 5, 22, 23, 40};
  const int T = 40;
  std::vector<float> h(T * 768);
  for (auto& v : h) v = nd(rng);
  std::vector<int32_t> pos(T);
  for (int s = 0; s < 4; ++s)
    for (size_t t = offsets[s]; t < offsets[s + 1]; ++t) pos[t] = (int32_t)(t - offsets[s]);
  std::vector<float> h1(h), h3(h);
  or_layer_forward(&L, 1e-6f, h1.data(), pos.data(), offsets, 4, 1);
  or_layer_forward(&L, 1e-6f, h3.data(), pos.data(), offsets, 4, 3);
  check(!std::memcmp(h1.data(), h3.data(), h1.size() * 4), "oracle layer thread-count invariant");
  bool finite = true;
  for (float v : h1) finite = finite && std::isfinite(v);
  check(finite, "oracle layer output finite");
  std::vector<float> pooled(768);
  or_mean_pool_rms_l2(h1.data() + 5 * 768, 17, f32("output_norm.weight"), 1e-6f, pooled.data());
  double ss = 0;
  for (float v : pooled) ss += (double)v * v;
  check(std::fabs(ss - 1.0) < 1e-5, "pooled embedding has unit norm");
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: host_check <workdir>\n");
    return 2;
  }
  const std::string dir = argv[1];
  std::mt19937_64 rng(12345);
  ei_gguf model{};
  check_model(dir, model);
  check_attention_plan(rng);
  check_tiles(rng);
  check_packer(rng);
  check_format(rng);
  check_tokenizer(dir);
  if (model.n_tensors) {
    check_oracle(model, rng);
    eg2_gguf_close(&model);
  }
  if (failures) {
    std::fprintf(stderr, "%d host checks failed\n", failures);
    return 1;
  }
  std::printf("host checks passed\n");
  return 0;
}
