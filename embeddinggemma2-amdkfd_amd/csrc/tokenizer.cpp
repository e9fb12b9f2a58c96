// Text -> token ids (include/eg2_tokenizer.h), bit-exact with the
// reference's tokenizer (vendor/embeddinggemma.c/src/tokenizer.c).
//
// The algorithm, as the reference runs it:
//  - special pieces (control, user-defined and unknown tokens, plus the
//    BOS/EOS/PAD and UNK ids; tokenizer.c:128-146) are cut out of the text
//    first, longest piece first (ties by id), each at its non-overlapping
//    left-to-right occurrences in what is left (:304-350);
//  - each remaining run has its spaces escaped to U+2581, with one more in
//    front when the run follows a special or starts the text and the model
//    adds a space prefix (:552-572);
//  - the run is cut into UTF-8 characters (a malformed lead byte is one
//    byte; a character cut by the end of the run is what remains), and
//    adjacent symbols merge while some adjacent pair is a vocabulary piece
//    (or, in the ranked-merge mode, a "left right" merge rule): the pair of
//    highest score first, the leftmost among equal scores, re-checking after
//    each merge the pairs it created (:441-550);
//  - every final symbol becomes its piece's id; one that is not a piece is
//    split again into the two symbols last recorded as forming that text
//    (by their current extent), and failing that into byte-fallback ids
//    (:472-495);
//  - BOS / EOS come from the model flags when asked (:574-631).
// In the ranked-merge mode a run is further cut into newline and
// non-newline stretches; a newline stretch that is a piece is one id.
#include "eg2_tokenizer.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <deque>
#include <queue>
#include <stdexcept>
#include <string>
#include <string_view>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

constexpr int32_t kTypeUnknown = 2, kTypeControl = 3, kTypeUserDefined = 4, kTypeByte = 6;
constexpr uint32_t kAttrUnknown = 1u << 0, kAttrControl = 1u << 3, kAttrUserDefined = 1u << 4, kAttrByte = 1u << 5;
const char kSpace[3] = {(char)0xE2, (char)0x96, (char)0x81};  // U+2581

bool key_is(const ei_str& s, const char* z) {
  const size_t n = std::strlen(z);
  return s.len == n && std::memcmp(s.str, z, n) == 0;
}

const ei_kv* find_kv(const ei_gguf* g, const char* key) {
  for (uint64_t i = 0; i < g->n_kv; ++i)
    if (key_is(g->kv[i].key, key)) return &g->kv[i];
  return nullptr;
}

const ei_kv* find_array(const ei_gguf* g, const char* key, uint32_t elem, bool required) {
  const ei_kv* kv = find_kv(g, key);
  if (!kv) {
    if (required) throw std::runtime_error(std::string("missing tokenizer key ") + key);
    return nullptr;
  }
  if (kv->type != EI_GGUF_ARRAY || kv->arr_type != elem) throw std::runtime_error(std::string("bad array ") + key);
  return kv;
}

}  // namespace

struct eg2_tokenizer {
  struct Special {
    int32_t id;
    uint32_t attr;
    size_t len;
  };
  struct Symbol {
    int prev, next;
    const char* text;
    size_t n;
  };
  struct Bigram {
    int left, right;
    float score;
    size_t size;
  };

  std::vector<std::string_view> pieces;
  std::vector<float> scores;
  std::unordered_map<std::string_view, std::pair<int32_t, float>> vocab;  // piece -> (id, score)
  std::unordered_map<std::string_view, float> merges;                     // "left right" -> -rank
  bool ranked = false;
  int32_t byte_id[256];
  std::vector<Special> specials;
  std::deque<std::string> owned;  // keys of empty pieces
  int32_t bos = 2, eos = 1, unk = 3, pad = 0;
  bool add_bos = true, add_eos = false, add_space_prefix = true;

  explicit eg2_tokenizer(const ei_gguf* g) {
    const ei_kv* toks = find_array(g, "tokenizer.ggml.tokens", EI_GGUF_STRING, true);
    const ei_kv* sc = find_array(g, "tokenizer.ggml.scores", EI_GGUF_F32, true);
    const ei_kv* ty = find_array(g, "tokenizer.ggml.token_type", EI_GGUF_I32, true);
    const size_t n = toks->arr_n;
    if (n == 0 || n > (size_t)INT32_MAX || sc->arr_n < n || ty->arr_n < n)
      throw std::runtime_error("tokenizer arrays disagree in length");
    auto u64 = [&](const char* key, uint64_t dflt) {
      const ei_kv* kv = find_kv(g, key);
      return kv ? kv->v.u64 : dflt;
    };
    auto flag = [&](const char* key, bool dflt) {
      const ei_kv* kv = find_kv(g, key);
      return kv ? kv->v.b : dflt;
    };
    bos = (int32_t)u64("tokenizer.ggml.bos_token_id", 2);
    eos = (int32_t)u64("tokenizer.ggml.eos_token_id", 1);
    unk = (int32_t)u64("tokenizer.ggml.unknown_token_id", 3);
    pad = (int32_t)u64("tokenizer.ggml.padding_token_id", 0);
    add_bos = flag("tokenizer.ggml.add_bos_token", true);
    add_eos = flag("tokenizer.ggml.add_eos_token", false);
    add_space_prefix = flag("tokenizer.ggml.add_space_prefix", true);

    const ei_str* strs = static_cast<const ei_str*>(toks->arr_data);
    pieces.resize(n);
    scores.resize(n);
    std::vector<int32_t> types(n);
    vocab.reserve(2 * n);
    for (size_t id = 0; id < n; ++id) {
      pieces[id] = std::string_view(strs[id].str, strs[id].len);
      std::memcpy(&scores[id], static_cast<const char*>(sc->arr_data) + 4 * id, 4);
      std::memcpy(&types[id], static_cast<const char*>(ty->arr_data) + 4 * id, 4);
      std::string_view key = pieces[id];
      if (key.empty()) {
        owned.push_back("[EMPTY_" + std::to_string(id) + "]");
        key = owned.back();
      }
      vocab.insert_or_assign(key, std::make_pair((int32_t)id, scores[id]));
    }
    static const char hex[] = "0123456789ABCDEF";
    for (int b = 0; b < 256; ++b) {
      const char name[6] = {'<', '0', 'x', hex[b >> 4], hex[b & 15], '>'};
      int32_t id = text_to_id(name, 6);
      if (id < 0) {
        const char raw = (char)b;
        id = text_to_id(&raw, 1);
      }
      if (id < 0) {
        char msg[64];
        std::snprintf(msg, sizeof msg, "missing byte fallback token for 0x%02X", b);
        throw std::runtime_error(msg);
      }
      byte_id[b] = id;
    }
    for (size_t id = 0; id < n; ++id) {
      uint32_t attr = 0;
      switch (types[id]) {
        case kTypeUnknown: attr |= kAttrUnknown; break;
        case kTypeControl: attr |= kAttrControl; break;
        case kTypeUserDefined: attr |= kAttrUserDefined; break;
        case kTypeByte: attr |= kAttrByte; break;
        default: break;
      }
      const int32_t i = (int32_t)id;
      if (i == bos || i == eos || i == pad) attr |= kAttrControl;
      if (i == unk) attr |= kAttrUnknown;
      if ((attr & (kAttrControl | kAttrUserDefined | kAttrUnknown)) && !pieces[id].empty())
        specials.push_back({i, attr, pieces[id].size()});
    }
    std::sort(specials.begin(), specials.end(), [](const Special& a, const Special& b) {
      return a.len != b.len ? a.len > b.len : a.id < b.id;
    });
    if (const ei_kv* mg = find_array(g, "tokenizer.ggml.merges", EI_GGUF_STRING, false)) {
      ranked = true;
      const ei_str* ms = static_cast<const ei_str*>(mg->arr_data);
      merges.reserve(2 * mg->arr_n);
      for (uint64_t i = 0; i < mg->arr_n; ++i) merges.emplace(std::string_view(ms[i].str, ms[i].len), -(float)i);
    }
  }

  int32_t text_to_id(const char* text, size_t len) const {
    const auto it = vocab.find(std::string_view(text, len));
    return it == vocab.end() ? -1 : it->second.first;
  }

  // One escaped run through the bigram merges, ids appended to out.
  void merge_run(const char* text, size_t len, std::vector<int32_t>& out) const {
    if (len == 0) return;
    std::vector<Symbol> sym;
    sym.reserve(len);
    for (size_t off = 0; off < len;) {
      const uint8_t lead = (uint8_t)text[off];
      size_t n = (lead & 0x80u) == 0 ? 1 : (lead & 0xE0u) == 0xC0u ? 2 : (lead & 0xF0u) == 0xE0u ? 3
                                                                    : (lead & 0xF8u) == 0xF0u ? 4 : 1;
      n = std::min(n, len - off);
      const int i = (int)sym.size();
      sym.push_back({i - 1, off + n == len ? -1 : i + 1, text + off, n});
      off += n;
    }
    auto worse = [](const Bigram& a, const Bigram& b) {  // priority: score, then leftmost
      return a.score < b.score || (a.score == b.score && a.left > b.left);
    };
    std::priority_queue<Bigram, std::vector<Bigram>, decltype(worse)> heap(worse);
    std::unordered_map<std::string_view, std::pair<int, int>> formed;  // text -> last pair forming it
    auto try_pair = [&](int left, int right) {
      if (left < 0 || right < 0) return;
      const Symbol& l = sym[left];
      const Symbol& r = sym[right];
      const size_t n = l.n + r.n;
      float score;
      if (ranked) {
        if (std::memchr(l.text, '\n', n)) return;
        std::string key;
        key.reserve(n + 1);
        key.append(l.text, l.n).push_back(' ');
        key.append(r.text, r.n);
        const auto it = merges.find(key);
        if (it == merges.end()) return;
        score = it->second;
      } else {
        const auto it = vocab.find(std::string_view(l.text, n));
        if (it == vocab.end()) return;
        score = it->second.second;
      }
      heap.push({left, right, score, n});
      formed.insert_or_assign(std::string_view(l.text, n), std::make_pair(left, right));
    };
    for (int i = 1; i < (int)sym.size(); ++i) try_pair(i - 1, i);
    while (!heap.empty()) {
      const Bigram b = heap.top();
      heap.pop();
      Symbol& l = sym[b.left];
      Symbol& r = sym[b.right];
      if (l.n == 0 || r.n == 0 || l.n + r.n != b.size) continue;  // a stale pair
      l.n += r.n;
      r.n = 0;
      l.next = r.next;
      if (r.next >= 0) sym[r.next].prev = b.left;
      try_pair(l.prev, b.left);
      try_pair(b.left, l.next);
    }
    // Final symbols to ids (tokenizer.c:472-495).
    auto emit = [&](auto&& self, int idx) -> void {
      if (idx < 0 || idx >= (int)sym.size()) return;
      const Symbol& s = sym[idx];
      if (s.n == 0) return;
      const std::string_view text(s.text, s.n);
      const auto v = vocab.find(text);
      if (v != vocab.end()) {
        out.push_back(v->second.first);
        return;
      }
      const auto f = formed.find(text);
      if (f != formed.end() && f->second.first != idx && f->second.second != idx) {
        self(self, f->second.first);
        self(self, f->second.second);
        return;
      }
      for (size_t i = 0; i < s.n; ++i) out.push_back(byte_id[(uint8_t)s.text[i]]);
    };
    for (int i = 0; i != -1; i = sym[i].next) emit(emit, i);
  }

  void tokenize(const char* text, size_t len, bool add_special, bool parse_special, std::vector<int32_t>& out) const {
    struct Frag {
      bool token;
      size_t off, len;
      int32_t id;
    };
    std::vector<Frag> frags, next;
    if (len > 0) {
      frags.push_back({false, 0, len, 0});
      for (const Special& sp : specials) {
        if (!parse_special && (sp.attr & (kAttrControl | kAttrUnknown))) continue;
        const std::string_view piece = pieces[sp.id];
        next.clear();
        for (const Frag& f : frags) {
          if (f.token) {
            next.push_back(f);
            continue;
          }
          const std::string_view hay(text + f.off, f.len);
          size_t pos = 0;
          for (;;) {
            const size_t m = hay.find(piece, pos);
            if (m == std::string_view::npos) break;
            if (m > pos) next.push_back({false, f.off + pos, m - pos, 0});
            next.push_back({true, 0, 0, sp.id});
            pos = m + piece.size();
          }
          if (pos < f.len) next.push_back({false, f.off + pos, f.len - pos, 0});
        }
        frags.swap(next);
      }
    }
    if (add_special && add_bos) out.push_back(bos);
    bool prev_special = true;
    std::string esc;
    for (const Frag& f : frags) {
      if (f.token) {
        out.push_back(f.id);
        prev_special = true;
        continue;
      }
      esc.clear();
      if (add_space_prefix && prev_special) esc.append(kSpace, 3);
      for (size_t i = 0; i < f.len; ++i) {
        if (text[f.off + i] == ' ') esc.append(kSpace, 3);
        else esc.push_back(text[f.off + i]);
      }
      if (ranked) {
        for (size_t start = 0; start < esc.size();) {
          const bool nl = esc[start] == '\n';
          size_t end = start + 1;
          while (end < esc.size() && (esc[end] == '\n') == nl) ++end;
          const int32_t id = nl ? text_to_id(esc.data() + start, end - start) : -1;
          if (id >= 0) out.push_back(id);
          else merge_run(esc.data() + start, end - start, out);
          start = end;
        }
      } else {
        merge_run(esc.data(), esc.size(), out);
      }
      prev_special = false;
    }
    if (add_special && add_eos) out.push_back(eos);
  }
};

extern "C" eg2_tokenizer* eg2_tokenizer_create(const ei_gguf* g, char* err, size_t len) {
  try {
    if (!g) throw std::runtime_error("empty GGUF");
    return new eg2_tokenizer(g);
  } catch (const std::exception& e) {
    if (err && len) std::snprintf(err, len, "HIP: %s", e.what());
    return nullptr;
  }
}

extern "C" void eg2_tokenizer_free(eg2_tokenizer* tok) { delete tok; }

extern "C" int32_t eg2_tokenizer_text_to_id(const eg2_tokenizer* tok, const char* text, size_t len) {
  return tok && (text || !len) ? tok->text_to_id(text, len) : -1;
}

extern "C" size_t eg2_tokenize(const eg2_tokenizer* tok, const char* text, size_t len, bool add_special,
                               bool parse_special, int32_t* ids, size_t cap) {
  if (!tok || (!text && len)) return 0;
  std::vector<int32_t> out;
  tok->tokenize(text, len, add_special, parse_special, out);
  if (ids) std::copy_n(out.begin(), std::min(cap, out.size()), ids);
  return out.size();
}

extern "C" size_t eg2_tokenize_batch(const eg2_tokenizer* tok, const char* texts, const size_t* text_offsets,
                                     size_t n, bool add_special, bool parse_special, int32_t* ids, size_t cap,
                                     size_t* id_offsets, unsigned threads) {
  if (!tok || !text_offsets || !id_offsets || (n && !texts)) return SIZE_MAX;
  std::vector<std::vector<int32_t>> per(n);
  unsigned t = threads ? threads : std::max(1u, std::thread::hardware_concurrency());
  t = (unsigned)std::min<size_t>(std::min(t, 32u), std::max<size_t>(n, 1));
  std::vector<std::thread> pool;
  for (unsigned w = 0; w < t; ++w)
    pool.emplace_back([&, w] {
      for (size_t i = w; i < n; i += t)
        tok->tokenize(texts + text_offsets[i], text_offsets[i + 1] - text_offsets[i], add_special, parse_special,
                      per[i]);
    });
  for (auto& th : pool) th.join();
  size_t total = 0;
  for (const auto& v : per) total += v.size();
  if (total > cap || (total && !ids)) return SIZE_MAX;
  id_offsets[0] = 0;
  for (size_t i = 0; i < n; ++i) {
    std::copy(per[i].begin(), per[i].end(), ids + id_offsets[i]);
    id_offsets[i + 1] = id_offsets[i] + per[i].size();
  }
  return total;
}
