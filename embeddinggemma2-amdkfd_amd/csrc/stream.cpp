// Deterministic wave packing (the dynamic batcher's fit rules) and the
// stream runner on top of the executor's C ABI (include/eg2_stream.h).
#include "eg2_stream.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <list>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "eg2_hip.h"
#include "gemma2_kfd.h"

namespace {

constexpr int kEmbd = 768;
constexpr double kWaitSeconds = 30.0;  // polling for a finished lane, as long as a lane's own wait

bool valid(const eg2_batch_config* c) {
  return c && c->max_batch_tokens > 0 && c->max_batch_sequence_tokens > 0 && c->max_batch_requests > 0;
}

// ei_sum_squares, SSE2 branch (kernels.c:82-94): two 4-wide accumulators
// over a stride of 8, products rounded before each addition, then
// (v0 + v2) + (v1 + v3) (kernels.c:35-39) and a scalar tail.
float sum_squares_sse2(const float* x, int n) {
  float a[4] = {0, 0, 0, 0}, b[4] = {0, 0, 0, 0};
  int i = 0;
  for (; i + 7 < n; i += 8)
    for (int j = 0; j < 4; ++j) {
      const float p = x[i + j] * x[i + j], q = x[i + 4 + j] * x[i + 4 + j];
      a[j] = a[j] + p;
      b[j] = b[j] + q;
    }
  float v[4];
  for (int j = 0; j < 4; ++j) v[j] = a[j] + b[j];
  float sum = (v[0] + v[2]) + (v[1] + v[3]);
  for (; i < n; ++i) {
    const float p = x[i] * x[i];
    sum = sum + p;
  }
  return sum;
}

}  // namespace

extern "C" void eg2_batch_config_default(eg2_batch_config* cfg) {
  if (!cfg) return;
  cfg->max_batch_tokens = 2048;
  cfg->max_batch_sequence_tokens = 2048;
  cfg->max_batch_requests = 32;
  cfg->lookahead = 1;
  cfg->sort_longest_first = 1;
}

extern "C" size_t eg2_pack_waves(const size_t* lengths, size_t n, const eg2_batch_config* cfg, size_t* order,
                                 size_t* wave_end) {
  if (!lengths || !order || !wave_end || !valid(cfg)) return 0;
  for (size_t i = 0; i < n; ++i)
    if (lengths[i] == 0) return 0;
  const size_t budget = cfg->max_batch_tokens, seq_limit = cfg->max_batch_sequence_tokens;
  const size_t max_req = cfg->max_batch_requests;
  const size_t max_scan = max_req <= SIZE_MAX / 8 ? max_req * 8 : SIZE_MAX;  // inference_service.c:415-417
  std::list<size_t> queue;
  for (size_t i = 0; i < n; ++i) queue.push_back(i);
  size_t placed = 0, waves = 0;
  std::vector<size_t> wave;
  while (!queue.empty()) {
    wave.clear();
    // The head always starts the wave.
    const size_t head = queue.front();
    queue.pop_front();
    wave.push_back(head);
    size_t total = lengths[head];
    if (lengths[head] <= seq_limit) {
      if (cfg->lookahead) {
        size_t scanned = 0;
        for (auto it = queue.begin(); it != queue.end() && wave.size() < max_req && scanned < max_scan;) {
          ++scanned;
          const size_t len = lengths[*it];
          if (len <= seq_limit && total + len <= budget) {
            wave.push_back(*it);
            total += len;
            it = queue.erase(it);
          } else {
            ++it;
          }
        }
      } else {
        while (!queue.empty() && wave.size() < max_req) {
          const size_t len = lengths[queue.front()];
          if (len > seq_limit || total + len > budget) break;
          wave.push_back(queue.front());
          total += len;
          queue.pop_front();
        }
      }
    }
    if (cfg->sort_longest_first && wave.size() > 1)
      std::stable_sort(wave.begin(), wave.end(), [&](size_t a, size_t b) { return lengths[a] > lengths[b]; });
    for (size_t s : wave) order[placed++] = s;
    wave_end[waves++] = placed;
  }
  return waves;
}

extern "C" bool eg2_normalize_prefix(float* embedding, unsigned dims) {
  if (!embedding || (dims != 128 && dims != 256 && dims != 512 && dims != (unsigned)kEmbd)) return false;
  if (dims < (unsigned)kEmbd) {
    const float ss = sum_squares_sse2(embedding, (int)dims);
    if (ss != 0.0f) {
      const float scale = 1.0f / std::sqrt(ss);
      for (unsigned i = 0; i < dims; ++i) embedding[i] = embedding[i] * scale;
    }
  }
  return true;
}

namespace {

std::string strip_hip(const char* msg) {
  const std::string m(msg);
  return m.rfind("HIP: ", 0) == 0 ? m.substr(5) : m;
}

// Lanes taken from the executor's pool for one stream; returned on every exit.
struct HeldLanes {
  void* ctx;
  std::vector<int> lanes;
  ~HeldLanes() {
    for (int l : lanes)
      if (l >= 0) eg2_kfd_release_lane(ctx, (unsigned)l);
  }
};

}  // namespace

extern "C" bool eg2_stream_embed(void* ctx, const int32_t* ids, const size_t* text_offsets, size_t n_texts,
                                 const unsigned* dims, const eg2_batch_config* cfg, float* out, size_t* n_waves,
                                 char* err, size_t len) {
  try {
    if (!ctx || !ids || !text_offsets || !dims || !out || !valid(cfg) || n_texts == 0)
      throw std::runtime_error("invalid stream arguments");
    std::vector<size_t> lengths(n_texts);
    for (size_t i = 0; i < n_texts; ++i) {
      if (text_offsets[i + 1] <= text_offsets[i]) throw std::runtime_error("empty or unordered text");
      if (dims[i] != 128 && dims[i] != 256 && dims[i] != 512 && dims[i] != (unsigned)kEmbd)
        throw std::runtime_error("unsupported embedding dimensions");
      lengths[i] = text_offsets[i + 1] - text_offsets[i];
    }
    std::vector<size_t> order(n_texts), wave_end(n_texts);
    const size_t waves = eg2_pack_waves(lengths.data(), n_texts, cfg, order.data(), wave_end.data());
    if (!waves) throw std::runtime_error("packing failed");

    // Each slot is a lane held for the whole stream; wave w runs on a free
    // slot, or else on the first slot whose wave finishes (collected just
    // before the slot is reused), so up to L waves are in flight and a long
    // wave never holds up the slots behind it. The lanes are taken before the first
    // wave: one waiting for a free lane (nothing is held yet), the others
    // only if free at once, so that a stream never waits while holding
    // lanes (concurrent streams could otherwise each hold some lanes and
    // wait for the others' forever). L is the number taken.
    const size_t want = std::min<size_t>(std::max(1u, eg2_kfd_lanes(ctx)), waves);
    HeldLanes held{ctx, {}};
    held.lanes.push_back(eg2_kfd_acquire_lane(ctx));
    while (held.lanes.size() < want) {
      const int l = eg2_kfd_try_acquire_lane(ctx);
      if (l < 0) break;
      held.lanes.push_back(l);
    }
    const size_t L = held.lanes.size();
    std::vector<size_t> pend_begin(L), pend_end(L);
    std::vector<bool> busy(L, false);
    std::vector<int32_t> wave_ids;
    std::vector<size_t> offsets;
    std::vector<float> wave_out;
    char msg[512] = {0};
    auto finish = [&](size_t slot) {
      const size_t b = pend_end[slot] - pend_begin[slot];
      wave_out.resize(b * kEmbd);
      busy[slot] = false;
      if (!eg2_kfd_collect_lane(ctx, (unsigned)held.lanes[slot], wave_out.data(), msg, sizeof msg))
        throw std::runtime_error(strip_hip(msg));
      for (size_t k = 0; k < b; ++k) {
        const size_t i = order[pend_begin[slot] + k];
        float* e = out + i * kEmbd;
        std::memcpy(e, wave_out.data() + k * kEmbd, kEmbd * sizeof(float));
        eg2_normalize_prefix(e, dims[i]);
        std::fill(e + dims[i], e + kEmbd, 0.0f);
      }
    };
    // A free slot, or the first busy one whose wave is done (polled, as the
    // executor's own waits are); past kWaitSeconds the oldest wave's
    // collect takes over, whose wait reports a time-out or failure.
    std::vector<size_t> started(L, 0);
    auto free_slot = [&]() -> size_t {
      for (size_t s = 0; s < L; ++s)
        if (!busy[s]) return s;
      const auto t0 = std::chrono::steady_clock::now();
      for (;;) {
        for (size_t s = 0; s < L; ++s) {
          if (eg2_kfd_lane_ready(ctx, (unsigned)held.lanes[s], msg, sizeof msg) != 0) {
            finish(s);  // done, or failed: collect reports the failure
            return s;
          }
        }
        if (std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > kWaitSeconds) {
          const size_t oldest = (size_t)(std::min_element(started.begin(), started.end()) - started.begin());
          finish(oldest);
          return oldest;
        }
        std::this_thread::yield();
      }
    };
    size_t begin = 0;
    for (size_t w = 0; w < waves; ++w) {
      const size_t slot = free_slot(), end = wave_end[w];
      wave_ids.clear();
      offsets.assign(1, 0);
      for (size_t k = begin; k < end; ++k) {
        const size_t i = order[k];
        wave_ids.insert(wave_ids.end(), ids + text_offsets[i], ids + text_offsets[i + 1]);
        offsets.push_back(wave_ids.size());
      }
      const unsigned lane = (unsigned)held.lanes[slot];
      if (!eg2_kfd_stage_lane(ctx, lane, wave_ids.data(), offsets.data(), end - begin, msg, sizeof msg) ||
          !eg2_kfd_launch_lane(ctx, lane, 1, msg, sizeof msg))
        throw std::runtime_error(strip_hip(msg));
      pend_begin[slot] = begin;
      pend_end[slot] = end;
      busy[slot] = true;
      started[slot] = w;
      begin = end;
    }
    for (size_t s = 0; s < L; ++s)
      if (busy[s]) finish(s);
    if (n_waves) *n_waves = waves;
    return true;
  } catch (const std::exception& e) {
    if (err && len) std::snprintf(err, len, "HIP: %s", e.what());
    return false;
  }
}
