// Runtime state of the KV-cache path (host C++ over the HIP runtime).
// Replaces src/gemma4_runtime.cu of gemma.c: sizes and allocates the sliding
// ring caches and the full-length global caches, owns the page tables, the
// sequence lengths and the token metadata of each step, and the RoPE tables
// the prepared Q/K use.
#include <hip/hip_bf16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <new>
#include <vector>

#include "gemma4_runtime.h"

namespace {

constexpr int32_t kMaxPositions = 262144;       // src/gemma4.h:10
constexpr int32_t kSlidingWindow = 1024;        // src/gemma4.h:22-23
constexpr int32_t kSlidingHeadDim = 256;
constexpr int32_t kGlobalHeadDim = 512;
constexpr int32_t kGlobalRotaryDim = kGlobalHeadDim / 4;  // partial rotary 0.25
constexpr float kSlidingTheta = 10000.0f;
constexpr float kGlobalTheta = 1000000.0f;

int32_t div_up(int32_t a, int32_t b) { return (a + b - 1) / b; }

size_t cache_elements(const Gemma4KvCacheConfig &c) {
  return (size_t)c.num_layers * c.num_pages * c.page_size * c.num_heads * c.head_dim;
}

// Ring slots a sliding cache needs so that any live window, including one
// straddling page boundaries, is mapped (src/gemma4_runtime.cu:18-24).
int32_t sliding_pages_per_sequence(int32_t max_seq_len, int32_t page_size) {
  if (max_seq_len <= kSlidingWindow) return div_up(max_seq_len, page_size);
  return div_up(kSlidingWindow + page_size - 1, page_size);
}

// cos/sin of pos * theta^(-2i/exponent_dim), row-major [pos][i]
// (src/gemma4_runtime.cu:27-44).
void rope_tables(std::vector<float> &cos_t, std::vector<float> &sin_t, int32_t positions,
                 int32_t half, float theta, int32_t exponent_dim) {
  cos_t.resize((size_t)positions * half);
  sin_t.resize(cos_t.size());
  for (int32_t i = 0; i < half; ++i) {
    const float inv_freq = std::pow(theta, -2.0f * (float)i / (float)exponent_dim);
    for (int32_t pos = 0; pos < positions; ++pos) {
      const float angle = (float)pos * inv_freq;
      cos_t[(size_t)pos * half + i] = std::cos(angle);
      sin_t[(size_t)pos * half + i] = std::sin(angle);
    }
  }
}

template <typename T>
hipError_t alloc(T **p, size_t count) {
  return hipMalloc(reinterpret_cast<void **>(p), std::max<size_t>(count, 1) * sizeof(T));
}

template <typename T>
hipError_t upload(T *dst, const T *src, size_t count, hipStream_t stream) {
  if (count == 0) return hipSuccess;
  return hipMemcpyAsync(dst, src, count * sizeof(T), hipMemcpyHostToDevice, stream);
}

hipError_t upload_all(Gemma4RuntimeState *s, size_t tokens, hipStream_t stream) {
  hipError_t e;
  if ((e = upload(s->sliding_page_table, s->h_sliding_page_table.data(),
                  s->h_sliding_page_table.size(), stream)) != hipSuccess) return e;
  if ((e = upload(s->global_page_table, s->h_global_page_table.data(),
                  s->h_global_page_table.size(), stream)) != hipSuccess) return e;
  if ((e = upload(s->seq_lengths, s->h_seq_lengths.data(), s->h_seq_lengths.size(),
                  stream)) != hipSuccess) return e;
  if ((e = upload(s->token_batch, s->h_token_batch.data(), tokens, stream)) != hipSuccess) return e;
  if ((e = upload(s->token_position, s->h_token_position.data(), tokens, stream)) != hipSuccess) return e;
  if ((e = upload(s->sliding_slot_logical_pages, s->h_sliding_slot_logical_pages.data(),
                  s->h_sliding_slot_logical_pages.size(), stream)) != hipSuccess) return e;
  return upload(s->global_slot_logical_pages, s->h_global_slot_logical_pages.data(),
                s->h_global_slot_logical_pages.size(), stream);
}

template <typename T>
hipError_t download(std::vector<T> &dst, const T *src, size_t count, hipStream_t stream) {
  if (count == 0) return hipSuccess;
  return hipMemcpyAsync(dst.data(), src, count * sizeof(T), hipMemcpyDeviceToHost, stream);
}

}  // namespace

void gemma4_runtime_state_free(Gemma4RuntimeState *s) {
  void *ptrs[] = {s->sliding_cache_k, s->sliding_cache_v, s->global_cache_k, s->global_cache_v,
                  s->sliding_page_table, s->global_page_table, s->seq_lengths,
                  s->token_batch, s->token_position, s->sliding_cos, s->sliding_sin,
                  s->global_cos, s->global_sin, s->sliding_slot_logical_pages,
                  s->global_slot_logical_pages, s->device_step_status};
  for (void *p : ptrs) {
    if (p != nullptr) (void)hipFree(p);
  }
  *s = Gemma4RuntimeState();
}

hipError_t gemma4_runtime_state_init(Gemma4RuntimeState *s, int32_t batch_size,
                                     int32_t max_seq_len, int32_t page_size,
                                     hipStream_t stream) {
  if (s == nullptr || batch_size <= 0 || max_seq_len <= 0 || page_size <= 0 ||
      max_seq_len > kMaxPositions) {
    return hipErrorInvalidValue;
  }
  const int32_t global_pps = div_up(max_seq_len, page_size);
  const int32_t sliding_pps = sliding_pages_per_sequence(max_seq_len, page_size);
  const size_t token_rows = (size_t)batch_size * max_seq_len;

  *s = Gemma4RuntimeState();
  s->batch_size = batch_size;
  s->max_seq_len = max_seq_len;
  s->page_size = page_size;
  s->sliding_cache_config =
      gemma4_kv_cache_make_config(false, batch_size * sliding_pps, page_size, sliding_pps);
  s->sliding_cache_config.batch_size = batch_size;
  s->sliding_cache_config.window_size = std::min(max_seq_len, kSlidingWindow);
  s->global_cache_config =
      gemma4_kv_cache_make_config(true, batch_size * global_pps, page_size, global_pps);
  s->global_cache_config.batch_size = batch_size;

  s->h_sliding_page_table.assign((size_t)batch_size * sliding_pps, -1);
  s->h_global_page_table.assign((size_t)batch_size * global_pps, -1);
  s->h_sliding_slot_logical_pages.assign(s->h_sliding_page_table.size(), -1);
  s->h_global_slot_logical_pages.assign(s->h_global_page_table.size(), -1);
  s->h_seq_lengths.assign(batch_size, 0);
  s->h_token_batch.assign(token_rows, 0);
  s->h_token_position.assign(token_rows, 0);

  std::vector<float> sc, ss, gc, gs;
  rope_tables(sc, ss, max_seq_len, kSlidingHeadDim / 2, kSlidingTheta, kSlidingHeadDim);
  rope_tables(gc, gs, max_seq_len, kGlobalRotaryDim / 2, kGlobalTheta, kGlobalHeadDim);

  hipError_t e = hipSuccess;
  auto step = [&](hipError_t r) {
    if (e == hipSuccess) e = r;
  };
  step(alloc(&s->sliding_cache_k, cache_elements(s->sliding_cache_config)));
  step(alloc(&s->sliding_cache_v, cache_elements(s->sliding_cache_config)));
  step(alloc(&s->global_cache_k, cache_elements(s->global_cache_config)));
  step(alloc(&s->global_cache_v, cache_elements(s->global_cache_config)));
  step(alloc(&s->sliding_page_table, s->h_sliding_page_table.size()));
  step(alloc(&s->global_page_table, s->h_global_page_table.size()));
  step(alloc(&s->seq_lengths, s->h_seq_lengths.size()));
  step(alloc(&s->token_batch, token_rows));
  step(alloc(&s->token_position, token_rows));
  step(alloc(&s->sliding_cos, sc.size()));
  step(alloc(&s->sliding_sin, ss.size()));
  step(alloc(&s->global_cos, gc.size()));
  step(alloc(&s->global_sin, gs.size()));
  step(alloc(&s->sliding_slot_logical_pages, s->h_sliding_slot_logical_pages.size()));
  step(alloc(&s->global_slot_logical_pages, s->h_global_slot_logical_pages.size()));
  step(alloc(&s->device_step_status, 1));
  if (e == hipSuccess) step(hipMemsetAsync(s->device_step_status, 0, sizeof(int32_t), stream));
  if (e == hipSuccess) {
    step(upload(s->sliding_cos, sc.data(), sc.size(), stream));
    step(upload(s->sliding_sin, ss.data(), ss.size(), stream));
    step(upload(s->global_cos, gc.data(), gc.size(), stream));
    step(upload(s->global_sin, gs.data(), gs.size(), stream));
    step(upload_all(s, 0, stream));
    // The tables are uploaded from function-local vectors.
    step(hipStreamSynchronize(stream));
  }
  if (e != hipSuccess) gemma4_runtime_state_free(s);
  return e;
}

hipError_t gemma4_runtime_prepare_prefill(Gemma4RuntimeState *s, int32_t seq_len,
                                          hipStream_t stream) {
  if (s == nullptr || seq_len < 0 || seq_len > s->max_seq_len) return hipErrorInvalidValue;
  // Rebuild the mappings on copies so a failure leaves the state untouched.
  std::vector<int32_t> spt(s->h_sliding_page_table.size(), -1), sslot(spt.size(), -1);
  std::vector<int32_t> gpt(s->h_global_page_table.size(), -1), gslot(gpt.size(), -1);
  for (int32_t b = 0; b < s->batch_size; ++b) {
    if (gemma4_kv_cache_ensure_range(spt, sslot, s->sliding_cache_config, b, 0, seq_len) < 0 ||
        gemma4_kv_cache_ensure_range(gpt, gslot, s->global_cache_config, b, 0, seq_len) < 0) {
      return hipErrorInvalidValue;
    }
  }
  s->h_sliding_page_table.swap(spt);
  s->h_sliding_slot_logical_pages.swap(sslot);
  s->h_global_page_table.swap(gpt);
  s->h_global_slot_logical_pages.swap(gslot);
  for (int32_t b = 0; b < s->batch_size; ++b) {
    s->h_seq_lengths[b] = seq_len;
    for (int32_t pos = 0; pos < seq_len; ++pos) {  // batch-major rows
      const size_t row = (size_t)b * seq_len + pos;
      s->h_token_batch[row] = b;
      s->h_token_position[row] = pos;
    }
  }
  s->token_count = s->batch_size * seq_len;
  hipError_t e = upload_all(s, (size_t)s->token_count, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);  // host vectors may change next
  if (e == hipSuccess) s->host_stale = false;  // rebuilt from scratch on the host
  return e;
}

hipError_t gemma4_runtime_sync_host(Gemma4RuntimeState *s, hipStream_t stream) {
  if (s == nullptr) return hipErrorInvalidValue;
  hipError_t e;
  if ((e = download(s->h_sliding_page_table, s->sliding_page_table,
                    s->h_sliding_page_table.size(), stream)) != hipSuccess) return e;
  if ((e = download(s->h_global_page_table, s->global_page_table,
                    s->h_global_page_table.size(), stream)) != hipSuccess) return e;
  if ((e = download(s->h_sliding_slot_logical_pages, s->sliding_slot_logical_pages,
                    s->h_sliding_slot_logical_pages.size(), stream)) != hipSuccess) return e;
  if ((e = download(s->h_global_slot_logical_pages, s->global_slot_logical_pages,
                    s->h_global_slot_logical_pages.size(), stream)) != hipSuccess) return e;
  if ((e = download(s->h_seq_lengths, s->seq_lengths, s->h_seq_lengths.size(), stream)) != hipSuccess) return e;
  const size_t tokens = (size_t)std::max(s->token_count, 0);
  if ((e = download(s->h_token_batch, s->token_batch, tokens, stream)) != hipSuccess) return e;
  if ((e = download(s->h_token_position, s->token_position, tokens, stream)) != hipSuccess) return e;
  if ((e = hipStreamSynchronize(stream)) != hipSuccess) return e;
  s->host_stale = false;
  return hipSuccess;
}

hipError_t gemma4_runtime_device_step_status(const Gemma4RuntimeState *s, int32_t *status) {
  if (s == nullptr || status == nullptr || s->device_step_status == nullptr) return hipErrorInvalidValue;
  return hipMemcpy(status, s->device_step_status, sizeof(int32_t), hipMemcpyDeviceToHost);
}

hipError_t gemma4_runtime_prepare_decode_step(Gemma4RuntimeState *s, hipStream_t stream) {
  if (s == nullptr) return hipErrorInvalidValue;
  if (s->host_stale) {  // device-side steps ran since the host vectors were current
    const hipError_t se = gemma4_runtime_sync_host(s, stream);
    if (se != hipSuccess) return se;
  }
  const Gemma4KvCacheConfig &sc = s->sliding_cache_config;
  const Gemma4KvCacheConfig &gc = s->global_cache_config;
  // Validate every sequence before any mutation: the position must fit and
  // neither ring slot may hold a newer logical page (the reference checks the
  // position first, src/gemma4_runtime.cu:279-285; the slot check is done
  // here too so a refused step never leaves a partial mapping behind).
  for (int32_t b = 0; b < s->batch_size; ++b) {
    const int32_t pos = s->h_seq_lengths[b];
    if (pos < 0 || pos >= s->max_seq_len) return hipErrorInvalidValue;
    const int32_t slp = pos / sc.page_size, glp = pos / gc.page_size;
    if (s->h_sliding_slot_logical_pages[(size_t)b * sc.max_pages_per_seq +
                                        slp % sc.max_pages_per_seq] > slp ||
        s->h_global_slot_logical_pages[(size_t)b * gc.max_pages_per_seq +
                                       glp % gc.max_pages_per_seq] > glp) {
      return hipErrorInvalidValue;
    }
  }
  hipError_t e = hipSuccess;
  for (int32_t b = 0; b < s->batch_size; ++b) {
    const int32_t pos = s->h_seq_lengths[b];
    gemma4_kv_cache_ensure_page(s->h_sliding_page_table, s->h_sliding_slot_logical_pages,
                                sc, b, pos);
    gemma4_kv_cache_ensure_page(s->h_global_page_table, s->h_global_slot_logical_pages, gc,
                                b, pos);
    s->h_token_batch[b] = b;
    s->h_token_position[b] = pos;
    const size_t si = (size_t)b * sc.max_pages_per_seq + (pos / sc.page_size) % sc.max_pages_per_seq;
    const size_t gi = (size_t)b * gc.max_pages_per_seq + (pos / gc.page_size) % gc.max_pages_per_seq;
    if (e == hipSuccess) e = upload(s->sliding_page_table + si, &s->h_sliding_page_table[si], 1, stream);
    if (e == hipSuccess) e = upload(s->global_page_table + gi, &s->h_global_page_table[gi], 1, stream);
    if (e == hipSuccess)
      e = upload(s->sliding_slot_logical_pages + si, &s->h_sliding_slot_logical_pages[si], 1, stream);
    if (e == hipSuccess)
      e = upload(s->global_slot_logical_pages + gi, &s->h_global_slot_logical_pages[gi], 1, stream);
  }
  for (int32_t b = 0; b < s->batch_size; ++b) ++s->h_seq_lengths[b];
  s->token_count = s->batch_size;
  if (e == hipSuccess) e = upload(s->seq_lengths, s->h_seq_lengths.data(), s->h_seq_lengths.size(), stream);
  if (e == hipSuccess) e = upload(s->token_batch, s->h_token_batch.data(), (size_t)s->batch_size, stream);
  if (e == hipSuccess) e = upload(s->token_position, s->h_token_position.data(), (size_t)s->batch_size, stream);
  return e;
}

// ---- opaque-handle C-ABI -------------------------------------------------------

struct Gemma4Runtime {
  Gemma4RuntimeState state;
};

hipError_t gemma4_runtime_prepare_decode_walk(Gemma4RuntimeState *s, int32_t steps,
                                              hipStream_t stream) {
  if (s == nullptr || steps < 1) return hipErrorInvalidValue;
  if (s->host_stale) {
    const hipError_t se = gemma4_runtime_sync_host(s, stream);
    if (se != hipSuccess) return se;
  }
  const Gemma4KvCacheConfig &sc = s->sliding_cache_config;
  const Gemma4KvCacheConfig &gc = s->global_cache_config;
  // Every step of every sequence is mapped on copies first, so a refused
  // walk leaves the state as it was (the per-step checks of
  // gemma4_runtime_prepare_decode_step, applied to each position in order).
  std::vector<int32_t> spt = s->h_sliding_page_table, sslot = s->h_sliding_slot_logical_pages;
  std::vector<int32_t> gpt = s->h_global_page_table, gslot = s->h_global_slot_logical_pages;
  std::vector<int32_t> before(s->h_seq_lengths.begin(), s->h_seq_lengths.begin() + s->batch_size);
  for (int32_t b = 0; b < s->batch_size; ++b) {
    const int32_t pos0 = before[b];
    if (pos0 < 0 || (int64_t)pos0 + steps > s->max_seq_len) return hipErrorInvalidValue;
    for (int32_t t = 0; t < steps; ++t) {
      if (gemma4_kv_cache_ensure_page(spt, sslot, sc, b, pos0 + t) < 0 ||
          gemma4_kv_cache_ensure_page(gpt, gslot, gc, b, pos0 + t) < 0)
        return hipErrorInvalidValue;
    }
  }
  s->h_sliding_page_table.swap(spt);
  s->h_sliding_slot_logical_pages.swap(sslot);
  s->h_global_page_table.swap(gpt);
  s->h_global_slot_logical_pages.swap(gslot);
  for (int32_t b = 0; b < s->batch_size; ++b) {
    s->h_token_batch[b] = b;
    s->h_token_position[b] = before[b] + steps - 1;
    s->h_seq_lengths[b] = before[b] + steps;
  }
  s->token_count = s->batch_size;
  hipError_t e = upload(s->sliding_page_table, s->h_sliding_page_table.data(),
                        s->h_sliding_page_table.size(), stream);
  if (e == hipSuccess)
    e = upload(s->global_page_table, s->h_global_page_table.data(), s->h_global_page_table.size(),
               stream);
  if (e == hipSuccess)
    e = upload(s->sliding_slot_logical_pages, s->h_sliding_slot_logical_pages.data(),
               s->h_sliding_slot_logical_pages.size(), stream);
  if (e == hipSuccess)
    e = upload(s->global_slot_logical_pages, s->h_global_slot_logical_pages.data(),
               s->h_global_slot_logical_pages.size(), stream);
  if (e == hipSuccess)
    e = upload(s->token_batch, s->h_token_batch.data(), (size_t)s->batch_size, stream);
  // The device lengths stay at their values before the walk, which is what
  // the walk reads (it leaves the last step's lengths and positions).
  if (e == hipSuccess) e = upload(s->seq_lengths, before.data(), before.size(), stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);  // `before` is a local
  return e;
}

extern "C" {

hipError_t gemma4_runtime_decode_walk(Gemma4Runtime *rt, int32_t steps, hipStream_t stream) {
  return rt == nullptr ? hipErrorInvalidValue
                       : gemma4_runtime_prepare_decode_walk(&rt->state, steps, stream);
}

hipError_t gemma4_runtime_create(Gemma4Runtime **out, int32_t batch_size, int32_t max_seq_len,
                                 int32_t page_size, hipStream_t stream) {
  if (out == nullptr) return hipErrorInvalidValue;
  *out = nullptr;
  Gemma4Runtime *rt = new (std::nothrow) Gemma4Runtime();
  if (rt == nullptr) return hipErrorOutOfMemory;
  const hipError_t e = gemma4_runtime_state_init(&rt->state, batch_size, max_seq_len, page_size, stream);
  if (e != hipSuccess) {
    delete rt;
    return e;
  }
  *out = rt;
  return hipSuccess;
}

void gemma4_runtime_destroy(Gemma4Runtime *rt) {
  if (rt == nullptr) return;
  gemma4_runtime_state_free(&rt->state);
  delete rt;
}

hipError_t gemma4_runtime_prefill(Gemma4Runtime *rt, int32_t seq_len, hipStream_t stream) {
  return rt == nullptr ? hipErrorInvalidValue
                       : gemma4_runtime_prepare_prefill(&rt->state, seq_len, stream);
}

hipError_t gemma4_runtime_decode_step(Gemma4Runtime *rt, hipStream_t stream) {
  return rt == nullptr ? hipErrorInvalidValue
                       : gemma4_runtime_prepare_decode_step(&rt->state, stream);
}

hipError_t gemma4_runtime_decode_step_device(Gemma4Runtime *rt, hipStream_t stream) {
  return rt == nullptr ? hipErrorInvalidValue
                       : gemma4_runtime_prepare_decode_step_device(&rt->state, stream);
}

hipError_t gemma4_runtime_sync_host_state(Gemma4Runtime *rt, hipStream_t stream) {
  return rt == nullptr ? hipErrorInvalidValue : gemma4_runtime_sync_host(&rt->state, stream);
}

hipError_t gemma4_runtime_get_device_step_status(const Gemma4Runtime *rt, int32_t *status) {
  return rt == nullptr ? hipErrorInvalidValue
                       : gemma4_runtime_device_step_status(&rt->state, status);
}

hipError_t gemma4_runtime_get_config(const Gemma4Runtime *rt, int32_t which,
                                     Gemma4KvCacheConfig *out) {
  if (rt == nullptr || out == nullptr || which < 0 || which > 1) return hipErrorInvalidValue;
  *out = which == 0 ? rt->state.sliding_cache_config : rt->state.global_cache_config;
  return hipSuccess;
}

hipError_t gemma4_runtime_get_scalars(const Gemma4Runtime *rt, int32_t *out4) {
  if (rt == nullptr || out4 == nullptr) return hipErrorInvalidValue;
  out4[0] = rt->state.batch_size;
  out4[1] = rt->state.max_seq_len;
  out4[2] = rt->state.page_size;
  out4[3] = rt->state.token_count;
  return hipSuccess;
}

static const std::vector<int32_t> *host_vector(const Gemma4RuntimeState &s, int32_t which) {
  switch (which) {
    case 0: return &s.h_sliding_page_table;
    case 1: return &s.h_global_page_table;
    case 2: return &s.h_sliding_slot_logical_pages;
    case 3: return &s.h_global_slot_logical_pages;
    case 4: return &s.h_seq_lengths;
    case 5: return &s.h_token_batch;
    case 6: return &s.h_token_position;
    default: return nullptr;
  }
}

hipError_t gemma4_runtime_get_host_vector(const Gemma4Runtime *rt, int32_t which, int32_t *dst,
                                          int64_t capacity, int64_t *size) {
  if (rt == nullptr) return hipErrorInvalidValue;
  const std::vector<int32_t> *v = host_vector(rt->state, which);
  if (v == nullptr || capacity < 0 || (capacity > 0 && dst == nullptr)) return hipErrorInvalidValue;
  const int64_t n = std::min<int64_t>(capacity, (int64_t)v->size());
  std::copy(v->begin(), v->begin() + n, dst);
  if (size != nullptr) *size = (int64_t)v->size();
  return hipSuccess;
}

hipError_t gemma4_runtime_set_host_seq_lengths(Gemma4Runtime *rt, const int32_t *src,
                                               int64_t count) {
  if (rt == nullptr || src == nullptr || count != (int64_t)rt->state.h_seq_lengths.size()) {
    return hipErrorInvalidValue;
  }
  std::copy(src, src + count, rt->state.h_seq_lengths.begin());
  return hipSuccess;
}

void *gemma4_runtime_device_ptr(const Gemma4Runtime *rt, int32_t which) {
  if (rt == nullptr) return nullptr;
  const Gemma4RuntimeState &s = rt->state;
  void *const ptrs[] = {s.sliding_cache_k, s.sliding_cache_v, s.global_cache_k, s.global_cache_v,
                        s.sliding_page_table, s.global_page_table, s.seq_lengths,
                        s.token_batch, s.token_position, s.sliding_cos, s.sliding_sin,
                        s.global_cos, s.global_sin, s.sliding_slot_logical_pages,
                        s.global_slot_logical_pages};
  if (which < 0 || which >= (int32_t)(sizeof(ptrs) / sizeof(ptrs[0]))) return nullptr;
  return ptrs[which];
}

}  // extern "C"
