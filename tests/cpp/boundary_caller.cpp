// A C++ caller of the drop-in boundary written the way gemma.c's own sources
// call the reference API (src/gemma4_kv_cache.cuh:20-53,
// src/gemma4_runtime.cuh:45-64, src/gemma4_flash_attention.cuh:9-45), with
// HIP types in place of the CUDA ones. It must compile against include/*.h
// unchanged, link against libgemma4_kv.so, and (host-only functions, no GPU
// needed) return 0. Built and run by tests/test_cpp_boundary.py.
#include <hip/hip_bf16.h>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <vector>

#include "gemma4_attention_output.h"
#include "gemma4_flash_attention.h"
#include "gemma4_kv_cache.h"
#include "gemma4_runtime.h"

namespace {

// The offset is usable in constant expressions, as the reference's
// __host__ __device__ constexpr one is (src/gemma4_kv_cache.cuh:28-38).
constexpr Gemma4KvCacheConfig kCfg = {3, 10, 16, 5, 2, 8, 256, 1024};
static_assert(gemma4_kv_cache_offset(kCfg, 0, 0, 0, 0, 0) == 0, "origin");
static_assert(gemma4_kv_cache_offset(kCfg, 0, 0, 0, 0, 1) == 1, "dim stride");
static_assert(gemma4_kv_cache_offset(kCfg, 0, 0, 0, 1, 0) == 256, "head stride");
static_assert(gemma4_kv_cache_offset(kCfg, 0, 0, 1, 0, 0) == 8 * 256, "token stride");
static_assert(gemma4_kv_cache_offset(kCfg, 0, 1, 0, 0, 0) == 16 * 8 * 256, "page stride");
static_assert(gemma4_kv_cache_offset(kCfg, 1, 0, 0, 0, 0) == 10LL * 16 * 8 * 256, "layer");
static_assert(gemma4_kv_cache_offset(kCfg, 2, 9, 15, 7, 255) ==
                  3LL * 10 * 16 * 8 * 256 - 1, "last element");

// The reference's entry points, as function pointers of the reference's
// parameter lists (CUDA types -> HIP types): a declaration that differs in
// any parameter does not convert.
using WriteFn = hipError_t (*)(__hip_bfloat16 *, __hip_bfloat16 *, Gemma4KvCacheConfig,
                               const int32_t *, const int32_t *, const int32_t *, int32_t,
                               int32_t, const __hip_bfloat16 *, const __hip_bfloat16 *,
                               hipStream_t);
using SlidingFwdFn = hipError_t (*)(__hip_bfloat16 *, __hip_bfloat16 *, __hip_bfloat16 *,
                                    __hip_bfloat16 *, const __hip_bfloat16 *,
                                    const __hip_bfloat16 *, const __hip_bfloat16 *,
                                    const __hip_bfloat16 *, const __hip_bfloat16 *,
                                    const float *, const float *, const int32_t *, int, int,
                                    int, int, float, hipStream_t);
using GlobalFwdFn = hipError_t (*)(__hip_bfloat16 *, __hip_bfloat16 *, __hip_bfloat16 *,
                                   __hip_bfloat16 *, const __hip_bfloat16 *,
                                   const __hip_bfloat16 *, const __hip_bfloat16 *,
                                   const __hip_bfloat16 *, const float *, const float *,
                                   const int32_t *, int, int, int, float, hipStream_t);
using StateInitFn = hipError_t (*)(Gemma4RuntimeState *, int32_t, int32_t, int32_t,
                                   hipStream_t);
using StateFreeFn = void (*)(Gemma4RuntimeState *);
using PrefillFn = hipError_t (*)(Gemma4RuntimeState *, int32_t, hipStream_t);
using DecodeStepFn = hipError_t (*)(Gemma4RuntimeState *, hipStream_t);

int failures = 0;
void expect(bool ok, const char *what) {
  if (!ok) {
    std::printf("FAIL: %s\n", what);
    ++failures;
  }
}

}  // namespace

int main() {
  const WriteFn write = gemma4_kv_cache_write_bf16;
  const SlidingFwdFn sliding = gemma4_flash_attention_sliding_fwd_bf16_norm_rope;
  const GlobalFwdFn global = gemma4_flash_attention_global_fwd_bf16_norm_rope;
  const StateInitFn init = gemma4_runtime_state_init;
  const StateFreeFn release = gemma4_runtime_state_free;
  const PrefillFn prefill = gemma4_runtime_prepare_prefill;
  const DecodeStepFn step = gemma4_runtime_prepare_decode_step;
  expect(write && sliding && global && init && release && prefill && step, "entry points");

  // Argument checks run on the host before any launch (no GPU needed).
  expect(write(nullptr, nullptr, kCfg, nullptr, nullptr, nullptr, 1, 0, nullptr, nullptr,
               nullptr) == hipErrorInvalidValue, "write rejects null pointers");

  // src/gemma4_kv_cache.cu:76-91 with the model constants of src/gemma4.h.
  const Gemma4KvCacheConfig s = gemma4_kv_cache_make_config(false, 64, 16, 65);
  const Gemma4KvCacheConfig g = gemma4_kv_cache_make_config(true, 256, 16, 128);
  expect(s.num_layers == 40 && s.num_heads == 8 && s.head_dim == 256 && s.window_size == 1024 &&
             s.batch_size == 0 && s.page_size == 16,
         "sliding config");
  expect(g.num_layers == 8 && g.num_heads == 1 && g.head_dim == 512 && g.window_size == 0 &&
             g.batch_size == 2,
         "global config");

  // src/gemma4_kv_cache.cu:94-105: the 5:1 cadence, last layer global.
  int sliding_seen = 0, global_seen = 0;
  for (int32_t l = 0; l < 48; ++l) {
    const bool is_global = l == 47 || (l + 1) % 6 == 0;
    const int32_t si = gemma4_kv_cache_layer_index(l, false);
    const int32_t gi = gemma4_kv_cache_layer_index(l, true);
    expect(is_global ? (si == -1 && gi == global_seen++) : (gi == -1 && si == sliding_seen++),
           "layer index");
  }
  expect(sliding_seen == 40 && global_seen == 8, "layer counts");

  // std::vector ring bookkeeping, as gemma4_runtime.cu calls it: a 4-slot
  // ring of page 2 for 2 sequences.
  Gemma4KvCacheConfig r = gemma4_kv_cache_make_config(false, 8, 2, 4);
  r.batch_size = 2;
  std::vector<int32_t> table(8, -1), slots(8, -1);
  expect(gemma4_kv_cache_ensure_range(table, slots, r, 1, 0, 8) == 0, "range fills the ring");
  expect(table[4] == 4 && table[7] == 7 && slots[7] == 3, "ring slots of sequence 1");
  expect(gemma4_kv_cache_ensure_page(table, slots, r, 1, 9) == 4, "wrap reuses slot 0");
  expect(slots[4] == 4, "slot 0 now holds logical page 4");
  expect(gemma4_kv_cache_ensure_page(table, slots, r, 1, 1) == -1, "older page refused");
  expect(table[0] == -1 && slots[0] == -1, "sequence 0 untouched");

  // A zero-initialised runtime state frees as a no-op.
  Gemma4RuntimeState state;
  expect(state.sliding_cache_k == nullptr && state.h_seq_lengths.empty(), "state defaults");

  if (failures == 0) std::printf("boundary caller ok\n");
  return failures == 0 ? 0 : 1;
}
