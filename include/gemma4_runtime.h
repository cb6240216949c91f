// Runtime state of the KV-cache path: cache allocation, page tables, sequence
// lengths and the per-step token metadata, MI355X (gfx950) build.
//
// Drop-in for src/gemma4_runtime.cuh: same struct fields and functions
// (CUDA types replaced by HIP ones), plus an opaque-handle C-ABI for FFI
// callers that cannot use the C++ struct with its std::vector members.
#pragma once

#include "gemma4_kv_cache.h"

#ifdef __cplusplus
#include <vector>

// Replaces src/gemma4_runtime.cuh:12-43.
struct Gemma4RuntimeState {
  int32_t batch_size = 0;
  int32_t max_seq_len = 0;
  int32_t page_size = 0;
  int32_t token_count = 0;

  Gemma4KvCacheConfig sliding_cache_config = {};
  Gemma4KvCacheConfig global_cache_config = {};
  gemma4_bf16 *sliding_cache_k = nullptr;
  gemma4_bf16 *sliding_cache_v = nullptr;
  gemma4_bf16 *global_cache_k = nullptr;
  gemma4_bf16 *global_cache_v = nullptr;

  int32_t *sliding_page_table = nullptr;
  int32_t *global_page_table = nullptr;
  int32_t *seq_lengths = nullptr;
  int32_t *token_batch = nullptr;
  int32_t *token_position = nullptr;
  float *sliding_cos = nullptr;
  float *sliding_sin = nullptr;
  float *global_cos = nullptr;
  float *global_sin = nullptr;

  std::vector<int32_t> h_sliding_page_table;
  std::vector<int32_t> h_global_page_table;
  std::vector<int32_t> h_sliding_slot_logical_pages;
  std::vector<int32_t> h_global_slot_logical_pages;
  std::vector<int32_t> h_seq_lengths;
  std::vector<int32_t> h_token_batch;
  std::vector<int32_t> h_token_position;

  // Extensions of this build (not in the reference struct): device copies of
  // the ring bookkeeping for the device-side decode step, its status word,
  // and whether device metadata is ahead of the host vectors.
  int32_t *sliding_slot_logical_pages = nullptr;
  int32_t *global_slot_logical_pages = nullptr;
  int32_t *device_step_status = nullptr;
  bool host_stale = false;
};

// Replaces src/gemma4_runtime.cuh:45-64 (src/gemma4_runtime.cu:95-341).
// Allocates caches, page tables, token metadata and RoPE tables; `state`
// must be zero-initialized or freed. A failed call frees what it allocated.
hipError_t gemma4_runtime_state_init(Gemma4RuntimeState *state, int32_t batch_size,
                                     int32_t max_seq_len, int32_t page_size,
                                     hipStream_t stream);
void gemma4_runtime_state_free(Gemma4RuntimeState *state);
// Page tables and absolute token positions for an initial prompt of
// `seq_len` tokens per sequence (rows batch-major).
hipError_t gemma4_runtime_prepare_prefill(Gemma4RuntimeState *state, int32_t seq_len,
                                          hipStream_t stream);
// Appends one decode position per sequence: validates every sequence before
// mutating anything, maps the ring slots, advances seq_lengths and uploads
// the changed metadata.
hipError_t gemma4_runtime_prepare_decode_step(Gemma4RuntimeState *state,
                                              hipStream_t stream);
// Device-side decode step (no counterpart in the reference; it removes the
// per-step host bookkeeping and H2D copies, as the reference's TODO.md:7
// plans): one kernel validates every sequence (position < max_seq_len, no
// ring slot holding a newer logical page) and, only if all pass, maps the
// ring slots, writes token_batch/token_position and advances seq_lengths on
// the device. Stream-ordered and asynchronous: a refused step changes
// nothing and sets the device status word to 1 (0 after an applied step),
// read with gemma4_runtime_device_step_status. The host vectors are then
// stale until gemma4_runtime_sync_host (the host prepare_* functions sync
// first by themselves).
hipError_t gemma4_runtime_prepare_decode_step_device(Gemma4RuntimeState *state,
                                                     hipStream_t stream);
// Metadata for a persistent walk of `steps` decode steps
// (gemma4_decode_walk_bf16; no counterpart in the reference, whose loop
// prepares one step at a time with gemma4_runtime_prepare_decode_step):
// validates every step of every sequence before mutating anything, maps the
// ring slots of all `steps` positions, uploads the page tables, and leaves
// the host vectors as after the last step. The device seq_lengths hold the
// lengths before the walk, which the walk advances itself; run the walk next
// in the same stream. Synchronises `stream` once.
hipError_t gemma4_runtime_prepare_decode_walk(Gemma4RuntimeState *state, int32_t steps,
                                              hipStream_t stream);
// Copies the device metadata into the host vectors (synchronous).
hipError_t gemma4_runtime_sync_host(Gemma4RuntimeState *state, hipStream_t stream);
// Status of the last device-side step (synchronous read): 0 applied, 1 refused.
hipError_t gemma4_runtime_device_step_status(const Gemma4RuntimeState *state,
                                             int32_t *status);
extern "C" {
#endif

// Opaque-handle form for C / FFI callers. The handle owns a
// Gemma4RuntimeState; accessors copy host metadata out and return device
// pointers (cast to void*). All return hipError_t except the pointer getter.
typedef struct Gemma4Runtime Gemma4Runtime;
hipError_t gemma4_runtime_create(Gemma4Runtime **out, int32_t batch_size,
                                 int32_t max_seq_len, int32_t page_size,
                                 hipStream_t stream);
void gemma4_runtime_destroy(Gemma4Runtime *rt);
hipError_t gemma4_runtime_prefill(Gemma4Runtime *rt, int32_t seq_len, hipStream_t stream);
hipError_t gemma4_runtime_decode_step(Gemma4Runtime *rt, hipStream_t stream);
// Handle forms of the device-side step, the host sync and the status read
// (no counterparts in the reference; see the C++ functions above).
hipError_t gemma4_runtime_decode_step_device(Gemma4Runtime *rt, hipStream_t stream);
hipError_t gemma4_runtime_decode_walk(Gemma4Runtime *rt, int32_t steps, hipStream_t stream);
hipError_t gemma4_runtime_sync_host_state(Gemma4Runtime *rt, hipStream_t stream);
hipError_t gemma4_runtime_get_device_step_status(const Gemma4Runtime *rt, int32_t *status);
// which: 0 sliding config, 1 global config.
hipError_t gemma4_runtime_get_config(const Gemma4Runtime *rt, int32_t which,
                                     Gemma4KvCacheConfig *out);
// Scalars: batch_size, max_seq_len, page_size, token_count (4 int32).
hipError_t gemma4_runtime_get_scalars(const Gemma4Runtime *rt, int32_t *out4);
// Host vectors: 0 sliding page table, 1 global page table, 2 sliding slot
// logical pages, 3 global slot logical pages, 4 seq_lengths, 5 token_batch,
// 6 token_position. Copies min(capacity, size) entries; *size = full size.
hipError_t gemma4_runtime_get_host_vector(const Gemma4Runtime *rt, int32_t which,
                                          int32_t *dst, int64_t capacity,
                                          int64_t *size);
// Sets host seq_lengths (the reference test edits h_seq_lengths directly).
hipError_t gemma4_runtime_set_host_seq_lengths(Gemma4Runtime *rt, const int32_t *src,
                                               int64_t count);
// Device pointers: 0 sliding K, 1 sliding V, 2 global K, 3 global V,
// 4 sliding page table, 5 global page table, 6 seq_lengths, 7 token_batch,
// 8 token_position, 9 sliding cos, 10 sliding sin, 11 global cos, 12 global sin,
// 13 sliding slot logical pages, 14 global slot logical pages.
void *gemma4_runtime_device_ptr(const Gemma4Runtime *rt, int32_t which);

#ifdef __cplusplus
}  // extern "C"
#endif
