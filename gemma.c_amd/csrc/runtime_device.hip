// Device-side decode-step preparation (gfx950): the bookkeeping of
// gemma4_runtime_prepare_decode_step (src/gemma4_runtime.cu:276-341) done by
// one small kernel on the stream, so a decode loop needs no host round trip
// and no H2D copies per step (the reference plans this in TODO.md:7).
//
// One workgroup. Every thread checks its sequences first: the position
// (the old seq_len) must be below max_seq_len and neither ring slot may hold
// a newer logical page (the rule of gemma4_kv_cache_ensure_page,
// src/gemma4_kv_cache.cu:108-123). Only if every sequence passes
// (__syncthreads_and) does any thread write: the ring slot gets its identity
// physical page and logical page, token_batch/token_position get the
// sequence and its position, seq_lengths advances. A refused step writes
// nothing but the status word.
#include <hip/hip_runtime.h>

#include "gemma4_runtime.h"

namespace {

constexpr int kStepThreads = 256;

struct DeviceStepParams {
  int32_t *sliding_page_table;
  int32_t *global_page_table;
  int32_t *sliding_slots;   // logical page held by each ring slot
  int32_t *global_slots;
  int32_t *seq_lengths;
  int32_t *token_batch;
  int32_t *token_position;
  int32_t *status;
  Gemma4KvCacheConfig sliding;
  Gemma4KvCacheConfig global;
  int32_t batch_size;
  int32_t max_seq_len;
};

// Index of the slot that holds `position`'s page, and its logical page.
__device__ __forceinline__ int64_t slot_index(const Gemma4KvCacheConfig &c, int32_t batch,
                                              int32_t position, int32_t *logical) {
  *logical = position / c.page_size;
  return (int64_t)batch * c.max_pages_per_seq + *logical % c.max_pages_per_seq;
}

__global__ __launch_bounds__(kStepThreads) void runtime_decode_step_kernel(DeviceStepParams p) {
  bool ok = true;
  for (int32_t b = threadIdx.x; b < p.batch_size; b += kStepThreads) {
    const int32_t pos = p.seq_lengths[b];
    if (pos < 0 || pos >= p.max_seq_len) {
      ok = false;
      continue;
    }
    int32_t slp, glp;
    const int64_t si = slot_index(p.sliding, b, pos, &slp);
    const int64_t gi = slot_index(p.global, b, pos, &glp);
    ok = ok && p.sliding_slots[si] <= slp && p.global_slots[gi] <= glp;
  }
  if (!__syncthreads_and(ok)) {
    if (threadIdx.x == 0) p.status[0] = 1;
    return;
  }
  for (int32_t b = threadIdx.x; b < p.batch_size; b += kStepThreads) {
    const int32_t pos = p.seq_lengths[b];
    int32_t slp, glp;
    const int64_t si = slot_index(p.sliding, b, pos, &slp);
    const int64_t gi = slot_index(p.global, b, pos, &glp);
    p.sliding_page_table[si] = (int32_t)si;  // physical = batch * max_pages + slot
    p.sliding_slots[si] = slp;
    p.global_page_table[gi] = (int32_t)gi;
    p.global_slots[gi] = glp;
    p.token_batch[b] = b;
    p.token_position[b] = pos;
    p.seq_lengths[b] = pos + 1;
  }
  if (threadIdx.x == 0) p.status[0] = 0;
}

}  // namespace

hipError_t gemma4_runtime_prepare_decode_step_device(Gemma4RuntimeState *s, hipStream_t stream) {
  if (s == nullptr || s->batch_size <= 0 || s->seq_lengths == nullptr ||
      s->sliding_slot_logical_pages == nullptr || s->global_slot_logical_pages == nullptr ||
      s->device_step_status == nullptr) {
    return hipErrorInvalidValue;
  }
  DeviceStepParams p{};
  p.sliding_page_table = s->sliding_page_table;
  p.global_page_table = s->global_page_table;
  p.sliding_slots = s->sliding_slot_logical_pages;
  p.global_slots = s->global_slot_logical_pages;
  p.seq_lengths = s->seq_lengths;
  p.token_batch = s->token_batch;
  p.token_position = s->token_position;
  p.status = s->device_step_status;
  p.sliding = s->sliding_cache_config;
  p.global = s->global_cache_config;
  p.batch_size = s->batch_size;
  p.max_seq_len = s->max_seq_len;
  hipLaunchKernelGGL(runtime_decode_step_kernel, dim3(1), dim3(kStepThreads), 0, stream, p);
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) {
    s->token_count = s->batch_size;  // a decode step's rows, applied or refused
    s->host_stale = true;
  }
  return e;
}
