// Wave64 reduction helpers, cache-row lookups and device-coherent accesses
// shared by the decode-attention kernels (per-layer split kernel and the
// persistent layer-walking kernel).
#pragma once

#include "gemma4_device.hpp"
#include "gemma4_kv_cache.h"

namespace gemma4 {

// Arguments of the split-K decode kernels (decode_attention.hip).
struct DecodeParams {
  uint16_t *out;
  float *partial_m;
  float *partial_l;
  float *partial_acc;
  const uint16_t *q;
  uint16_t *cache_k;  // written only by the fused append
  uint16_t *cache_v;
  const int32_t *page_table;
  const int32_t *seq_lengths;
  const int32_t *token_position;  // null: no append
  int32_t *counters;              // null: separate combine kernel
  const uint16_t *new_k;
  const uint16_t *new_v;
  // Fused preparation (null q_norm_weight: q and the new K/V come prepared).
  const uint16_t *q_norm_weight;
  const uint16_t *k_norm_weight;
  const float *cos;              // [position][rotary / 2]
  const float *sin;
  Gemma4KvCacheConfig c;
  int32_t layer;
  float q_scale;  // softmax_scale * log2(e)
  int32_t split_size;
  int32_t num_splits;
  // Non-null (persistent decode step only): a nonzero word here turns the
  // launch into zeros for its output rows, with no append.
  const int32_t *gate;
  // Nonzero: a full ring may be split by ring slot rather than by position
  // (the partials are internal to the launch).
  int32_t slot_splits = 0;
};

constexpr int kRowInvalid = -1;   // key outside the split or unmapped page
constexpr int kRowNewToken = -2;  // key being appended in this launch

// Value-splitting butterfly: N partial values per lane are summed over the
// 2*O lanes of a group (bit O first, down to bit 1); each exchange sends the
// half of the values the partner keeps, so after log2(N) steps every lane
// carries one fully reduced value, whose index is given by the lane bits
// [log2(O*2/N), log2(O)]. Remaining offsets are plain all-reduce steps (the
// value then repeats across those low lanes).
template <int N, int O>
__device__ __forceinline__ void split_butterfly(float *v, int lane) {
  if constexpr (N > 1 && (O == 32 || O == 16)) {
    // One VALU swap per pair leaves each lane exactly its two addends.
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      float x, y;
      swap_halves<O>(v[i], v[i + N / 2], x, y);
      v[i] = x + y;
    }
    split_butterfly<N / 2, O / 2>(v, lane);
  } else if constexpr (N > 1) {
    const bool hi = (lane & O) != 0;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const float send = hi ? v[i] : v[i + N / 2];
      const float keep = hi ? v[i + N / 2] : v[i];
      v[i] = keep + lane_pair<O>(send);
    }
    split_butterfly<N / 2, O / 2>(v, lane);
  } else if constexpr (O == 32 || O == 16) {
    v[0] = xor_sum<O>(v[0]);
    split_butterfly<1, O / 2>(v, lane);
  } else if constexpr (O >= 1) {
    v[0] += lane_pair<O>(v[0]);
    split_butterfly<1, O / 2>(v, lane);
  }
}

// Max / sum of one value over all lanes that differ only in lane bits at or
// above kFrom (lower bits select duplicates or another GQA head).
template <int kFrom>
__device__ __forceinline__ float reduce_max_from(float v) {
  if constexpr (kFrom < kWave) {
    v = xor_max<kFrom>(v);
    return reduce_max_from<kFrom * 2>(v);
  } else {
    return v;
  }
}
template <int kFrom>
__device__ __forceinline__ float reduce_sum_from(float v) {
  if constexpr (kFrom < kWave) {
    v = xor_sum<kFrom>(v);
    return reduce_sum_from<kFrom * 2>(v);
  } else {
    return v;
  }
}

// Collect a per-head value held by the lanes of head `my_g` into out[g] for
// every head g of the wave (lanes of head g differ in bits [S, S+GB)).
template <int GW, int S, int D = 1>
__device__ __forceinline__ void gather_other(float mine, float (&other)[GW]) {
  if constexpr (D < GW) {
    other[D] = lane_xor<(D << S)>(mine);
    gather_other<GW, S, D + 1>(mine, other);
  }
}
template <int GW, int S>
__device__ __forceinline__ void gather_heads(float mine, int my_g, float (&out)[GW]) {
  float other[GW];
  other[0] = mine;
  gather_other<GW, S>(mine, other);
#pragma unroll
  for (int g = 0; g < GW; ++g) {
    const int d = my_g ^ g;
    float v = other[0];
#pragma unroll
    for (int dd = 1; dd < GW; ++dd) v = (d == dd) ? other[dd] : v;
    out[g] = v;
  }
}

// Sum over the RPL key rows of a load (lane bits >= LPR).
template <int LPR>
__device__ __forceinline__ float sum_rows(float v) {
  if constexpr (LPR < kWave) {
    v = xor_sum<LPR>(v);
    return sum_rows<LPR * 2>(v);
  } else {
    return v;
  }
}

__device__ __forceinline__ void wave_lds_sync() {
  // LDS operations of one wave complete in issue order; this only stops the
  // compiler from moving LDS accesses across the exchange point.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Cache row index of `key` for sequence `b`, or kRowInvalid for an unmapped
// page (src/gemma4_flash_attention_decode.cu:791-805).
__device__ __forceinline__ int32_t key_row(const Gemma4KvCacheConfig &c,
                                           const int32_t *__restrict__ page_table,
                                           int32_t layer, int32_t b, int32_t key) {
  const int32_t logical_page = key / c.page_size;
  const int32_t slot = logical_page % c.max_pages_per_seq;
  const int32_t physical = page_table[b * c.max_pages_per_seq + slot];
  if (physical < 0 || physical >= c.num_pages) return kRowInvalid;
  const int32_t page_offset = key - logical_page * c.page_size;
  return ((int32_t)layer * c.num_pages + physical) * c.page_size + page_offset;
}

// Cache row the fused append writes for (b, position), or -1 when the
// reference skip rules drop it (src/gemma4_kv_cache.cu:25-34).
__device__ __forceinline__ int32_t append_row(const Gemma4KvCacheConfig &c,
                                              const int32_t *__restrict__ page_table,
                                              int32_t layer, int32_t b, int32_t position) {
  if (position < 0 || b >= c.batch_size) return -1;
  const int32_t logical_page = position / c.page_size;
  if (c.window_size == 0 && logical_page >= c.max_pages_per_seq) return -1;
  return key_row(c, page_table, layer, b, position);
}

// Device-coherent (sc1) accesses for data exchanged between workgroups of
// one launch: they bypass the per-XCD L2 write-back state, so no whole-cache
// maintenance is needed (agent-scope relaxed atomics compile to the same).
constexpr int kCoherentAux = 16;  // cache-policy bit sc1
__device__ __forceinline__ void coherent_store(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
using u32x4 = __attribute__((ext_vector_type(4))) unsigned;
// 8 floats at byte offset `off` (per lane) from the wave-uniform `base`: a
// buffer descriptor must be uniform, or the compiler loops over the lanes.
__device__ __forceinline__ void coherent_store8(float *base, int32_t off, const float (&v)[8]) {
  const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7fffffff, 0x00020000);
  const u32x4 lo = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                    __float_as_uint(v[3])};
  const u32x4 hi = {__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                    __float_as_uint(v[7])};
  __builtin_amdgcn_raw_buffer_store_b128(lo, rsrc, off, 0, kCoherentAux);
  __builtin_amdgcn_raw_buffer_store_b128(hi, rsrc, off + 16, 0, kCoherentAux);
}
// Wait until this thread's outstanding memory operations have completed
// (the signal fences keep the compiler from moving memory accesses across).
__device__ __forceinline__ void wait_stores_complete() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Buffer view of `count` floats for coherent loads; out-of-range loads read 0.
__device__ __forceinline__ auto coherent_view(const float *p, int32_t count) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(p), 0, count * 4, 0x00020000);
}

// Whether a decode entry point accepts this cache geometry, cache layer,
// batch and split plan (the checks decode_entry makes before any launch).
bool decode_geometry_ok(const Gemma4KvCacheConfig &c, int32_t layer, int32_t batch_count,
                        int32_t split_size, int32_t num_splits);

// The fused append + split-K decode with the separate combine
// (decode_attention.hip) for the persistent step's 1 x 512 global layers:
// while the word at `gate` (the step workspace's status) is nonzero the
// launches append nothing and write zeros to `out`.
hipError_t decode_append_gated(uint16_t *out, float *pm, float *pl, float *pacc,
                               const uint16_t *q, uint16_t *cache_k, uint16_t *cache_v,
                               const int32_t *page_table, const int32_t *seq_lengths,
                               const int32_t *token_position, const uint16_t *new_k,
                               const uint16_t *new_v, const Gemma4KvCacheConfig &c,
                               int32_t layer, float softmax_scale, int32_t split_size,
                               int32_t num_splits, int32_t batch_count, const int32_t *gate,
                               hipStream_t stream, const uint16_t *q_norm_weight = nullptr,
                               const uint16_t *k_norm_weight = nullptr,
                               const float *cos = nullptr, const float *sin = nullptr);

}  // namespace gemma4
