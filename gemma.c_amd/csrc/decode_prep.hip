// Decode-token preparation with the fused cache append, gfx950: learned
// RMSNorm + split-half RoPE of every query head and of the KV head's key,
// scale-free RMSNorm of the value (or, for the global geometry, of the raw
// key, which stands in for V), and the bf16 write of K and V into the paged
// cache row of the token. Replaces phase_decode_q_paged_kv_norm_rope
// (src/gemma4_flash_attention_decode.cu:285-375 with its helpers :216-283,
// src/gemma4_rope.cu:8-20, src/gemma4_rmsnorm.cu:90-101).
//
// Workgroup (kv_head, sequence); one wave per prepared head: the G query
// heads of the kv head, then K, then V (sliding geometry only); the
// per-head arithmetic is shared with the prefill prep (prep_common.hpp).
// The data per token is a few KiB, so the kernel is latency bound; it
// exists to feed the decode attention kernels prepared q rows and cache
// rows.
#include "gemma4_device.hpp"
#include "decode_common.hpp"
#include "prep_common.hpp"

#include "gemma4_flash_attention.h"

#include <math.h>

namespace gemma4 {
namespace {

struct PrepParams {
  uint16_t *q_prepared;
  uint16_t *cache_k;
  uint16_t *cache_v;
  const int32_t *page_table;
  const int32_t *token_position;
  const uint16_t *q;
  const uint16_t *k;
  const uint16_t *v;
  const uint16_t *q_norm_weight;
  const uint16_t *k_norm_weight;
  const float *cos;
  const float *sin;
  Gemma4KvCacheConfig c;
  int32_t layer;
};

template <int kHeads, int kDim, int kRotary, bool kHasV>
__global__ __launch_bounds__((prep_waves<kHeads, kHasV>() * kWave)) void decode_prep_append_kernel(
    PrepParams p) {
  constexpr int kGroup = kQueryHeads / kHeads;
  constexpr int kPer = kDim / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = wave_uniform(threadIdx.x / kWave);
  const int32_t head = blockIdx.x;
  const int32_t b = blockIdx.y;
  const int32_t position = wave_uniform(p.token_position[b]);
  if (position < 0) return;  // src/gemma4_flash_attention_decode.cu:331
  const float *cos_row = p.cos + (int64_t)position * (kRotary / 2);
  const float *sin_row = p.sin + (int64_t)position * (kRotary / 2);

  float x[kPer];

  if (wave < kGroup) {
    const int64_t off = ((int64_t)b * kQueryHeads + head * kGroup + wave) * kDim;
    load_head<kDim>(p.q + off, x, lane);
    store_weighted_rope<kDim, kRotary>(p.q_prepared + off, x, p.q_norm_weight, cos_row, sin_row,
                                       lane);
    if (kHasV || wave != 0) return;
  }
  const bool k_wave = kHasV ? wave == kGroup : wave == 0;
  // Cache row of the token (src/gemma4_flash_attention_decode.cu:288-303):
  // the ring slot of its page, skipped when the page is not mapped.
  const Gemma4KvCacheConfig &c = p.c;
  const int32_t logical_page = position / c.page_size;
  const int32_t slot = logical_page % c.max_pages_per_seq;
  const int32_t physical = wave_uniform(p.page_table[(int64_t)b * c.max_pages_per_seq + slot]);
  if (physical < 0 || physical >= c.num_pages) return;
  const int64_t row = ((int64_t)p.layer * c.num_pages + physical) * c.page_size +
                      (position - logical_page * c.page_size);
  const int64_t dst = (row * kHeads + head) * kDim;
  const int64_t src = ((int64_t)b * kHeads + head) * kDim;
  if (k_wave) {
    load_head<kDim>(p.k + src, x, lane);
    store_weighted_rope<kDim, kRotary>(p.cache_k + dst, x, p.k_norm_weight, cos_row, sin_row,
                                       lane);
    if constexpr (!kHasV) store_scale_free<kDim>(p.cache_v + dst, x, lane);
  } else {
    load_head<kDim>(p.v + src, x, lane);
    store_scale_free<kDim>(p.cache_v + dst, x, lane);
  }
}

}  // namespace
}  // namespace gemma4

using namespace gemma4;

extern "C" hipError_t gemma4_decode_prep_append_bf16(
    gemma4_bf16 *q_prepared, gemma4_bf16 *cache_k, gemma4_bf16 *cache_v,
    Gemma4KvCacheConfig config, const int32_t *page_table, const int32_t *token_position,
    int32_t layer, const gemma4_bf16 *q, const gemma4_bf16 *k, const gemma4_bf16 *v,
    const gemma4_bf16 *q_norm_weight, const gemma4_bf16 *k_norm_weight, const float *cos,
    const float *sin, int32_t batch_count, hipStream_t stream) {
  const bool sliding = config.num_heads == 8 && config.head_dim == 256;
  const bool global = config.num_heads == 1 && config.head_dim == 512;
  if (batch_count < 0 || !(sliding || global)) return hipErrorInvalidValue;
  if (batch_count == 0) return hipSuccess;
  if (q_prepared == nullptr || cache_k == nullptr || cache_v == nullptr || page_table == nullptr ||
      token_position == nullptr || q == nullptr || k == nullptr || (sliding && v == nullptr) ||
      q_norm_weight == nullptr || k_norm_weight == nullptr || cos == nullptr || sin == nullptr ||
      layer < 0 || layer >= config.num_layers || config.page_size <= 0 ||
      config.max_pages_per_seq <= 0 || config.num_pages <= 0 || batch_count > config.batch_size)
    return hipErrorInvalidValue;
  PrepParams p{};
  p.q_prepared = reinterpret_cast<uint16_t *>(q_prepared);
  p.cache_k = reinterpret_cast<uint16_t *>(cache_k);
  p.cache_v = reinterpret_cast<uint16_t *>(cache_v);
  p.page_table = page_table;
  p.token_position = token_position;
  p.q = reinterpret_cast<const uint16_t *>(q);
  p.k = reinterpret_cast<const uint16_t *>(k);
  p.v = reinterpret_cast<const uint16_t *>(v);
  p.q_norm_weight = reinterpret_cast<const uint16_t *>(q_norm_weight);
  p.k_norm_weight = reinterpret_cast<const uint16_t *>(k_norm_weight);
  p.cos = cos;
  p.sin = sin;
  p.c = config;
  p.layer = layer;
  if (sliding) {
    // Sliding geometry: RoPE over the whole head, V projection present
    // (src/gemma4_flash_attention_decode.cu:141-148).
    hipLaunchKernelGGL((decode_prep_append_kernel<8, 256, 256, true>), dim3(8, batch_count),
                       dim3(prep_waves<8, true>() * kWave), 0, stream, p);
  } else {
    // Global geometry: RoPE over a quarter of the head, V from raw K
    // (src/gemma4_flash_attention_decode.cu:150-157).
    hipLaunchKernelGGL((decode_prep_append_kernel<1, 512, 128, false>), dim3(1, batch_count),
                       dim3(prep_waves<1, false>() * kWave), 0, stream, p);
  }
  return hipGetLastError();
}
