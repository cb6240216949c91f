// Paged K/V cache: host geometry / ring bookkeeping and the gfx950 append
// kernel. Replaces src/gemma4_kv_cache.cu of gemma.c.
//
// Append design: the copy is flattened to one 128-bit pack per thread
// (K and V pack of the same (token, head, dim/8) slot), so a launch of any
// token count is one grid of fully coalesced 16-byte loads and stores; the
// page-table lookup and skip rules are evaluated per thread (they hit L1/L2).
#include "gemma4_device.hpp"

#include <algorithm>
#include <vector>

namespace gemma4 {
namespace {

// Reference model constants (src/gemma4.h:8-24).
constexpr int kNumLayers = 48;
constexpr int kGlobalLayerPeriod = 6;
constexpr int kGlobalLayerCount = 8;
constexpr int kSlidingLayerCount = 40;
constexpr int kSlidingKvHeads = 8;
constexpr int kGlobalKvHeads = 1;
constexpr int kSlidingHeadDim = 256;
constexpr int kGlobalHeadDim = 512;
constexpr int kSlidingWindow = 1024;

constexpr bool is_global_layer(int32_t layer) {
  return layer == kNumLayers - 1 || (layer + 1) % kGlobalLayerPeriod == 0;
}

constexpr int kAppendThreads = 256;

// Destination row of one (batch, position) in Layout-A, or -1 when the
// reference skip rules reject it (src/gemma4_kv_cache.cu:25-34).
__device__ __forceinline__ int64_t append_row(const Gemma4KvCacheConfig &c,
                                              const int32_t *__restrict__ page_table,
                                              int32_t layer, int32_t batch,
                                              int32_t position) {
  if (batch < 0 || position < 0 || batch >= c.batch_size) return -1;
  const int32_t logical_page = position / c.page_size;
  if (c.window_size == 0 && logical_page >= c.max_pages_per_seq) return -1;
  const int32_t slot = logical_page % c.max_pages_per_seq;
  const int32_t physical = page_table[batch * c.max_pages_per_seq + slot];
  if (physical < 0 || physical >= c.num_pages) return -1;
  const int32_t page_offset = position - logical_page * c.page_size;
  return ((int64_t)layer * c.num_pages + physical) * c.page_size + page_offset;
}

// One thread = one 16-byte pack of K and of V. Source rows are selected by
// `row = row_base(t)`: for plain writes t itself; for the prefill tail policy
// batch-major rows starting at `first_live` within each batch of `seq_len`.
__global__ __launch_bounds__(kAppendThreads) void kv_append_kernel(
    uint16_t *__restrict__ cache_k, uint16_t *__restrict__ cache_v,
    Gemma4KvCacheConfig c, const int32_t *__restrict__ page_table,
    const int32_t *__restrict__ token_batch,
    const int32_t *__restrict__ token_position, int32_t layer,
    const uint16_t *__restrict__ k, const uint16_t *__restrict__ v,
    int64_t total_packs, int32_t packs_per_token, int32_t rows_per_batch,
    int32_t seq_len, int32_t first_live) {
  const int64_t p = (int64_t)blockIdx.x * kAppendThreads + threadIdx.x;
  if (p >= total_packs) return;
  const int32_t t = (int32_t)(p / packs_per_token);
  const int32_t within = (int32_t)(p - (int64_t)t * packs_per_token);
  // Map the launch row to its source row (identity unless the tail policy).
  const int32_t b = t / rows_per_batch;
  const int32_t src_row = b * seq_len + first_live + (t - b * rows_per_batch);
  const int64_t dst_row = append_row(c, page_table, layer, token_batch[src_row],
                                     token_position[src_row]);
  if (dst_row < 0) return;
  const int64_t row_elems = (int64_t)c.num_heads * c.head_dim;
  const int64_t src = (int64_t)src_row * row_elems + (int64_t)within * kPackElems;
  const int64_t dst = dst_row * row_elems + (int64_t)within * kPackElems;
  const uint4 kp = load128(k + src);
  const uint4 vp = load128(v + src);
  store128(cache_k + dst, kp);
  store128(cache_v + dst, vp);
}

bool valid_append_config(const Gemma4KvCacheConfig &c, int32_t layer) {
  return layer >= 0 && layer < c.num_layers && c.num_pages > 0 &&
         c.page_size > 0 && c.max_pages_per_seq > 0 && c.batch_size > 0 &&
         c.window_size >= 0 && c.num_heads > 0 && c.head_dim > 0 &&
         c.head_dim % kPackElems == 0;
}

hipError_t launch_append(uint16_t *cache_k, uint16_t *cache_v,
                         const Gemma4KvCacheConfig &c, const int32_t *page_table,
                         const int32_t *token_batch, const int32_t *token_position,
                         int32_t rows, int32_t layer, const uint16_t *k,
                         const uint16_t *v, int32_t rows_per_batch,
                         int32_t seq_len, int32_t first_live,
                         hipStream_t stream) {
  const int32_t packs_per_token = c.num_heads * (c.head_dim / kPackElems);
  const int64_t total = (int64_t)rows * packs_per_token;
  const int64_t blocks = (total + kAppendThreads - 1) / kAppendThreads;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL(kv_append_kernel, dim3((uint32_t)blocks), dim3(kAppendThreads),
                     0, stream, cache_k, cache_v, c, page_table, token_batch,
                     token_position, layer, k, v, total, packs_per_token,
                     rows_per_batch, seq_len, first_live);
  return hipGetLastError();
}

}  // namespace
}  // namespace gemma4

using namespace gemma4;

// src/gemma4_kv_cache.cu:108-122
int32_t gemma4_kv_cache_ensure_page(std::vector<int32_t> &page_table,
                                    std::vector<int32_t> &slot_logical_pages,
                                    const Gemma4KvCacheConfig &config,
                                    int32_t batch, int32_t position) {
  return gemma4_kv_cache_ensure_page_ptr(
      page_table.data(), slot_logical_pages.data(),
      (int64_t)std::min(page_table.size(), slot_logical_pages.size()), &config,
      batch, position);
}

// src/gemma4_kv_cache.cu:125-146
int32_t gemma4_kv_cache_ensure_range(std::vector<int32_t> &page_table,
                                     std::vector<int32_t> &slot_logical_pages,
                                     const Gemma4KvCacheConfig &config,
                                     int32_t batch, int32_t first_position,
                                     int32_t token_count) {
  return gemma4_kv_cache_ensure_range_ptr(
      page_table.data(), slot_logical_pages.data(),
      (int64_t)std::min(page_table.size(), slot_logical_pages.size()), &config,
      batch, first_position, token_count);
}

extern "C" {

Gemma4KvCacheConfig gemma4_kv_cache_make_config(bool global, int32_t num_pages,
                                                int32_t page_size,
                                                int32_t max_pages_per_seq) {
  Gemma4KvCacheConfig c;
  c.num_layers = global ? kGlobalLayerCount : kSlidingLayerCount;
  c.num_pages = num_pages;
  c.page_size = page_size;
  c.max_pages_per_seq = max_pages_per_seq;
  c.batch_size = max_pages_per_seq != 0 ? num_pages / max_pages_per_seq : 0;
  c.num_heads = global ? kGlobalKvHeads : kSlidingKvHeads;
  c.head_dim = global ? kGlobalHeadDim : kSlidingHeadDim;
  c.window_size = global ? 0 : kSlidingWindow;
  return c;
}

int32_t gemma4_kv_cache_layer_index(int32_t model_layer, bool global_cache) {
  if (model_layer < 0 || model_layer >= kNumLayers) return -1;
  if (is_global_layer(model_layer) != global_cache) return -1;
  int32_t index = 0;
  for (int32_t l = 0; l < model_layer; ++l) {
    if (is_global_layer(l) == global_cache) ++index;
  }
  return index;
}

int32_t gemma4_kv_cache_ensure_page_ptr(int32_t *page_table,
                                        int32_t *slot_logical_pages,
                                        int64_t entries,
                                        const Gemma4KvCacheConfig *config,
                                        int32_t batch, int32_t position) {
  if (page_table == nullptr || slot_logical_pages == nullptr ||
      config == nullptr || config->page_size <= 0 ||
      config->max_pages_per_seq <= 0 || batch < 0 || position < 0) {
    return -1;
  }
  const int32_t logical_page = position / config->page_size;
  const int32_t slot = logical_page % config->max_pages_per_seq;
  const int64_t index = (int64_t)batch * config->max_pages_per_seq + slot;
  if (index >= entries) return -1;
  // A slot already holding a newer logical page means a stale backwards use.
  if (slot_logical_pages[index] > logical_page) return -1;
  const int32_t physical = batch * config->max_pages_per_seq + slot;
  page_table[index] = physical;
  slot_logical_pages[index] = logical_page;
  return physical;
}

int32_t gemma4_kv_cache_ensure_range_ptr(int32_t *page_table,
                                         int32_t *slot_logical_pages,
                                         int64_t entries,
                                         const Gemma4KvCacheConfig *config,
                                         int32_t batch, int32_t first_position,
                                         int32_t token_count) {
  if (token_count == 0) return 0;
  if (config == nullptr || config->page_size <= 0 || token_count < 0) return -1;
  const int32_t first_page = first_position / config->page_size;
  const int32_t last_page = (first_position + token_count - 1) / config->page_size;
  for (int32_t page = first_page; page <= last_page; ++page) {
    if (gemma4_kv_cache_ensure_page_ptr(page_table, slot_logical_pages, entries,
                                        config, batch,
                                        page * config->page_size) < 0) {
      return -1;
    }
  }
  return 0;
}

hipError_t gemma4_kv_cache_write_bf16(
    gemma4_bf16 *d_cache_k, gemma4_bf16 *d_cache_v, Gemma4KvCacheConfig config,
    const int32_t *d_page_table, const int32_t *d_token_batch,
    const int32_t *d_token_position, int32_t token_count, int32_t layer,
    const gemma4_bf16 *d_k, const gemma4_bf16 *d_v, hipStream_t stream) {
  if (token_count == 0) return hipSuccess;
  if (token_count < 0 || !valid_append_config(config, layer) ||
      d_cache_k == nullptr || d_cache_v == nullptr || d_page_table == nullptr ||
      d_token_batch == nullptr || d_token_position == nullptr ||
      d_k == nullptr || d_v == nullptr) {
    return hipErrorInvalidValue;
  }
  return launch_append(reinterpret_cast<uint16_t *>(d_cache_k),
                       reinterpret_cast<uint16_t *>(d_cache_v), config,
                       d_page_table, d_token_batch, d_token_position,
                       token_count, layer, reinterpret_cast<const uint16_t *>(d_k),
                       reinterpret_cast<const uint16_t *>(d_v),
                       /*rows_per_batch=*/token_count, /*seq_len=*/0,
                       /*first_live=*/0, stream);
}

hipError_t gemma4_kv_cache_write_prefill_bf16(
    gemma4_bf16 *d_cache_k, gemma4_bf16 *d_cache_v, Gemma4KvCacheConfig config,
    const int32_t *d_page_table, const int32_t *d_token_batch,
    const int32_t *d_token_position, int32_t batch_size, int32_t seq_len,
    int32_t layer, const gemma4_bf16 *d_k, const gemma4_bf16 *d_v,
    hipStream_t stream) {
  if (batch_size == 0 || seq_len == 0) return hipSuccess;
  if (batch_size < 0 || seq_len < 0 || !valid_append_config(config, layer) ||
      d_cache_k == nullptr || d_cache_v == nullptr || d_page_table == nullptr ||
      d_token_batch == nullptr || d_token_position == nullptr ||
      d_k == nullptr || d_v == nullptr) {
    return hipErrorInvalidValue;
  }
  // Global caches and short chunks write every row; a long sliding chunk
  // writes only its last window_size rows per batch.
  const bool tail = config.window_size > 0 && seq_len > config.window_size;
  const int32_t rows_per_batch = tail ? config.window_size : seq_len;
  const int32_t first_live = tail ? seq_len - config.window_size : 0;
  const int64_t rows = (int64_t)batch_size * rows_per_batch;
  if (rows > 0x7fffffff) return hipErrorInvalidValue;
  return launch_append(reinterpret_cast<uint16_t *>(d_cache_k),
                       reinterpret_cast<uint16_t *>(d_cache_v), config,
                       d_page_table, d_token_batch, d_token_position,
                       (int32_t)rows, layer,
                       reinterpret_cast<const uint16_t *>(d_k),
                       reinterpret_cast<const uint16_t *>(d_v), rows_per_batch,
                       seq_len, first_live, stream);
}

}  // extern "C"
