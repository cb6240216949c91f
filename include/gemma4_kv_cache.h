// Paged bf16 K/V cache for gemma.c's attention layers, MI355X (gfx950) build.
//
// Drop-in for the reference header src/gemma4_kv_cache.cuh: same struct
// layout, names, argument order and error convention, with HIP types
// (hipError_t / hipStream_t / __hip_bfloat16) in place of the CUDA ones.
// Every device entry point is extern "C" and takes plain pointers and sizes.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
struct __hip_bfloat16;  // complete in <hip/hip_bf16.h>; only pointers cross this API
typedef struct __hip_bfloat16 gemma4_bf16;
#include <vector>
#else
#include <stdbool.h>
typedef uint16_t gemma4_bf16;  // C callers pass raw bf16 bit patterns
#endif

#if defined(__HIPCC__)
#define GEMMA4_HOST_DEVICE __host__ __device__
#else
#define GEMMA4_HOST_DEVICE
#endif
#ifdef __cplusplus
#define GEMMA4_CONSTEXPR constexpr
#else
#define GEMMA4_CONSTEXPR
#endif

// Replaces src/gemma4_kv_cache.cuh:9-18 (same 8 x int32 layout, 32 bytes).
// window_size == 0 marks a full-length global cache; > 0 a sliding ring.
typedef struct Gemma4KvCacheConfig {
  int32_t num_layers;
  int32_t num_pages;
  int32_t page_size;
  int32_t max_pages_per_seq;
  int32_t batch_size;
  int32_t num_heads;
  int32_t head_dim;
  int32_t window_size;
} Gemma4KvCacheConfig;

// Replaces src/gemma4_kv_cache.cuh:27-38. Flat Layout-A element offset
// [layer][page][page_offset][head][dim]; constexpr in C++ (usable in
// constant expressions, as the reference's is).
static inline GEMMA4_CONSTEXPR GEMMA4_HOST_DEVICE int64_t gemma4_kv_cache_offset(
    const Gemma4KvCacheConfig *config, int32_t layer, int32_t page,
    int32_t page_offset, int32_t head, int32_t dim) {
  const int64_t layer_page = (int64_t)layer * config->num_pages + page;
  const int64_t token = layer_page * config->page_size + page_offset;
  return (token * config->num_heads + head) * config->head_dim + dim;
}

#ifdef __cplusplus
// Reference-style overload taking the config by reference
// (src/gemma4_kv_cache.cuh:28, __host__ __device__ constexpr).
static inline constexpr GEMMA4_HOST_DEVICE int64_t gemma4_kv_cache_offset(
    const Gemma4KvCacheConfig &config, int32_t layer, int32_t page,
    int32_t page_offset, int32_t head, int32_t dim) {
  return gemma4_kv_cache_offset(&config, layer, page, page_offset, head, dim);
}

// Replaces src/gemma4_kv_cache.cuh:42-53 (host ring-slot bookkeeping with the
// reference's std::vector arguments). Return the physical page, or -1 when
// the slot already holds a newer logical page.
int32_t gemma4_kv_cache_ensure_page(std::vector<int32_t> &page_table,
                                    std::vector<int32_t> &slot_logical_pages,
                                    const Gemma4KvCacheConfig &config,
                                    int32_t batch, int32_t position);
int32_t gemma4_kv_cache_ensure_range(std::vector<int32_t> &page_table,
                                     std::vector<int32_t> &slot_logical_pages,
                                     const Gemma4KvCacheConfig &config,
                                     int32_t batch, int32_t first_position,
                                     int32_t token_count);
extern "C" {
#endif

// Replaces src/gemma4_kv_cache.cuh:20-23 (src/gemma4_kv_cache.cu:76-91).
Gemma4KvCacheConfig gemma4_kv_cache_make_config(bool global, int32_t num_pages,
                                                int32_t page_size,
                                                int32_t max_pages_per_seq);

// Replaces src/gemma4_kv_cache.cuh:25 (src/gemma4_kv_cache.cu:94-105).
int32_t gemma4_kv_cache_layer_index(int32_t model_layer, bool global_cache);

// Plain-pointer forms of the two std::vector helpers above, for C / FFI
// callers. `entries` is the length of both arrays
// (batch_size * max_pages_per_seq); out-of-range slots return -1.
int32_t gemma4_kv_cache_ensure_page_ptr(int32_t *page_table,
                                        int32_t *slot_logical_pages,
                                        int64_t entries,
                                        const Gemma4KvCacheConfig *config,
                                        int32_t batch, int32_t position);
int32_t gemma4_kv_cache_ensure_range_ptr(int32_t *page_table,
                                         int32_t *slot_logical_pages,
                                         int64_t entries,
                                         const Gemma4KvCacheConfig *config,
                                         int32_t batch, int32_t first_position,
                                         int32_t token_count);

// Replaces src/gemma4_kv_cache.cuh:55-66 (src/gemma4_kv_cache.cu:149-180).
// Stream-ordered bit-exact copy of prepared K/V rows [token][num_heads][head_dim]
// into the paged cache. Rows whose batch/position/page is out of range are
// skipped on the device. token_count == 0 is a no-op success; bad geometry or
// null pointers return hipErrorInvalidValue before any launch.
hipError_t gemma4_kv_cache_write_bf16(
    gemma4_bf16 *d_cache_k, gemma4_bf16 *d_cache_v, Gemma4KvCacheConfig config,
    const int32_t *d_page_table, const int32_t *d_token_batch,
    const int32_t *d_token_position, int32_t token_count, int32_t layer,
    const gemma4_bf16 *d_k, const gemma4_bf16 *d_v, hipStream_t stream);

// Prefill-chunk cache write policy of src/gemma4_prefill_megakernel.cu:189-207:
// rows are batch-major [batch][seq_len]; a global cache, or a chunk of at most
// `window_size` rows, writes every row; a longer chunk into a sliding ring
// writes only the last `window_size` rows of each batch (the live ring tail).
// One launch covers all batches.
hipError_t gemma4_kv_cache_write_prefill_bf16(
    gemma4_bf16 *d_cache_k, gemma4_bf16 *d_cache_v, Gemma4KvCacheConfig config,
    const int32_t *d_page_table, const int32_t *d_token_batch,
    const int32_t *d_token_position, int32_t batch_size, int32_t seq_len,
    int32_t layer, const gemma4_bf16 *d_k, const gemma4_bf16 *d_v,
    hipStream_t stream);

#ifdef __cplusplus
}  // extern "C"
#endif
