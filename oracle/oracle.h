/*
 * CPU oracle for the gemma.c KV-cache + decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product library links, loads or
 * calls this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / the timed CPU baseline.
 *
 * Every function restates the reference algorithm in plain C and cites the
 * reference file:line it follows (paths relative to the gemma.c source tree).
 * bf16 values are carried as raw uint16_t bit patterns.
 *
 * Pinning status (what independent evidence checks each function):
 *   oracle_bf16_*            : IEEE bit-level known answers (tests/test_oracle.py)
 *   oracle_kv_cache_*        : reference tests/test_kv_cache.cu:94-133 and
 *                              tests/test_runtime_state.cu:29-107 expectations,
 *                              brute-force layout enumeration
 *   oracle_kv_cache_write    : bit-exact round trip, invalid-row known answer
 *   oracle_decode_attention  : torch float64 SDPA (library routine) and closed
 *                              forms (q=0 -> mean of live V, one key -> V,
 *                              window perturbation invariance)
 *   oracle_decode_split/combine : equals the unsplit oracle (split invariance)
 *   oracle_prefill_attention : torch float64 SDPA with explicit mask, the
 *                              reference q=0 running-mean known answer
 *                              (tests/test_flash_attention.cu:335-345)
 *   oracle_attention_o_projection: float64 matmul (numpy), closed forms
 *                              (one-hot attention row selects a weight
 *                              element; a constant residual row normalises
 *                              to the weight), residual identity
 *   oracle_rms_* / oracle_rope_*: reference known answers
 *                              (tests/test_flash_attention.cu:285-333,
 *                              tests/test_runtime_state.cu:110-140)
 */
#ifndef GEMMA4_ORACLE_H
#define GEMMA4_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same field order as the reference Gemma4KvCacheConfig
 * (src/gemma4_kv_cache.cuh:9-18). */
typedef struct {
  int32_t num_layers;
  int32_t num_pages;
  int32_t page_size;
  int32_t max_pages_per_seq;
  int32_t batch_size;
  int32_t num_heads;
  int32_t head_dim;
  int32_t window_size;
} OracleKvCacheConfig;

float oracle_bf16_to_f32(uint16_t bits);
uint16_t oracle_f32_to_bf16(float value);
void oracle_f32_to_bf16_array(const float *in, uint16_t *out, int64_t n);
void oracle_bf16_to_f32_array(const uint16_t *in, float *out, int64_t n);

int64_t oracle_kv_cache_offset(const OracleKvCacheConfig *config, int32_t layer,
                               int32_t page, int32_t page_offset, int32_t head,
                               int32_t dim);
void oracle_kv_cache_make_config(OracleKvCacheConfig *out, int32_t global,
                                 int32_t num_pages, int32_t page_size,
                                 int32_t max_pages_per_seq);
int32_t oracle_is_global_layer(int32_t layer);
int32_t oracle_kv_cache_layer_index(int32_t model_layer, int32_t global_cache);
int32_t oracle_kv_cache_ensure_page(int32_t *page_table,
                                    int32_t *slot_logical_pages,
                                    const OracleKvCacheConfig *config,
                                    int32_t batch, int32_t position);
int32_t oracle_kv_cache_ensure_range(int32_t *page_table,
                                     int32_t *slot_logical_pages,
                                     const OracleKvCacheConfig *config,
                                     int32_t batch, int32_t first_position,
                                     int32_t token_count);
int32_t oracle_sliding_pages_per_sequence(int32_t max_seq_len,
                                          int32_t page_size);

void oracle_kv_cache_write(uint16_t *cache_k, uint16_t *cache_v,
                           const OracleKvCacheConfig *config,
                           const int32_t *page_table,
                           const int32_t *token_batch,
                           const int32_t *token_position, int32_t token_count,
                           int32_t layer, const uint16_t *k,
                           const uint16_t *v);

/* Decode attention, two-pass softmax over the live keys of each row. */
void oracle_decode_attention(uint16_t *out, const uint16_t *q,
                             const uint16_t *cache_k, const uint16_t *cache_v,
                             const int32_t *page_table,
                             const int32_t *seq_lengths,
                             const OracleKvCacheConfig *config, int32_t layer,
                             float softmax_scale, int32_t batch_count,
                             int32_t q_heads);

/* One (sequence b, query head qh) row of oracle_decode_attention; scratch:
 * qf, acc hold head_dim floats, scores/rows hold seq_len entries. */
void oracle_decode_attention_row(uint16_t *out, const uint16_t *q,
                                 const uint16_t *cache_k, const uint16_t *cache_v,
                                 const int32_t *page_table, int32_t seq_len,
                                 const OracleKvCacheConfig *config, int32_t layer,
                                 float softmax_scale, int32_t b, int32_t qh,
                                 int32_t q_heads, float *qf, float *acc,
                                 float *scores, int64_t *rows);

/* Split-K partials (online update per key) and the log-sum-exp combine. */
void oracle_decode_split(float *partial_m, float *partial_l,
                         float *partial_acc, const uint16_t *q,
                         const uint16_t *cache_k, const uint16_t *cache_v,
                         const int32_t *page_table, const int32_t *seq_lengths,
                         const OracleKvCacheConfig *config, int32_t layer,
                         float softmax_scale, int32_t split_size,
                         int32_t num_splits, int32_t batch_count,
                         int32_t q_heads);
void oracle_decode_combine(uint16_t *out, const float *partial_m,
                           const float *partial_l, const float *partial_acc,
                           const int32_t *seq_lengths,
                           const OracleKvCacheConfig *config,
                           int32_t split_size, int32_t num_splits,
                           int32_t batch_count, int32_t q_heads);

/* Causal (optionally windowed) GQA prefill attention on contiguous rows.
 * q/out: [batch][seqlen_q][q_heads][head_dim], k/v: [batch][seqlen_k][kv_heads][head_dim].
 * Query row r sees keys [left, key_row] with key_row = r + seqlen_k - seqlen_q. */
void oracle_prefill_attention(uint16_t *out, const uint16_t *q,
                              const uint16_t *k, const uint16_t *v,
                              int32_t batch_size, int32_t seqlen_q,
                              int32_t seqlen_k, int32_t q_heads,
                              int32_t kv_heads, int32_t head_dim,
                              int32_t window_size, float softmax_scale);

/* RMSNorm scale and the split-half RoPE store used by Q/K preparation. */
float oracle_rms_scale(const float *values, int32_t width, float eps);
void oracle_prep_head(uint16_t *out, const uint16_t *in,
                      const uint16_t *weight /* NULL: scale-free */,
                      const float *cos_row, const float *sin_row,
                      int32_t head_dim, int32_t rotary_dim, float eps);
void oracle_attention_o_projection(uint16_t *residual_out, uint16_t *normed_out,
                                   uint16_t *ffn_residual, const uint16_t *attn,
                                   const uint16_t *w_col_major, const uint16_t *norm_weight,
                                   const uint16_t *x, int32_t rows, int32_t attention_width,
                                   int32_t hidden, float eps);
void oracle_fill_rope_tables(float *cos_table, float *sin_table,
                             int32_t max_seq_len, int32_t rotary_half,
                             float theta, int32_t exponent_dim);

/* CPU baseline timings (oracle/cpu_baseline.c): the oracle's append and
 * decode attention timed on 1 or more host threads, split over (sequence,
 * KV head) tasks. Return seconds of compute (inputs generated beforehand). */
void oracle_fill_normal_bf16(uint16_t *dst, int64_t n, uint64_t seed, float scale,
                             int32_t threads);
double oracle_time_decode_layer(uint16_t *out, const uint16_t *q, uint16_t *cache_k,
                                uint16_t *cache_v, const int32_t *page_table,
                                const int32_t *seq_lengths, const int32_t *token_position,
                                const uint16_t *k_new, const uint16_t *v_new,
                                const OracleKvCacheConfig *config, int32_t layer,
                                float scale, int32_t batch, int32_t q_heads,
                                int32_t threads);
double oracle_time_config1(uint16_t *out, const uint16_t *q, const uint16_t *k,
                           const uint16_t *v, uint16_t *cache_k, uint16_t *cache_v,
                           int32_t *page_table, int32_t *slot_logical_pages,
                           const OracleKvCacheConfig *config, float scale, int32_t steps,
                           int32_t q_heads, int32_t threads);

#ifdef __cplusplus
}
#endif

#endif
