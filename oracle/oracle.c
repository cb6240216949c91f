/*
 * CPU oracle for the gemma.c KV-cache + decode-attention path.
 *
 * TEST INFRASTRUCTURE ONLY: never linked into or called by the product
 * library. See oracle.h for what pins each function.
 *
 * Reference paths are relative to the gemma.c source tree.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Constants of the reference model (src/gemma4.h:8-24). */
#define ORACLE_NUM_LAYERS 48
#define ORACLE_GLOBAL_LAYER_PERIOD 6
#define ORACLE_GLOBAL_LAYER_COUNT 8
#define ORACLE_SLIDING_LAYER_COUNT 40
#define ORACLE_SLIDING_KV_HEADS 8
#define ORACLE_GLOBAL_KV_HEADS 1
#define ORACLE_SLIDING_HEAD_DIM 256
#define ORACLE_GLOBAL_HEAD_DIM 512
#define ORACLE_SLIDING_WINDOW 1024

float oracle_bf16_to_f32(uint16_t bits) {
  uint32_t u = (uint32_t)bits << 16;
  float f;
  memcpy(&f, &u, sizeof(f));
  return f;
}

/* Round-to-nearest-even float -> bf16, NaN kept quiet with its sign. */
uint16_t oracle_f32_to_bf16(float value) {
  uint32_t u;
  memcpy(&u, &value, sizeof(u));
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    return (uint16_t)((u >> 16) | 0x0040u);
  }
  const uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

void oracle_f32_to_bf16_array(const float *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_bf16(in[i]);
}

void oracle_bf16_to_f32_array(const uint16_t *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_bf16_to_f32(in[i]);
}

/* Layout-A offset [layer][page][page_offset][head][dim]
 * (src/gemma4_kv_cache.cuh:28-38). */
int64_t oracle_kv_cache_offset(const OracleKvCacheConfig *c, int32_t layer,
                               int32_t page, int32_t page_offset, int32_t head,
                               int32_t dim) {
  const int64_t layer_page = (int64_t)layer * c->num_pages + page;
  const int64_t token = layer_page * c->page_size + page_offset;
  return (token * c->num_heads + head) * c->head_dim + dim;
}

/* src/gemma4_kv_cache.cu:76-91 */
void oracle_kv_cache_make_config(OracleKvCacheConfig *out, int32_t global,
                                 int32_t num_pages, int32_t page_size,
                                 int32_t max_pages_per_seq) {
  out->num_layers =
      global ? ORACLE_GLOBAL_LAYER_COUNT : ORACLE_SLIDING_LAYER_COUNT;
  out->num_pages = num_pages;
  out->page_size = page_size;
  out->max_pages_per_seq = max_pages_per_seq;
  out->batch_size = num_pages / max_pages_per_seq;
  out->num_heads = global ? ORACLE_GLOBAL_KV_HEADS : ORACLE_SLIDING_KV_HEADS;
  out->head_dim = global ? ORACLE_GLOBAL_HEAD_DIM : ORACLE_SLIDING_HEAD_DIM;
  out->window_size = global ? 0 : ORACLE_SLIDING_WINDOW;
}

/* src/gemma4.h:105-108 */
int32_t oracle_is_global_layer(int32_t layer) {
  return layer == ORACLE_NUM_LAYERS - 1 ||
         (layer + 1) % ORACLE_GLOBAL_LAYER_PERIOD == 0;
}

/* src/gemma4_kv_cache.cu:94-105 */
int32_t oracle_kv_cache_layer_index(int32_t model_layer, int32_t global_cache) {
  if (model_layer < 0 || model_layer >= ORACLE_NUM_LAYERS) return -1;
  if (oracle_is_global_layer(model_layer) != (global_cache != 0)) return -1;
  int32_t index = 0;
  for (int32_t l = 0; l < model_layer; ++l) {
    if (oracle_is_global_layer(l) == (global_cache != 0)) ++index;
  }
  return index;
}

/* src/gemma4_kv_cache.cu:108-122 */
int32_t oracle_kv_cache_ensure_page(int32_t *page_table,
                                    int32_t *slot_logical_pages,
                                    const OracleKvCacheConfig *c,
                                    int32_t batch, int32_t position) {
  const int32_t logical_page = position / c->page_size;
  const int32_t slot = logical_page % c->max_pages_per_seq;
  const int64_t index = (int64_t)batch * c->max_pages_per_seq + slot;
  if (slot_logical_pages[index] > logical_page) return -1;
  const int32_t physical = batch * c->max_pages_per_seq + slot;
  page_table[index] = physical;
  slot_logical_pages[index] = logical_page;
  return physical;
}

/* src/gemma4_kv_cache.cu:125-146 */
int32_t oracle_kv_cache_ensure_range(int32_t *page_table,
                                     int32_t *slot_logical_pages,
                                     const OracleKvCacheConfig *c,
                                     int32_t batch, int32_t first_position,
                                     int32_t token_count) {
  if (token_count == 0) return 0;
  const int32_t first_page = first_position / c->page_size;
  const int32_t last_page = (first_position + token_count - 1) / c->page_size;
  for (int32_t page = first_page; page <= last_page; ++page) {
    if (oracle_kv_cache_ensure_page(page_table, slot_logical_pages, c, batch,
                                    page * c->page_size) < 0) {
      return -1;
    }
  }
  return 0;
}

/* src/gemma4_runtime.cu:18-24 */
int32_t oracle_sliding_pages_per_sequence(int32_t max_seq_len,
                                          int32_t page_size) {
  if (max_seq_len <= ORACLE_SLIDING_WINDOW) {
    return (max_seq_len + page_size - 1) / page_size;
  }
  return (ORACLE_SLIDING_WINDOW + page_size - 1 + page_size - 1) / page_size;
}

/* Append with the reference skip rules (src/gemma4_kv_cache.cu:25-54). */
void oracle_kv_cache_write(uint16_t *cache_k, uint16_t *cache_v,
                           const OracleKvCacheConfig *c,
                           const int32_t *page_table,
                           const int32_t *token_batch,
                           const int32_t *token_position, int32_t token_count,
                           int32_t layer, const uint16_t *k,
                           const uint16_t *v) {
  for (int32_t t = 0; t < token_count; ++t) {
    const int32_t batch = token_batch[t];
    const int32_t position = token_position[t];
    if (batch < 0 || position < 0 || batch >= c->batch_size) continue;
    const int32_t logical_page = position / c->page_size;
    if (c->window_size == 0 && logical_page >= c->max_pages_per_seq) continue;
    const int32_t slot = logical_page % c->max_pages_per_seq;
    const int32_t physical = page_table[batch * c->max_pages_per_seq + slot];
    if (physical < 0 || physical >= c->num_pages) continue;
    const int32_t page_offset = position - logical_page * c->page_size;
    for (int32_t h = 0; h < c->num_heads; ++h) {
      const int64_t src = ((int64_t)t * c->num_heads + h) * c->head_dim;
      const int64_t dst =
          oracle_kv_cache_offset(c, layer, physical, page_offset, h, 0);
      memcpy(cache_k + dst, k + src, sizeof(uint16_t) * c->head_dim);
      memcpy(cache_v + dst, v + src, sizeof(uint16_t) * c->head_dim);
    }
  }
}

/* Physical page of one live key, or -1 when the page is unmapped
 * (src/gemma4_flash_attention_decode.cu:791-805). */
static int32_t key_physical_page(const OracleKvCacheConfig *c,
                                 const int32_t *page_table, int32_t batch,
                                 int32_t pos) {
  const int32_t logical_page = pos / c->page_size;
  const int32_t slot = logical_page % c->max_pages_per_seq;
  const int32_t physical = page_table[batch * c->max_pages_per_seq + slot];
  if (physical < 0 || physical >= c->num_pages) return -1;
  return physical;
}

static void live_key_range(const OracleKvCacheConfig *c, int32_t seq_len,
                           int32_t *first, int32_t *count) {
  int32_t f = c->window_size > 0 ? seq_len - c->window_size : 0;
  if (f < 0) f = 0;
  int32_t n = seq_len - f;
  if (n < 0) n = 0;
  *first = f;
  *count = n;
}

/* Two-pass fp32 softmax of one query row over its live paged keys: the
 * reference host attention (tests/test_flash_attention.cu:124-172) applied to
 * the last query row, with keys gathered through the page table and the
 * sliding window counting the current token (src/gemma4.h:22-23,
 * src/gemma4_flash_attention_decode.cu:730-732). One (sequence, query head)
 * row; the scratch buffers hold head_dim floats (qf, acc) and seq_len
 * entries (scores, rows). */
void oracle_decode_attention_row(uint16_t *out, const uint16_t *q,
                                 const uint16_t *cache_k, const uint16_t *cache_v,
                                 const int32_t *page_table, int32_t seq_len,
                                 const OracleKvCacheConfig *c, int32_t layer,
                                 float softmax_scale, int32_t b, int32_t qh,
                                 int32_t q_heads, float *qf, float *acc,
                                 float *scores, int64_t *rows) {
  const int32_t D = c->head_dim;
  const int32_t group = q_heads / c->num_heads;
  int32_t first, count;
  live_key_range(c, seq_len, &first, &count);
  const int32_t kvh = qh / group;
  const int64_t q_base = ((int64_t)b * q_heads + qh) * D;
  for (int32_t d = 0; d < D; ++d) qf[d] = oracle_bf16_to_f32(q[q_base + d]);
  int32_t n = 0;
  float max_score = -INFINITY;
  for (int32_t i = 0; i < count; ++i) {
    const int32_t pos = first + i;
    const int32_t phys = key_physical_page(c, page_table, b, pos);
    if (phys < 0) continue;
    const int64_t row = oracle_kv_cache_offset(c, layer, phys, pos % c->page_size, kvh, 0);
    float score = 0.0f;
    for (int32_t d = 0; d < D; ++d) {
      score += qf[d] * oracle_bf16_to_f32(cache_k[row + d]);
    }
    score *= softmax_scale;
    rows[n] = row;
    scores[n] = score;
    if (score > max_score) max_score = score;
    ++n;
  }
  float denom = 0.0f;
  for (int32_t i = 0; i < n; ++i) {
    scores[i] = expf(scores[i] - max_score);
    denom += scores[i];
  }
  for (int32_t d = 0; d < D; ++d) acc[d] = 0.0f;
  for (int32_t i = 0; i < n; ++i) {
    const float w = scores[i] / denom;
    const uint16_t *vrow = cache_v + rows[i];
    for (int32_t d = 0; d < D; ++d) acc[d] += w * oracle_bf16_to_f32(vrow[d]);
  }
  for (int32_t d = 0; d < D; ++d) {
    out[q_base + d] = oracle_f32_to_bf16(n > 0 ? acc[d] : 0.0f);
  }
}

void oracle_decode_attention(uint16_t *out, const uint16_t *q,
                             const uint16_t *cache_k, const uint16_t *cache_v,
                             const int32_t *page_table,
                             const int32_t *seq_lengths,
                             const OracleKvCacheConfig *c, int32_t layer,
                             float softmax_scale, int32_t batch_count,
                             int32_t q_heads) {
  const int32_t D = c->head_dim;
  int32_t max_keys = 0;
  for (int32_t b = 0; b < batch_count; ++b) {
    if (seq_lengths[b] > max_keys) max_keys = seq_lengths[b];
  }
  const int32_t cap = max_keys > 0 ? max_keys : 1;
  float *qf = (float *)malloc(sizeof(float) * D);
  float *acc = (float *)malloc(sizeof(float) * D);
  float *scores = (float *)malloc(sizeof(float) * cap);
  int64_t *rows = (int64_t *)malloc(sizeof(int64_t) * cap);
  for (int32_t b = 0; b < batch_count; ++b) {
    for (int32_t qh = 0; qh < q_heads; ++qh) {
      oracle_decode_attention_row(out, q, cache_k, cache_v, page_table, seq_lengths[b], c,
                                  layer, softmax_scale, b, qh, q_heads, qf, acc, scores, rows);
    }
  }
  free(qf);
  free(acc);
  free(scores);
  free(rows);
}

/* Split-K partials: one (row, split) task runs the per-key online update
 * (src/gemma4_flash_attention_decode.cu:530-542) over keys
 * [first + split*S, min(seq, first + (split+1)*S)), skipping unmapped pages and
 * leaving splits at or beyond the live split count untouched
 * (src/gemma4_flash_attention_decode.cu:719-756, 858-877). */
void oracle_decode_split(float *partial_m, float *partial_l,
                         float *partial_acc, const uint16_t *q,
                         const uint16_t *cache_k, const uint16_t *cache_v,
                         const int32_t *page_table, const int32_t *seq_lengths,
                         const OracleKvCacheConfig *c, int32_t layer,
                         float softmax_scale, int32_t split_size,
                         int32_t num_splits, int32_t batch_count,
                         int32_t q_heads) {
  const int32_t D = c->head_dim;
  const int32_t group = q_heads / c->num_heads;
  float *qf = (float *)malloc(sizeof(float) * D);
  float *acc = (float *)malloc(sizeof(float) * D);
  for (int32_t b = 0; b < batch_count; ++b) {
    int32_t first, count;
    live_key_range(c, seq_lengths[b], &first, &count);
    const int32_t actual = (count + split_size - 1) / split_size;
    for (int32_t qh = 0; qh < q_heads; ++qh) {
      const int32_t kvh = qh / group;
      const int64_t q_base = ((int64_t)b * q_heads + qh) * D;
      for (int32_t d = 0; d < D; ++d) qf[d] = oracle_bf16_to_f32(q[q_base + d]);
      for (int32_t s = 0; s < num_splits && s < actual; ++s) {
        const int32_t begin = first + s * split_size;
        int32_t end = begin + split_size;
        if (end > seq_lengths[b]) end = seq_lengths[b];
        float m = -INFINITY, l = 0.0f;
        for (int32_t d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int32_t pos = begin; pos < end; ++pos) {
          const int32_t phys = key_physical_page(c, page_table, b, pos);
          if (phys < 0) continue;
          const int64_t row = oracle_kv_cache_offset(
              c, layer, phys, pos % c->page_size, kvh, 0);
          float score = 0.0f;
          for (int32_t d = 0; d < D; ++d) {
            score += qf[d] * oracle_bf16_to_f32(cache_k[row + d]);
          }
          score *= softmax_scale;
          const float new_m = score > m ? score : m;
          const float old_scale = expf(m - new_m);
          const float new_scale = expf(score - new_m);
          for (int32_t d = 0; d < D; ++d) {
            acc[d] = acc[d] * old_scale +
                     oracle_bf16_to_f32(cache_v[row + d]) * new_scale;
          }
          l = l * old_scale + new_scale;
          m = new_m;
        }
        const int64_t p = ((int64_t)b * q_heads + qh) * num_splits + s;
        partial_m[p] = m;
        partial_l[p] = l;
        for (int32_t d = 0; d < D; ++d) partial_acc[p * D + d] = acc[d];
      }
    }
  }
  free(qf);
  free(acc);
}

/* Log-sum-exp combine over the live splits of each row
 * (src/gemma4_flash_attention_decode.cu:880-977). */
void oracle_decode_combine(uint16_t *out, const float *partial_m,
                           const float *partial_l, const float *partial_acc,
                           const int32_t *seq_lengths,
                           const OracleKvCacheConfig *c, int32_t split_size,
                           int32_t num_splits, int32_t batch_count,
                           int32_t q_heads) {
  const int32_t D = c->head_dim;
  for (int32_t b = 0; b < batch_count; ++b) {
    int32_t first, count;
    live_key_range(c, seq_lengths[b], &first, &count);
    int32_t splits = (count + split_size - 1) / split_size;
    if (splits > num_splits) splits = num_splits;
    for (int32_t qh = 0; qh < q_heads; ++qh) {
      const int64_t row = (int64_t)b * q_heads + qh;
      const int64_t p0 = row * num_splits;
      float big_m = -INFINITY;
      for (int32_t s = 0; s < splits; ++s) {
        if (partial_m[p0 + s] > big_m) big_m = partial_m[p0 + s];
      }
      float big_l = 0.0f;
      for (int32_t s = 0; s < splits; ++s) {
        if (partial_l[p0 + s] > 0.0f) {
          big_l += partial_l[p0 + s] * expf(partial_m[p0 + s] - big_m);
        }
      }
      for (int32_t d = 0; d < D; ++d) {
        float value = 0.0f;
        for (int32_t s = 0; s < splits; ++s) {
          if (partial_l[p0 + s] > 0.0f) {
            value += partial_acc[(p0 + s) * D + d] *
                     expf(partial_m[p0 + s] - big_m);
          }
        }
        out[row * D + d] =
            oracle_f32_to_bf16(splits > 0 && big_l > 0.0f ? value / big_l : 0.0f);
      }
    }
  }
}

/* Causal GQA prefill attention with a prior-context offset: the reference
 * host attention (tests/test_flash_attention.cu:124-172) with the kernel's
 * mask generalised to seqlen_k >= seqlen_q
 * (src/gemma4_flash_attention_prefill.cu:524-535). A row with no visible key
 * produces zeros (src/gemma4_flash_attention_prefill.cu:483-497). */
void oracle_prefill_attention(uint16_t *out, const uint16_t *q,
                              const uint16_t *k, const uint16_t *v,
                              int32_t batch_size, int32_t seqlen_q,
                              int32_t seqlen_k, int32_t q_heads,
                              int32_t kv_heads, int32_t head_dim,
                              int32_t window_size, float softmax_scale) {
  const int32_t D = head_dim;
  const int32_t group = q_heads / kv_heads;
  float *scores = (float *)malloc(sizeof(float) * (seqlen_k > 0 ? seqlen_k : 1));
  float *qf = (float *)malloc(sizeof(float) * D);
  float *acc = (float *)malloc(sizeof(float) * D);
  for (int32_t b = 0; b < batch_size; ++b) {
    for (int32_t r = 0; r < seqlen_q; ++r) {
      const int32_t key_row = r + seqlen_k - seqlen_q;
      int32_t right = key_row + 1;
      if (right > seqlen_k) right = seqlen_k;
      int32_t left = 0;
      if (window_size > 0) {
        left = key_row - window_size + 1;
        if (left < 0) left = 0;
      }
      for (int32_t qh = 0; qh < q_heads; ++qh) {
        const int32_t kvh = qh / group;
        const int64_t q_base = (((int64_t)b * seqlen_q + r) * q_heads + qh) * D;
        for (int32_t d = 0; d < D; ++d) qf[d] = oracle_bf16_to_f32(q[q_base + d]);
        float max_score = -INFINITY;
        for (int32_t col = left; col < right; ++col) {
          const int64_t k_base = (((int64_t)b * seqlen_k + col) * kv_heads + kvh) * D;
          float score = 0.0f;
          for (int32_t d = 0; d < D; ++d) {
            score += qf[d] * oracle_bf16_to_f32(k[k_base + d]);
          }
          scores[col] = score * softmax_scale;
          if (scores[col] > max_score) max_score = scores[col];
        }
        float denom = 0.0f;
        for (int32_t col = left; col < right; ++col) {
          scores[col] = expf(scores[col] - max_score);
          denom += scores[col];
        }
        for (int32_t d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int32_t col = left; col < right; ++col) {
          const float w = scores[col] / denom;
          const int64_t v_base = (((int64_t)b * seqlen_k + col) * kv_heads + kvh) * D;
          for (int32_t d = 0; d < D; ++d) acc[d] += w * oracle_bf16_to_f32(v[v_base + d]);
        }
        for (int32_t d = 0; d < D; ++d) {
          out[q_base + d] = oracle_f32_to_bf16(right > left ? acc[d] : 0.0f);
        }
      }
    }
  }
  free(scores);
  free(qf);
  free(acc);
}

/* RMSNorm multiplier (src/gemma4_rmsnorm.cu:91-101,
 * tests/test_flash_attention.cu:119-121). */
float oracle_rms_scale(const float *values, int32_t width, float eps) {
  float sum_sq = 0.0f;
  for (int32_t i = 0; i < width; ++i) sum_sq = fmaf(values[i], values[i], sum_sq);
  return 1.0f / sqrtf(sum_sq / (float)width + eps);
}

/* Learned RMSNorm + split-half RoPE over the rotary prefix, plain normalised
 * tail (src/gemma4_flash_attention_decode.cu:240-269, src/gemma4_rope.cu:8-20);
 * with weight == NULL the scale-free V normalisation
 * (src/gemma4_flash_attention_decode.cu:273-283). */
void oracle_prep_head(uint16_t *out, const uint16_t *in, const uint16_t *weight,
                      const float *cos_row, const float *sin_row,
                      int32_t head_dim, int32_t rotary_dim, float eps) {
  float *vals = (float *)calloc((size_t)(head_dim > 0 ? head_dim : 1), sizeof(float));
  for (int32_t d = 0; d < head_dim; ++d) vals[d] = oracle_bf16_to_f32(in[d]);
  const float scale = oracle_rms_scale(vals, head_dim, eps);
  if (weight == NULL) {
    for (int32_t d = 0; d < head_dim; ++d) out[d] = oracle_f32_to_bf16(vals[d] * scale);
    free(vals);
    return;
  }
  const int32_t half = rotary_dim / 2;
  for (int32_t i = 0; i < half; ++i) {
    const float lo = vals[i] * scale * oracle_bf16_to_f32(weight[i]);
    const float hi = vals[half + i] * scale * oracle_bf16_to_f32(weight[half + i]);
    const float c = cos_row[i];
    const float s = sin_row[i];
    out[i] = oracle_f32_to_bf16(fmaf(-hi, s, lo * c));
    out[half + i] = oracle_f32_to_bf16(fmaf(lo, s, hi * c));
  }
  for (int32_t d = rotary_dim; d < head_dim; ++d) {
    out[d] = oracle_f32_to_bf16(vals[d] * scale * oracle_bf16_to_f32(weight[d]));
  }
  free(vals);
}

/* src/gemma4_runtime.cu:27-44 */
void oracle_fill_rope_tables(float *cos_table, float *sin_table,
                             int32_t max_seq_len, int32_t rotary_half,
                             float theta, int32_t exponent_dim) {
  for (int32_t pos = 0; pos < max_seq_len; ++pos) {
    for (int32_t i = 0; i < rotary_half; ++i) {
      const float exponent = -2.0f * (float)i / (float)exponent_dim;
      const float angle = (float)pos * powf(theta, exponent);
      cos_table[(int64_t)pos * rotary_half + i] = cosf(angle);
      sin_table[(int64_t)pos * rotary_half + i] = sinf(angle);
    }
  }
}

/* Attention output projection with the post-attention tail, per token row
 * (src/gemma4_flash_attention_decode.cu:34-129): residual_out[c] =
 * bf16(sum_e attn[e] * W[c][e]) with W stored column-major
 * ([hidden][attention_width]); normed_out = bf16(residual * s * weight),
 * s = rsqrt(mean(residual^2) + eps) over the bf16 residual row
 * (src/gemma4_rmsnorm.cu:28-85); ffn_residual = bf16(x + normed)
 * (src/gemma4_cuda_utils.cuh:105-122). Products are summed in float64 here,
 * so the reference's and the GPU's fp32 summation orders both sit within
 * rounding of this value. */
void oracle_attention_o_projection(uint16_t *residual_out, uint16_t *normed_out,
                                   uint16_t *ffn_residual, const uint16_t *attn,
                                   const uint16_t *w_col_major, const uint16_t *norm_weight,
                                   const uint16_t *x, int32_t rows, int32_t attention_width,
                                   int32_t hidden, float eps) {
  float *arow = (float *)malloc((size_t)attention_width * sizeof(float));
  float *res = (float *)malloc((size_t)hidden * sizeof(float));
  for (int32_t r = 0; r < rows; ++r) {
    const uint16_t *a = attn + (int64_t)r * attention_width;
    for (int32_t e = 0; e < attention_width; ++e) arow[e] = oracle_bf16_to_f32(a[e]);
    for (int32_t c = 0; c < hidden; ++c) {
      const uint16_t *w = w_col_major + (int64_t)c * attention_width;
      double sum = 0.0;
      for (int32_t e = 0; e < attention_width; ++e) sum += (double)arow[e] * oracle_bf16_to_f32(w[e]);
      const uint16_t bits = oracle_f32_to_bf16((float)sum);
      residual_out[(int64_t)r * hidden + c] = bits;
      res[c] = oracle_bf16_to_f32(bits);
    }
    const float s = oracle_rms_scale(res, hidden, eps);
    for (int32_t c = 0; c < hidden; ++c) {
      const int64_t o = (int64_t)r * hidden + c;
      const uint16_t n = oracle_f32_to_bf16(res[c] * s * oracle_bf16_to_f32(norm_weight[c]));
      normed_out[o] = n;
      ffn_residual[o] = oracle_f32_to_bf16(oracle_bf16_to_f32(x[o]) + oracle_bf16_to_f32(n));
    }
  }
  free(arow);
  free(res);
}
