// Attention output projection with the post-attention tail, MI355X (gfx950)
// build: the consumer of the decode attention output. extern "C",
// stream-ordered, allocates nothing; returns hipErrorInvalidValue on bad
// geometry or null pointers before any launch.
#pragma once

#include "gemma4_kv_cache.h"

#ifdef __cplusplus
extern "C" {
#endif

// Hidden width of the gemma4 text model (src/gemma4.h:6).
#define GEMMA4_ATTENTION_OUTPUT_HIDDEN 3840

// For each of `rows` token rows:
//   residual_out[c] = bf16(sum_e attention_out[e] * o_proj_col_major[c][e])
//   normed_out      = bf16(residual_out * s * post_norm_weight),
//                     s = rsqrt(mean(residual_out^2) + 1e-6) over the bf16 row
//   ffn_residual    = bf16(attention_x + normed_out)
// attention_out [rows][attention_width], o_proj_col_major
// [3840][attention_width] (hidden column c's weights contiguous),
// post_norm_weight [3840], attention_x / residual_out / normed_out /
// ffn_residual [rows][3840]. attention_width is 16 query heads x head_dim:
// 4096 (sliding layers) or 8192 (global layers).
// Replaces project_attention_out_post_attention
// (src/gemma4_flash_attention_decode.cu:34-129), a device phase of the
// reference's cooperative decode layer kernel with no entry point of its own;
// extended from one row to `rows` (each weight is read once per launch and
// applied to every row, so small decode batches cost one weight stream).
hipError_t gemma4_attention_o_projection_post_norm_bf16(
    gemma4_bf16 *residual_out, gemma4_bf16 *normed_out, gemma4_bf16 *ffn_residual,
    const gemma4_bf16 *attention_out, const gemma4_bf16 *o_proj_col_major,
    const gemma4_bf16 *post_norm_weight, const gemma4_bf16 *attention_x, int32_t rows,
    int32_t attention_width, hipStream_t stream);

#ifdef __cplusplus
}
#endif
