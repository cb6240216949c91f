// Per-head preparation shared by the decode-token and prefill prep kernels
// (gfx950): learned RMSNorm + split-half RoPE (Q, K) and scale-free RMSNorm
// (V), one wave per head. A wave holds its head lane-strided (lane owns dims
// lane + 64 i), so each rotary pair (d, d + rotary_dim/2) sits in one lane
// and a head's sum of squares is one wave reduction. Follows
// src/gemma4_flash_attention_decode.cu:216-283,
// src/gemma4_flash_attention_prefill.cu:960-1021, src/gemma4_rope.cu:8-20 and
// src/gemma4_rmsnorm.cu:90-101.
#pragma once

#include "gemma4_device.hpp"

#include <math.h>

namespace gemma4 {

constexpr float kRmsEps = 1.0e-6f;  // GEMMA4_RMS_NORM_EPS (src/gemma4.h:29)

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float((uint32_t)b << 16);
}

__device__ __forceinline__ float wave_sum(float v) {
  v += lane_xor<1>(v);
  v += lane_xor<2>(v);
  v += lane_xor<4>(v);
  v += lane_xor<8>(v);
  v += lane_xor<16>(v);
  v += lane_xor<32>(v);
  return v;
}

// Loads one head lane-strided as fp32.
template <int kDim>
__device__ __forceinline__ void load_head(const uint16_t *src, float (&x)[kDim / kWave], int lane) {
#pragma unroll
  for (int i = 0; i < kDim / kWave; ++i) x[i] = bf16_bits_to_f32(src[lane + i * kWave]);
}

// rsqrt(mean(x^2) + eps) of one head (src/gemma4_rmsnorm.cu:90-101).
template <int kDim>
__device__ __forceinline__ float head_rms_scale(const float (&x)[kDim / kWave]) {
  float sum_sq = 0.0f;
#pragma unroll
  for (int i = 0; i < kDim / kWave; ++i) sum_sq = fmaf(x[i], x[i], sum_sq);
  sum_sq = wave_sum(sum_sq);
  return 1.0f / sqrtf(sum_sq / (float)kDim + kRmsEps);
}

// Learned RMSNorm, then RoPE over the first kRotary dims (pairs d and
// d + kRotary/2), plain normalised tail (src/gemma4_flash_attention_decode.cu:233-269).
template <int kDim, int kRotary>
__device__ __forceinline__ void store_weighted_rope(uint16_t *out, const float (&x)[kDim / kWave],
                                                    const uint16_t *weight, const float *cos_row,
                                                    const float *sin_row, int lane) {
  constexpr int kPer = kDim / kWave;
  constexpr int kHalf = kRotary / 2;
  constexpr int kPairSteps = kHalf / kWave;  // lane-strided steps inside the first half
  static_assert(kDim % kWave == 0 && kHalf % kWave == 0, "lane-strided pairs");
  const float scale = head_rms_scale<kDim>(x);
  float y[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) y[i] = x[i] * scale * bf16_bits_to_f32(weight[lane + i * kWave]);
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int d = lane + i * kWave;
    float r;
    if (i < kPairSteps) {  // d in the first rotary half
      const float c = cos_row[d], s = sin_row[d];
      r = fmaf(-y[i + kPairSteps], s, y[i] * c);
    } else if (i < 2 * kPairSteps) {  // d in the second rotary half
      const float c = cos_row[d - kHalf], s = sin_row[d - kHalf];
      r = fmaf(y[i - kPairSteps], s, y[i] * c);
    } else {
      r = y[i];
    }
    out[d] = (uint16_t)f32_to_bf16_bits(r);
  }
}

// Scale-free RMSNorm (src/gemma4_flash_attention_decode.cu:271-283).
template <int kDim>
__device__ __forceinline__ void store_scale_free(uint16_t *out, const float (&x)[kDim / kWave],
                                                 int lane) {
  const float scale = head_rms_scale<kDim>(x);
#pragma unroll
  for (int i = 0; i < kDim / kWave; ++i)
    out[lane + i * kWave] = (uint16_t)f32_to_bf16_bits(x[i] * scale);
}

// Waves per workgroup of a prep kernel over one (token, kv head): the query
// heads of the kv head, then K and V for the 8x256 geometry; for the 1x512
// geometry (16 query heads) wave 0 also does K and the K-derived V, keeping
// the workgroup at 16 waves.
template <int kHeads, bool kHasV>
constexpr int prep_waves() {
  return kHasV ? kQueryHeads / kHeads + 2 : kQueryHeads / kHeads;
}

}  // namespace gemma4
