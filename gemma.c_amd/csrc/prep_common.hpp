// Per-head preparation shared by the decode-token and prefill prep kernels
// (gfx950): learned RMSNorm + split-half RoPE (Q, K) and scale-free RMSNorm
// (V), one wave per head; a head's sum of squares is one wave reduction.
// Follows src/gemma4_flash_attention_decode.cu:216-283,
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

// A wave holds a head in contiguous runs: lane l owns dims
// [l * kPer, (l + 1) * kPer), kPer = D / 64, loaded and stored as one
// vector. A rotary pair (d, d + R/2) then sits in lanes l and
// l + (R/2) / kPer, one cross-lane exchange apart.
template <int kDim>
struct HeadLayout {
  static constexpr int kPer = kDim / kWave;
  static_assert(kPer == 4 || kPer == 8, "4 or 8 bf16 per lane");
};

// Loads kPer consecutive bf16 as fp32.
template <int kPer>
__device__ __forceinline__ void load_run(const uint16_t *src, float (&x)[kPer]) {
  if constexpr (kPer == 4) {
    const uint2 w = *reinterpret_cast<const uint2 *>(src);
    x[0] = bf16_lo(w.x); x[1] = bf16_hi(w.x); x[2] = bf16_lo(w.y); x[3] = bf16_hi(w.y);
  } else {
    const uint4 w = *reinterpret_cast<const uint4 *>(src);
    unpack8(w, x);
  }
}

template <int kPer>
__device__ __forceinline__ void store_run(uint16_t *dst, const float (&y)[kPer]) {
  if constexpr (kPer == 4) {
    *reinterpret_cast<uint2 *>(dst) = make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
  } else {
    *reinterpret_cast<uint4 *>(dst) =
        make_uint4(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]), pack_bf16x2(y[4], y[5]),
                   pack_bf16x2(y[6], y[7]));
  }
}

// Loads one head (this lane's run) as fp32.
template <int kDim>
__device__ __forceinline__ void load_head(const uint16_t *src, float (&x)[kDim / kWave], int lane) {
  constexpr int kPer = HeadLayout<kDim>::kPer;
  load_run<kPer>(src + lane * kPer, x);
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
  constexpr int kPer = HeadLayout<kDim>::kPer;
  constexpr int kHalf = kRotary / 2;
  constexpr int kPartner = kHalf / kPer;  // lane distance of a rotary pair
  static_assert(kHalf % kPer == 0 && kPartner < kWave, "pairs in whole lanes");
  const float scale = head_rms_scale<kDim>(x);
  const int d0 = lane * kPer;
  float wv[kPer];
  load_run<kPer>(weight + d0, wv);
  float y[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) y[i] = x[i] * scale * wv[i];
  float partner[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) partner[i] = lane_xor<kPartner>(y[i]);
  float r[kPer];
  if (d0 < kRotary) {
    const int pair = d0 < kHalf ? d0 : d0 - kHalf;
    const float sign = d0 < kHalf ? -1.0f : 1.0f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const float c = cos_row[pair + i], s = sin_row[pair + i];
      r[i] = fmaf(sign * partner[i], s, y[i] * c);
    }
  } else {
#pragma unroll
    for (int i = 0; i < kPer; ++i) r[i] = y[i];
  }
  store_run<kPer>(out + d0, r);
}

// Scale-free RMSNorm (src/gemma4_flash_attention_decode.cu:271-283).
template <int kDim>
__device__ __forceinline__ void store_scale_free(uint16_t *out, const float (&x)[kDim / kWave],
                                                 int lane) {
  constexpr int kPer = HeadLayout<kDim>::kPer;
  const float scale = head_rms_scale<kDim>(x);
  float y[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) y[i] = x[i] * scale;
  store_run<kPer>(out + lane * kPer, y);
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
