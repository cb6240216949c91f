// Device helpers shared by the gfx950 kernels of the KV-cache path:
// bf16 packing, 128-bit global access and wave64 cross-lane operations.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

#include "gemma4_kv_cache.h"

namespace gemma4 {

constexpr int kWave = 64;            // CDNA wavefront width
constexpr int kPackElems = 8;        // bf16 elements per 128-bit pack
constexpr int kQueryHeads = 16;      // query heads of every gemma4 attention layer
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Low / high bf16 of a packed 32-bit word, widened exactly to fp32.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

__device__ __forceinline__ uint4 load128(const void *p) {
  return *reinterpret_cast<const uint4 *>(p);
}
__device__ __forceinline__ void store128(void *p, uint4 v) {
  *reinterpret_cast<uint4 *>(p) = v;
}

// Unpack a 128-bit pack of 8 bf16 into fp32 (element 0 in the low half of x).
__device__ __forceinline__ void unpack8(const uint4 &p, float (&f)[8]) {
  f[0] = bf16_lo(p.x); f[1] = bf16_hi(p.x);
  f[2] = bf16_lo(p.y); f[3] = bf16_hi(p.y);
  f[4] = bf16_lo(p.z); f[5] = bf16_hi(p.z);
  f[6] = bf16_lo(p.w); f[7] = bf16_hi(p.w);
}

// Cross-lane exchange within the wave (lane ^ mask).
__device__ __forceinline__ float xor_lane(float v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

// Wave-uniform value read from lane 0 (a scalar register after readfirstlane).
__device__ __forceinline__ int32_t wave_uniform(int32_t v) {
  return __builtin_amdgcn_readfirstlane(v);
}

}  // namespace gemma4
