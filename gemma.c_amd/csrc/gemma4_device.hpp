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
// Streaming read of K/V data touched once per launch: the nontemporal hint
// keeps it from displacing reused lines (flags, partials, tables) in L2.
__device__ __forceinline__ uint4 load128_stream(const void *p) {
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
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

// a.lo*b.lo + a.hi*b.hi + c for packed bf16 pairs (v_dot2c_f32_bf16): the
// products are exact in fp32 and the sum is rounded once per step.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                        __builtin_bit_cast(bf16x2_t, b), c, false);
}

// ---- cross-lane exchanges (wave64) ----------------------------------------
template <int kCtrl>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}
template <int kMask>
__device__ __forceinline__ float swizzle_xor(float v) {
  static_assert(kMask > 0 && kMask < 32, "ds_swizzle bitmask mode works within 32 lanes");
  return __builtin_bit_cast(
      float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x1F | (kMask << 10)));
}
__device__ __forceinline__ float xor_lane32(float v) {
  const unsigned bits = __builtin_bit_cast(unsigned, v);
  const auto swapped = __builtin_amdgcn_permlane32_swap(bits, bits, false, false);
  return __builtin_bit_cast(float, __lane_id() < 32 ? swapped[1] : swapped[0]);
}

// Value of lane (lane ^ 16) with v_permlane16_swap (a VALU exchange of
// adjacent 16-lane rows, no LDS round trip): with both operands x, result
// [1] holds the odd rows' values in the even rows and [0] the even rows'
// values in the odd rows.
__device__ __forceinline__ float xor_lane16(float v) {
  const unsigned bits = __builtin_bit_cast(unsigned, v);
  const auto swapped = __builtin_amdgcn_permlane16_swap(bits, bits, false, false);
  return __builtin_bit_cast(float, (__lane_id() & 16) == 0 ? swapped[1] : swapped[0]);
}

// Value of lane (lane ^ kMask): quad DPP for 1 and 2, two row rotates and a
// select for 4, DPP row_ror:8 for 8 (rotating a 16-lane row by 8 is exactly
// xor 8), v_permlane16_swap for 16, permlane32 swap across the two halves of
// the wave; a mask of several bits is one exchange per group of bits. All
// are VALU exchanges without an LDS round trip (ds_swizzle remains only for
// masks spanning bits 3 and 4 together).
template <int kMask>
__device__ __forceinline__ float lane_xor(float v) {
  static_assert(kMask > 0 && kMask < kWave, "lane mask");
  if constexpr (kMask == 1) {
    return dpp_move<0xB1>(v);  // quad_perm [1,0,3,2]
  } else if constexpr (kMask == 2) {
    return dpp_move<0x4E>(v);  // quad_perm [2,3,0,1]
  } else if constexpr (kMask == 4) {
    // Within a 16-lane row: lanes with bit 2 set read lane - 4 (row_ror:4),
    // the others lane + 4 (row_ror:12).
    const float down = dpp_move<0x124>(v), up = dpp_move<0x12C>(v);
    return (__lane_id() & 4) ? down : up;
  } else if constexpr (kMask == 8) {
    return dpp_move<0x128>(v);  // row_ror:8
  } else if constexpr (kMask == 16) {
    return xor_lane16(v);
  } else if constexpr (kMask < 32 && (kMask & 7) != 0 && (kMask & ~7) != 0) {
    // Masks over both the quad/row bits and bits 3..4: one exchange each.
    return lane_xor<kMask & ~7>(lane_xor<kMask & 7>(v));
  } else if constexpr (kMask < 32 && (kMask & 3) != 0 && (kMask & 4) != 0) {
    return lane_xor<4>(lane_xor<kMask & 3>(v));
  } else if constexpr (kMask < 32) {
    return swizzle_xor<kMask>(v);
  } else if constexpr (kMask == 32) {
    return xor_lane32(v);
  } else {
    return xor_lane32(lane_xor<kMask - 32>(v));
  }
}

// v_permlane32_swap / v_permlane16_swap of (a, b): lanes whose bit 5 (bit 4)
// is clear receive b from their partner lane ^ 32 (^ 16) in place of their
// own b, the others receive a from the partner in place of their own a. So
// result[0] + result[1] is, in a lane with the bit clear, a + a of the
// partner, and with the bit set, b of the partner + b: one swap serves a
// value-splitting butterfly step or, with a == b, a symmetric exchange.
template <int kMask>
__device__ __forceinline__ void swap_halves(float a, float b, float &x, float &y) {
  static_assert(kMask == 16 || kMask == 32, "VALU swaps exchange 16- or 32-lane halves");
  const unsigned ua = __builtin_bit_cast(unsigned, a), ub = __builtin_bit_cast(unsigned, b);
  const auto s = kMask == 32 ? __builtin_amdgcn_permlane32_swap(ua, ub, false, false)
                             : __builtin_amdgcn_permlane16_swap(ua, ub, false, false);
  unsigned sx = s[0], sy = s[1];
  // hipcc (ROCm 7.2) reads both results from the first result's register
  // when both feed further arithmetic (v_add v1, v1, v1 after the swap); an
  // empty asm on the pair keeps the second result's register.
  asm("" : "+v"(sx), "+v"(sy));
  x = __builtin_bit_cast(float, sx);
  y = __builtin_bit_cast(float, sy);
}

// v + (v of lane ^ kMask) and max(v, v of lane ^ kMask): for masks 16 and 32
// one swap and one add / max (the select of lane_xor is not needed for a
// symmetric operation; the result is bit-identical).
template <int kMask>
__device__ __forceinline__ float xor_sum(float v) {
  if constexpr (kMask == 16 || kMask == 32) {
    float x, y;
    swap_halves<kMask>(v, v, x, y);
    return x + y;
  } else {
    return v + lane_xor<kMask>(v);
  }
}
template <int kMask>
__device__ __forceinline__ float xor_max(float v) {
  if constexpr (kMask == 16 || kMask == 32) {
    float x, y;
    swap_halves<kMask>(v, v, x, y);
    return fmaxf(x, y);
  } else {
    return fmaxf(v, lane_xor<kMask>(v));
  }
}

// Value of a partner lane that differs from this lane in bit kBit and agrees
// on every higher bit (lower bits may differ); the pairing is an involution.
// Butterfly sums only need such a pairing, and row mirrors are plain DPP:
// bit 2 -> row_half_mirror (i <-> 7-i), bit 3 -> row_mirror (i <-> 15-i).
template <int kBit>
__device__ __forceinline__ float lane_pair(float v) {
  if constexpr (kBit == 4) {
    return dpp_move<0x141>(v);
  } else if constexpr (kBit == 8) {
    return dpp_move<0x140>(v);
  } else {
    return lane_xor<kBit>(v);
  }
}

// Wave-uniform value read from lane 0 (a scalar register after readfirstlane).
__device__ __forceinline__ int32_t wave_uniform(int32_t v) {
  return __builtin_amdgcn_readfirstlane(v);
}

}  // namespace gemma4
