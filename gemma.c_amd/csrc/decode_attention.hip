// Paged split-K decode attention for gfx950 (flash decoding), with an
// optional fused K/V append. Replaces the decode-attention phases of
// src/gemma4_flash_attention_decode.cu (phase_decode_paged_grouped_split,
// phase_decode_paged_reduce, phase_decode_q_paged_kv_norm_rope's cache write).
//
// Work decomposition
//   workgroup (kv_head, split, batch)   grid = (num_heads, num_splits, batch)
//   wave                                a key tile of kTileKeys keys at a time
//   lane (r, c)                         c = dim pack (8 bf16 = 16 bytes) of
//                                       key row r of each 128-bit load
// A K/V row of D bf16 is read by D/8 lanes with one 16-byte load each, so one
// wave-wide load instruction covers 64/(D/8) full rows: every load is 128-bit
// and fully coalesced. Q·K partial dots are reduced across the D/8 lanes of a
// row with a value-splitting butterfly (each exchange halves the number of
// values a lane carries), which leaves exactly one (key, head) score per lane.
// The online softmax then needs one wave reduction per key tile — there is no
// per-key barrier — and P·V accumulates in registers, each lane owning 8
// output dims of every GQA head. Probabilities travel from the score lanes to
// the V lanes through a 64-float LDS slot per wave.
// Per-key page-table lookups are made once per tile (one key per lane) and
// shared through a 64-entry LDS table; the next tile's lookups are issued
// before the current tile's math so their latency overlaps it.
// Scores live in the log2 domain (q pre-scaled by softmax_scale*log2(e)); the
// stored split maxima are converted back to the reference's natural-log units.
#include "gemma4_device.hpp"
#include "decode_common.hpp"
#include "lds_copy.hpp"
#include "prep_common.hpp"

#include "gemma4_flash_attention.h"

#include <algorithm>
#include <math.h>
#include <mutex>

// Scratch of the allocation-free entry point
// (gemma4_flash_attention_append_decode_paged_bf16_noalloc): the split
// partials m, l, acc of one call, carved from this file-scope array. Each GPU
// the library runs on holds its own copy (40 MiB) until the process ends;
// host code reaches it only through the per-device address that
// hipGetSymbolAddress returns (noalloc_scratch below).
constexpr size_t kNoAllocScratchBytes = size_t(40) << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

// Development builds only (-DSPLIT_TRACE=1): real-time stamps of the split
// kernel's phases, [workgroup][wave][8], read with gemma4_debug_split_trace.
#ifndef SPLIT_TRACE
#define SPLIT_TRACE 0
#endif
#if SPLIT_TRACE
__device__ uint64_t g_split_trace[8192 * 4 * 8];
#define SPLIT_MARK(k)                                                                        \
  do {                                                                                       \
    if (__lane_id() == 0)                                                                    \
      g_split_trace[(((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * \
                        32 +                                                                 \
                    (threadIdx.x / 64) * 8 + (k)] = __builtin_amdgcn_s_memrealtime();        \
  } while (0)
extern "C" hipError_t gemma4_debug_split_trace(void *dst, size_t bytes) {
  return hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_split_trace), bytes, 0, hipMemcpyDeviceToHost);
}
#else
#define SPLIT_MARK(k) \
  do {                \
  } while (0)
#endif

namespace gemma4 {
namespace {

constexpr int kMaxWaves = 4;


template <int kHeads, int kDim, int kHeadsPerWave, int kLoads, int kChunkTiles,
          int kWaves = kMaxWaves>
struct DecodeShape {
  static constexpr int G = kQueryHeads / kHeads;          // GQA group
  static constexpr int GW = kHeadsPerWave;                // heads per wave
  static constexpr int HG = G / GW;                       // head groups per kv head
  static constexpr int LPR = kDim / kPackElems;           // lanes per key row
  static constexpr int RPL = kWave / LPR;                 // rows per load
  static constexpr int LOADS = kLoads;                    // loads per lane per tile
  static constexpr int KT = RPL * kLoads;                 // keys per tile
  static constexpr int CT = kChunkTiles;                  // tiles per page-lookup chunk
  static constexpr int NP = kLoads * GW;                  // partial dots per lane
  static constexpr int S = __builtin_ctz(LPR / NP);       // duplicate-lane bits
  static constexpr int GB = __builtin_ctz(GW);            // head-select bits
  static constexpr int kRowElems = kHeads * kDim;
  // Rotary dims of the geometry: all of a sliding head, a quarter of a
  // global one (src/gemma4.h rotary settings).
  static constexpr int kRot = kHeads == 1 ? kDim / 4 : kDim;
  static constexpr int kMaxW = kWaves;  // waves of a split workgroup at most
  // Staged shapes: two waves per head group take alternate 8-key tiles that
  // the workgroup copies into LDS once (all heads read every key).
  static constexpr bool kStaged = kWaves == 2 * HG;
  static_assert(G % GW == 0, "heads per wave must divide the GQA group");
  static_assert(NP <= LPR, "one reduced score per lane at most");
  static_assert((NP & (NP - 1)) == 0 && (GW & (GW - 1)) == 0, "powers of two");
  static_assert(KT * kChunkTiles <= kWave, "one page lookup per lane per chunk");
  static_assert(RPL * NP <= kWave, "probability slot holds one tile");
};


// Log-sum-exp combine of `splits` partials for GW consecutive query heads
// starting at q_head0 of batch b, by one wave of the last-arriving split
// workgroup, reading the other workgroups' partials with coherent loads that
// are issued in independent batches (one memory round trip per batch).
// Lane (r, cpack) owns dims [8*cpack, 8*cpack+8) and takes the splits
// s == r (mod RPL); the RPL row groups are summed at the end. Same
// arithmetic as decode_combine_kernel.
template <int GW, int D, int LPR, int RPL>
__device__ __forceinline__ void combine_row_group(const DecodeParams &p, int32_t b,
                                                  int32_t q_head0, int32_t splits,
                                                  int r, int cpack) {
  constexpr int kBatch = 8;
  const int lane = __lane_id();
#pragma unroll 1
  for (int g = 0; g < GW; ++g) {
    const int64_t row = (int64_t)b * kQueryHeads + q_head0 + g;
    const auto pm = coherent_view(p.partial_m + row * p.num_splits, splits);
    const auto pl = coherent_view(p.partial_l + row * p.num_splits, splits);
    const auto pa = coherent_view(p.partial_acc + row * p.num_splits * D, splits * D);
    float big_m = -INFINITY;
    for (int32_t s0 = 0; s0 < splits; s0 += kWave * 4) {
      float mv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int32_t s = s0 + i * kWave + lane;
        mv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pm, s * 4, 0, kCoherentAux));
        mv[i] = s < splits ? mv[i] : -INFINITY;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) big_m = fmaxf(big_m, mv[i]);
    }
    big_m = reduce_max_from<1>(big_m);
    float big_l = 0.0f;
    float sum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int32_t s0 = r; s0 < splits; s0 += kBatch * RPL) {
      float ms[kBatch], ls[kBatch];
      u32x4 lo[kBatch], hi[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int32_t s = s0 + i * RPL;  // past `splits`: reads 0, weight 0
        ms[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pm, s * 4, 0, kCoherentAux));
        ls[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(pl, s * 4, 0, kCoherentAux));
        const int32_t off = (s * D + cpack * 8) * 4;
        lo[i] = __builtin_amdgcn_raw_buffer_load_b128(pa, off, 0, kCoherentAux);
        hi[i] = __builtin_amdgcn_raw_buffer_load_b128(pa, off + 16, 0, kCoherentAux);
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const float w = ls[i] > 0.0f ? __builtin_amdgcn_exp2f((ms[i] - big_m) * kLog2e) : 0.0f;
        big_l = fmaf(ls[i] > 0.0f ? ls[i] : 0.0f, w, big_l);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sum[j] = fmaf(__uint_as_float(lo[i][j]), w, sum[j]);
          sum[4 + j] = fmaf(__uint_as_float(hi[i][j]), w, sum[4 + j]);
        }
      }
    }
    big_l = sum_rows<LPR>(big_l);
#pragma unroll
    for (int j = 0; j < 8; ++j) sum[j] = sum_rows<LPR>(sum[j]);
    if (r == 0) {
      const float inv = (splits > 0 && big_l > 0.0f) ? 1.0f / big_l : 0.0f;
      uint4 o;
      o.x = pack_bf16x2(sum[0] * inv, sum[1] * inv);
      o.y = pack_bf16x2(sum[2] * inv, sum[3] * inv);
      o.z = pack_bf16x2(sum[4] * inv, sum[5] * inv);
      o.w = pack_bf16x2(sum[6] * inv, sum[7] * inv);
      store128(p.out + row * D + cpack * kPackElems, o);
    }
  }
}

// RMSNorm (learned weight, or scale-free with weight == null) and split-half
// RoPE over the first kRot dims of one head held in this kernel's layout:
// lane c of a row holds dims [8c, 8c + 8) of the D = 8 * LPR dims, so the sum
// of squares is a reduction over the LPR lanes of the row and the rotary
// partner of dim d (d + kRot/2 or d - kRot/2) sits kRot/16 lanes away.
// Follows src/gemma4_flash_attention_decode.cu:233-283 and
// src/gemma4_rope.cu:8-20; the result is rounded to bf16 as the reference
// stores prepared rows.
template <int LPR, int kRot>
__device__ __forceinline__ uint4 prep_pack(uint4 raw, const uint16_t *weight,
                                           const float *cos_row, const float *sin_row,
                                           int cpack) {
  float x[8];
  unpack8(raw, x);
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = fmaf(x[i], x[i], ss);
  ss += lane_xor<1>(ss);
  ss += lane_xor<2>(ss);
  ss += lane_xor<4>(ss);
  ss += lane_xor<8>(ss);
  ss = xor_sum<16>(ss);
  if constexpr (LPR == 64) ss = xor_sum<32>(ss);
  const float scale = 1.0f / sqrtf(ss / (float)(LPR * kPackElems) + kRmsEps);
  float y[8];
  if (weight == nullptr) {
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = x[i] * scale;
  } else {
    float w[8];
    unpack8(load128(weight + cpack * kPackElems), w);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = x[i] * scale * w[i];
    constexpr int kHalf = kRot / 2;
    float partner[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) partner[i] = lane_xor<kHalf / kPackElems>(y[i]);
    const int d0 = cpack * kPackElems;
    if (d0 < kRot) {
      const int pair = d0 < kHalf ? d0 : d0 - kHalf;
      const float sign = d0 < kHalf ? -1.0f : 1.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = fmaf(sign * partner[i], sin_row[pair + i], y[i] * cos_row[pair + i]);
    }
  }
  return make_uint4(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]), pack_bf16x2(y[4], y[5]),
                    pack_bf16x2(y[6], y[7]));
}

// The inputs prep_pack reads besides the row, loaded ahead of the math: the
// lane's 8 weights (packed bf16) and cos / sin of its rotary pair.
struct PrepInputs {
  uint4 w;
  float4 c0, c1, s0, s1;
};
template <int LPR, int kRot>
__device__ __forceinline__ PrepInputs prep_inputs(const uint16_t *weight, const float *cos_row,
                                                  const float *sin_row, int cpack) {
  PrepInputs in;
  in.w = weight != nullptr ? load128(weight + cpack * kPackElems) : make_uint4(0, 0, 0, 0);
  const int d0 = cpack * kPackElems;
  const int pair = d0 < kRot / 2 ? d0 : d0 - kRot / 2;
  const bool rot = weight != nullptr && d0 < kRot;
  // Scalar loads: the tables come through the C-ABI with no alignment promise.
  const float *cr = rot ? cos_row + pair : nullptr;
  const float *sr = rot ? sin_row + pair : nullptr;
  in.c0 = rot ? make_float4(cr[0], cr[1], cr[2], cr[3]) : make_float4(0.f, 0.f, 0.f, 0.f);
  in.c1 = rot ? make_float4(cr[4], cr[5], cr[6], cr[7]) : make_float4(0.f, 0.f, 0.f, 0.f);
  in.s0 = rot ? make_float4(sr[0], sr[1], sr[2], sr[3]) : make_float4(0.f, 0.f, 0.f, 0.f);
  in.s1 = rot ? make_float4(sr[4], sr[5], sr[6], sr[7]) : make_float4(0.f, 0.f, 0.f, 0.f);
  return in;
}
// prep_pack's arithmetic on preloaded inputs (weighted: learned RMSNorm +
// RoPE; otherwise the scale-free RMSNorm), the same operations in the same
// order.
template <int LPR, int kRot>
__device__ __forceinline__ uint4 prep_math(uint4 raw, bool weighted, const PrepInputs &in,
                                           int cpack) {
  float x[8];
  unpack8(raw, x);
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = fmaf(x[i], x[i], ss);
  ss += lane_xor<1>(ss);
  ss += lane_xor<2>(ss);
  ss += lane_xor<4>(ss);
  ss += lane_xor<8>(ss);
  ss = xor_sum<16>(ss);
  if constexpr (LPR == 64) ss = xor_sum<32>(ss);
  const float scale = 1.0f / sqrtf(ss / (float)(LPR * kPackElems) + kRmsEps);
  float y[8];
  if (!weighted) {
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = x[i] * scale;
  } else {
    float w[8];
    unpack8(in.w, w);
#pragma unroll
    for (int i = 0; i < 8; ++i) y[i] = x[i] * scale * w[i];
    constexpr int kHalf = kRot / 2;
    float partner[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) partner[i] = lane_xor<kHalf / kPackElems>(y[i]);
    const int d0 = cpack * kPackElems;
    if (d0 < kRot) {
      const float sign = d0 < kHalf ? -1.0f : 1.0f;
      const float c[8] = {in.c0.x, in.c0.y, in.c0.z, in.c0.w, in.c1.x, in.c1.y, in.c1.z, in.c1.w};
      const float sn[8] = {in.s0.x, in.s0.y, in.s0.z, in.s0.w, in.s1.x, in.s1.y, in.s1.z, in.s1.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) y[i] = fmaf(sign * partner[i], sn[i], y[i] * c[i]);
    }
  }
  return make_uint4(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]), pack_bf16x2(y[4], y[5]),
                    pack_bf16x2(y[6], y[7]));
}

template <class Sh>
__global__ __launch_bounds__(Sh::kMaxW * kWave) void decode_split_kernel(DecodeParams p) {
  constexpr int G = Sh::G, GW = Sh::GW, HG = Sh::HG, LPR = Sh::LPR, RPL = Sh::RPL;
  constexpr int LOADS = Sh::LOADS, KT = Sh::KT, NP = Sh::NP, S = Sh::S;
  constexpr int D = LPR * kPackElems;

  __shared__ int32_t s_rows[Sh::kMaxW][2][kWave];
  __shared__ float s_prob[Sh::kMaxW][kWave];
  __shared__ float s_ml[Sh::kMaxW][2][GW];
  // Staged shapes: kStages stages of K and V rows for kStepKeys keys (one
  // KT-key tile per key lane per step), rows of kWindowKeys keys at a time.
  constexpr int kStages = 2;
  constexpr int kLanes = Sh::kMaxW / HG;  // key lanes: tiles per step
  constexpr int kStepKeys = kLanes * KT;
  constexpr int kWindowKeys = Sh::kMaxW * kWave;
  constexpr int kStageUint4 = Sh::kStaged ? kStages * 2 * kStepKeys * LPR : 0;
  constexpr int kAccUint4 = Sh::kMaxW * GW * D / 4;
  // The cross-wave merge buffer s_acc shares LDS with the stages: the merge
  // runs after the last step's barrier.
  __shared__ __attribute__((aligned(1024)))
  uint4 s_lds[kStageUint4 > kAccUint4 ? kStageUint4 : kAccUint4];
  auto s_acc = reinterpret_cast<float (*)[GW][D]>(&s_lds[0]);

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = wave_uniform(threadIdx.x / kWave);  // scalar: wave-uniform control flow
  const int waves = wave_uniform(blockDim.x / kWave);
  const int hg = wave % HG;                 // head group of this wave
  const int key_lane = wave / HG;           // key-tile slot among same-group waves
  const int key_lanes = waves / HG;
  const int r = lane / LPR;                 // key row within a load
  const int cpack = lane % LPR;             // 16-byte pack within the row

  const int32_t split = blockIdx.y;  // heads fastest: co-running workgroups read whole token rows
  const int32_t head = blockIdx.x;
  const int32_t b = blockIdx.z;
  const Gemma4KvCacheConfig &c = p.c;

  SPLIT_MARK(0);
  // Split keys. A global cache's split covers positions split * split_size
  // onward whatever the length. A ring that is full (every one of its
  // ring_keys slots holds a live position) is split by slot instead: slot j
  // holds the one live position congruent to j modulo ring_keys, and its
  // page-table entry is entry j / page_size. In both cases the page-table
  // entry of this lane's first key is known before the length arrives and
  // is requested first (one dependent round trip fewer before the first
  // tile); a ring that turns out not to be full refetches it by position.
  const int32_t ring_keys = c.max_pages_per_seq * c.page_size;
  // 64-bit: this load precedes the live-split check, and a split past the
  // live ones may lie beyond int32 keys; the entry stays inside the row.
  const int64_t key0 = (int64_t)split * p.split_size +
                       ((lane / Sh::KT) * key_lanes + key_lane) * Sh::KT + lane % Sh::KT;
  // The per-sequence words the split depends on are all requested at once,
  // before anything waits: the length, the token position and the gate word
  // (an absent one reads the length's word and is ignored).
  const int32_t *tok_src = p.token_position != nullptr ? p.token_position + b : p.seq_lengths + b;
  const int32_t *gate_src = p.gate != nullptr ? p.gate : p.seq_lengths + b;
  const int32_t seq_word = p.seq_lengths[b];
  const int32_t tok_word = *tok_src;
  const int32_t gate_word = *gate_src;
  const int32_t early_page = Sh::kStaged ? 0
      : p.page_table[b * c.max_pages_per_seq +
                     (int32_t)((key0 / c.page_size) % c.max_pages_per_seq)];
  const int32_t seq_len = wave_uniform(seq_word);
  const int32_t token_pos = p.token_position != nullptr ? wave_uniform(tok_word) : -1;
  int32_t first = c.window_size > 0 ? seq_len - c.window_size : 0;
  first = first < 0 ? 0 : first;
  const int32_t key_count = seq_len > first ? seq_len - first : 0;
  const int32_t live_splits = (key_count + p.split_size - 1) / p.split_size;
  const bool direct = p.num_splits == 1;
  const bool by_slot =
      !Sh::kStaged && p.slot_splits != 0 && c.window_size > 0 && key_count == ring_keys;
  const bool early_ok = !Sh::kStaged && (c.window_size == 0 || by_slot);

  if (p.gate != nullptr && wave_uniform(gate_word) != 0) {
    // A failed step: no append; a direct launch zeroes its rows (the
    // combine kernel zeroes them otherwise).
    if (direct && split == 0) {
      uint16_t *rows = p.out + ((int64_t)b * kQueryHeads + head * G) * D;
      for (int e = threadIdx.x; e < G * D / kPackElems; e += blockDim.x)
        store128(rows + e * kPackElems, make_uint4(0, 0, 0, 0));
    }
    return;
  }

  // ---- fused append of the current token (one split per (b, head) owns it)
  int32_t new_pos = -1, new_row = -1;
  const bool prep = p.q_norm_weight != nullptr;
  // Without preparation the owner stores the token's K/V rows after its
  // attention work (append_late): the attention reads the new key from
  // new_k / new_v, so the append row's dependent page-table load stays off
  // the path to the first tile. Its entry is requested here.
  bool late_append = false;
  int32_t late_physical = -1;
  if (p.token_position != nullptr) {
    new_pos = token_pos;
    const bool in_live = new_pos >= first && new_pos < seq_len;
    const int32_t owner =
        !in_live ? 0 : (by_slot ? new_pos % ring_keys : new_pos - first) / p.split_size;
    // Only the owning split needs the cache row; no other split's key range
    // holds the new token.
    const bool owns = split == owner;
    if (!prep) {
      // The reference's skip rules (append_row): no position, or a global
      // cache position past its capacity.
      const bool droppable = new_pos < 0 || b >= c.batch_size ||
                             (c.window_size == 0 && new_pos / c.page_size >= c.max_pages_per_seq);
      late_append = owns && !droppable;
      if (late_append) {
        late_physical = p.page_table[b * c.max_pages_per_seq +
                                     (new_pos / c.page_size) % c.max_pages_per_seq];
      }
      // The new key attends from new_k / new_v when live and storable (an
      // unmapped page makes its row invalid in the key-row lookups).
      if (!in_live || droppable) new_pos = -1;
    }
    new_row = owns && prep ? wave_uniform(append_row(c, p.page_table, p.layer, b, new_pos)) : -1;
    const bool writes = owns && new_row >= 0;
    if (prep) {
      // Wave 0 prepares the token's K and V rows (both lane rows compute, the
      // first stores) and writes them; the workgroup then reads the new key
      // from the cache like any other, after the stores have completed.
      if (writes && wave == 0) {
        const int64_t src = ((int64_t)b * c.num_heads + head) * D + cpack * kPackElems;
        const float *cos_row = p.cos + (int64_t)new_pos * (Sh::kRot / 2);
        const float *sin_row = p.sin + (int64_t)new_pos * (Sh::kRot / 2);
        const uint4 raw_k = load128(p.new_k + src);
        const uint4 kp = prep_pack<LPR, Sh::kRot>(raw_k, p.k_norm_weight, cos_row, sin_row, cpack);
        // The 1x512 geometry derives V from the raw K (no V projection).
        const uint4 raw_v = p.new_v != nullptr ? load128(p.new_v + src) : raw_k;
        const uint4 vp = prep_pack<LPR, Sh::kRot>(raw_v, nullptr, cos_row, sin_row, cpack);
        if (r == 0) {
          const int64_t dst = (int64_t)new_row * Sh::kRowElems + (int64_t)head * D +
                              cpack * kPackElems;
          store128(p.cache_k + dst, kp);
          store128(p.cache_v + dst, vp);
        }
        wait_stores_complete();
      }
      if (writes) __syncthreads();
      new_pos = -1;
    }
  }
  auto append_late = [&]() __attribute__((always_inline)) {
    if (!late_append) return;
    const int32_t physical = wave_uniform(late_physical);
    if (physical < 0 || physical >= c.num_pages || threadIdx.x >= LPR) return;
    const int32_t pos = token_pos;
    const int32_t logical_page = pos / c.page_size;
    const int64_t row = ((int64_t)p.layer * c.num_pages + physical) * c.page_size +
                        (pos - logical_page * c.page_size);
    const int64_t src = ((int64_t)b * c.num_heads + head) * D + threadIdx.x * kPackElems;
    const int64_t dst = row * Sh::kRowElems + (int64_t)head * D + threadIdx.x * kPackElems;
    store128(p.cache_k + dst, load128(p.new_k + src));
    store128(p.cache_v + dst, load128(p.new_v + src));
  };

  if (key_count == 0 && direct) {
    // No live key: the row is defined as zeros (src/...decode.cu:733-743).
    if (key_lane == 0 && r == 0) {
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        const int qh = head * G + hg * GW + g;
        store128(p.out + ((int64_t)b * kQueryHeads + qh) * D + cpack * kPackElems,
                 make_uint4(0, 0, 0, 0));
      }
    }
    append_late();
    return;
  }
  if (split >= live_splits) {
    append_late();
    return;
  }

  // Keys of this split: positions, or ring slots when by_slot.
  const int32_t begin = (by_slot ? 0 : first) + split * p.split_size;
  const int32_t end = min(by_slot ? ring_keys : seq_len, begin + p.split_size);
  // The appended token's key in the same numbering (-1: none).
  const int32_t new_key = new_pos < 0 ? -1 : (by_slot ? new_pos % ring_keys : new_pos);

  SPLIT_MARK(1);
  // ---- Q for the GW heads of this wave, 8 dims per lane, pre-scaled
  // Q stays packed bf16 (two dims per register): Q·K runs on v_dot2 with
  // exact products and fp32 sums; the softmax scale is applied to the sum.
  uint32_t qw[GW][4];
  // With fused preparation q is normalised and rotated here, at the token's
  // position (a sequence without a token this step uses q as given).
  // Memory loads complete in order. Without preparation q is loaded after
  // the first tile's loads are issued (ahead of them it would hold up the
  // page lookup they wait for); with preparation its loads and the norm
  // weights and RoPE rows go out before the tile loads (q_issue) and the
  // arithmetic runs while the tiles are in flight (q_finish).
  const bool prep_q = prep && token_pos >= 0;
  const int32_t q_pos = prep_q ? token_pos : 0;
  uint4 q_raw[GW];
  PrepInputs q_in{};
  auto q_issue = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      const int qh = head * G + hg * GW + g;
      q_raw[g] = load128(p.q + ((int64_t)b * kQueryHeads + qh) * D + cpack * kPackElems);
    }
    if (prep_q) {
      q_in = prep_inputs<LPR, Sh::kRot>(p.q_norm_weight, p.cos + (int64_t)q_pos * (Sh::kRot / 2),
                                        p.sin + (int64_t)q_pos * (Sh::kRot / 2), cpack);
    }
  };
  auto q_finish = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      const uint4 qp = prep_q ? prep_math<LPR, Sh::kRot>(q_raw[g], true, q_in, cpack) : q_raw[g];
      qw[g][0] = qp.x; qw[g][1] = qp.y; qw[g][2] = qp.z; qw[g][3] = qp.w;
    }
  };
  auto load_q = [&]() __attribute__((always_inline)) {
    q_issue();
    q_finish();
  };

  // Score-lane identity after the butterfly: one (key, head) per lane.
  const int idx = cpack >> S;               // index into the lane's NP partials
  const int my_g = idx & (GW - 1);
  const int my_kl = idx / GW;

  float m[GW], acc[GW][8];
#pragma unroll
  for (int g = 0; g < GW; ++g) {
    m[g] = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.0f;
  }
  float l_lane = 0.0f;

  const uint16_t *kbase = p.cache_k + (int64_t)head * D + cpack * kPackElems;
  const uint16_t *vbase = p.cache_v + (int64_t)head * D + cpack * kPackElems;
  const int64_t new_off = ((int64_t)b * c.num_heads + head) * D + cpack * kPackElems;

  // This wave's keys: the split's KT-key tiles key_lane, key_lane +
  // key_lanes, ... (so a short split still spreads over the waves and no
  // wave carries more than one tile beyond another), grouped CT tiles to a
  // chunk of kWave keys with one page lookup per lane.
  constexpr int CT = Sh::CT;
  constexpr int CK = CT * KT;  // keys per chunk
  const int32_t n_keys = end - begin;
  const int32_t n_tiles = (n_keys + KT - 1) / KT;
  const int32_t my_tiles =
      n_tiles > key_lane ? (n_tiles - key_lane + key_lanes - 1) / key_lanes : 0;
  const int32_t my_chunks = (my_tiles + CT - 1) / CT;
  // Page lookups are split in two so the page-table load can stay in flight
  // for a whole chunk: fetch_page issues the (always in-bounds) load for the
  // lane's key of my chunk m; page_row turns it into a cache row, branch-free.
  const int32_t pt_row = b * c.max_pages_per_seq;
  auto chunk_key = [&](int32_t m) {
    return begin + ((m * CT + lane / KT) * key_lanes + key_lane) * KT + lane % KT;
  };
  auto fetch_page = [&](int32_t m) -> int32_t {
    const int32_t logical_page = chunk_key(m) / c.page_size;
    return p.page_table[pt_row + logical_page % c.max_pages_per_seq];
  };
  auto page_row = [&](int32_t m, int32_t physical) -> int32_t {
    const int32_t key = chunk_key(m);
    const int32_t logical_page = key / c.page_size;
    const bool ok = lane < CK && m < my_chunks && key < end && physical >= 0 &&
                    physical < c.num_pages;
    const int32_t row = ((int32_t)p.layer * c.num_pages + physical) * c.page_size +
                        (key - logical_page * c.page_size);
    return !ok ? kRowInvalid : (key == new_key ? kRowNewToken : row);
  };
  // Lane l's key goes to slot (tile, r, kl) = (l / KT, l % RPL, (l % KT) / RPL)
  // so a lane reads its LOADS rows of a tile as one contiguous run.
  const int table_slot = (lane / KT) * KT + (lane % RPL) * LOADS + (lane % KT) / RPL;
  auto publish = [&](int32_t m, int32_t row) {
    if (lane < CK) s_rows[wave][m & 1][table_slot] = row;
    wave_lds_sync();
  };

  struct TileBuf {
    uint4 k[LOADS], v[LOADS];
    uint32_t valid;
  };
  // Issue tile t of my chunk m into `tb`; a tile past the wave's keys is
  // dead: every row reads as invalid (loads still go out, to cache row 0).
  auto issue = [&](TileBuf &tb, int32_t m, int t) {
    const bool live = m * CT + t < my_tiles;
    const int32_t *rows_p = &s_rows[wave][m & 1][t * KT + r * LOADS];
    int32_t rows[LOADS];
#pragma unroll
    for (int kl = 0; kl < LOADS; ++kl) rows[kl] = live ? rows_p[kl] : kRowInvalid;
    TileBuf &t_ = tb;
    // Loads are unconditional (no exec-mask branches, so the wait counters
    // stay exact across the pipeline); an invalid key reads cache row 0 and
    // is masked: its score becomes -inf and its V pack zero.
    t_.valid = 0;
#pragma unroll
    for (int kl = 0; kl < LOADS; ++kl) {
      const int32_t row = rows[kl];
      t_.valid |= (row != kRowInvalid ? 1u : 0u) << kl;
      const bool fresh = row == kRowNewToken;
      const int64_t off = (int64_t)(row < 0 ? 0 : row) * Sh::kRowElems;
      t_.k[kl] = load128_stream(fresh ? p.new_k + new_off : kbase + off);
      t_.v[kl] = load128_stream(fresh ? p.new_v + new_off : vbase + off);
    }
  };

  auto compute = [&](const TileBuf &t) {
    // Partial Q·K over this lane's 8 dims: part[kl * GW + g].
    float part[NP];
#pragma unroll
    for (int kl = 0; kl < LOADS; ++kl) {
      const uint32_t kw[4] = {t.k[kl].x, t.k[kl].y, t.k[kl].z, t.k[kl].w};
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        float acc_s = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc_s = dot2_bf16(qw[g][j], kw[j], acc_s);
        part[kl * GW + g] = acc_s;
      }
    }
    split_butterfly<NP, LPR / 2>(part, lane);
    const bool valid = (t.valid >> my_kl) & 1u;
    const float score = valid ? part[0] * p.q_scale : -INFINITY;

    // Online softmax, once per tile.
    float tmax[GW];
    gather_heads<GW, S>(reduce_max_from<(1 << S) * GW>(score), my_g, tmax);
    float alpha[GW], m_use[GW];
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      const float m_new = fmaxf(m[g], tmax[g]);
      m_use[g] = m_new == -INFINITY ? 0.0f : m_new;
      alpha[g] = __builtin_amdgcn_exp2f(m[g] - m_use[g]);
      m[g] = m_new;
    }
    float my_m = m_use[0], my_alpha = alpha[0];
#pragma unroll
    for (int g = 1; g < GW; ++g) {
      my_m = my_g == g ? m_use[g] : my_m;
      my_alpha = my_g == g ? alpha[g] : my_alpha;
    }
    const float prob = __builtin_amdgcn_exp2f(score - my_m);
    l_lane = l_lane * my_alpha + prob;

    // Probabilities to the V lanes: slot [r][kl * GW + g].
    s_prob[wave][r * NP + idx] = prob;
    wave_lds_sync();
    float pv[NP];
#pragma unroll
    for (int i = 0; i < NP; i += 4) {
      const float4 q4 = *reinterpret_cast<const float4 *>(&s_prob[wave][r * NP + i]);
      pv[i] = q4.x; pv[i + 1] = q4.y; pv[i + 2] = q4.z; pv[i + 3] = q4.w;
    }
#pragma unroll
    for (int g = 0; g < GW; ++g) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] *= alpha[g];
    }
    if constexpr (GW >= 4) {
      // GQA-heavy shapes (the 1x512 geometry's 16 heads per KV head are
      // VALU-bound): P.V on v_dot2 over key pairs (kl, kl + 1), with bf16
      // probability pairs and the V words regrouped by dim with one byte
      // permute per word pair (28.8 against 31.6 us at 8193 keys). The 8x256
      // shape keeps the fp32 FMA form: the dot2 form measured 1.7% slower on
      // the HBM-bound batch-64 leg.
      // Staged tiles hold zero rows for unreadable keys (their probability
      // is 0 as well), so only register-loaded tiles mask V.
#pragma unroll
      for (int kl = 0; kl < LOADS; kl += 2) {
        const bool ok0 = Sh::kStaged || ((t.valid >> kl) & 1u);
        const bool ok1 = Sh::kStaged || ((t.valid >> (kl + 1)) & 1u);
        const uint32_t a[4] = {ok0 ? t.v[kl].x : 0u, ok0 ? t.v[kl].y : 0u, ok0 ? t.v[kl].z : 0u,
                               ok0 ? t.v[kl].w : 0u};
        const uint32_t c[4] = {ok1 ? t.v[kl + 1].x : 0u, ok1 ? t.v[kl + 1].y : 0u,
                               ok1 ? t.v[kl + 1].z : 0u, ok1 ? t.v[kl + 1].w : 0u};
        uint32_t pp[GW];
#pragma unroll
        for (int g = 0; g < GW; ++g) {
          const bf16x2_t pair = {(__bf16)pv[kl * GW + g], (__bf16)pv[(kl + 1) * GW + g]};
          pp[g] = __builtin_bit_cast(uint32_t, pair);
        }
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
          const uint32_t lo = __builtin_amdgcn_perm(c[wi], a[wi], 0x05040100u);
          const uint32_t hi = __builtin_amdgcn_perm(c[wi], a[wi], 0x07060302u);
#pragma unroll
          for (int g = 0; g < GW; ++g) {
            acc[g][2 * wi] = dot2_bf16(pp[g], lo, acc[g][2 * wi]);
            acc[g][2 * wi + 1] = dot2_bf16(pp[g], hi, acc[g][2 * wi + 1]);
          }
        }
      }
    } else {
#pragma unroll
      for (int kl = 0; kl < LOADS; ++kl) {
        float vf[8];
        const bool kl_valid = (t.valid >> kl) & 1u;
        const uint4 vp = kl_valid ? t.v[kl] : make_uint4(0, 0, 0, 0);
        unpack8(vp, vf);
#pragma unroll
        for (int g = 0; g < GW; ++g) {
          const float w = pv[kl * GW + g];
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[g][j] = fmaf(w, vf[j], acc[g][j]);
        }
      }
    }
  };

  if constexpr (Sh::kStaged) {
    // Every head group (the 1 x 512 geometry: four groups of four heads)
    // attends to every key of the split, so each step of kStepKeys keys (one
    // KT-key tile per key lane) is copied into LDS once per workgroup -- wave
    // w copies the K and V rows of kRowsPerWave keys with global_load_lds,
    // or zeros for an unreadable key -- and the waves read it from there:
    // two waves per SIMD, one tile each. Two stages, one barrier per step: at
    // step i a wave waits for its own copies of step i, the barrier
    // publishes them and frees the stage of step i - 1, which then receives
    // step i + 1. Rows of the split's keys come from a table filled once per
    // window of kWindowKeys keys (one page-table load per thread).
    constexpr int kRowsPerWave = kStepKeys / Sh::kMaxW;
    static_assert(RPL == 1 && KT == LOADS && kStepKeys % Sh::kMaxW == 0 &&
                      kWindowKeys % kStepKeys == 0,
                  "one row per load; whole rows per wave per step");
    load_q();
    auto s_kv = reinterpret_cast<uint4 (*)[2][kStepKeys * LPR]>(&s_lds[0]);
    __shared__ int32_t s_keyrow[kWindowKeys];
    const uint32_t kv_lds = wave_uniform(lds_address(&s_lds[0]));
    constexpr uint32_t kRowBytesKV = D * 2;
    constexpr uint32_t kHalfBytes = kStepKeys * kRowBytesKV;  // K (or V) of one stage
    const uint64_t kcache = reinterpret_cast<uint64_t>(p.cache_k + (int64_t)head * D);
    const uint64_t vcache = reinterpret_cast<uint64_t>(p.cache_v + (int64_t)head * D);
    const uint64_t knew = reinterpret_cast<uint64_t>(p.new_k + ((int64_t)b * c.num_heads + head) * D);
    const uint64_t vnew = reinterpret_cast<uint64_t>(p.new_v + ((int64_t)b * c.num_heads + head) * D);
    const uint32_t lane_off = (uint32_t)lane * 16;
    auto copy_step = [&](int32_t step, int stage) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < kRowsPerWave; ++i) {
        const int kk = kRowsPerWave * wave + i;
        const int32_t row = wave_uniform(s_keyrow[step * kStepKeys + kk]);
        const uint32_t dst = stage * 2 * kHalfBytes + kk * kRowBytesKV;
        if (row == kRowInvalid) {
          s_kv[stage][0][kk * LPR + lane] = make_uint4(0, 0, 0, 0);
          s_kv[stage][1][kk * LPR + lane] = make_uint4(0, 0, 0, 0);
        } else {
          const uint64_t off = (uint64_t)(row < 0 ? 0 : row) * Sh::kRowElems * 2;
          const bool fresh = row == kRowNewToken;
          copy_row_pair((fresh ? knew : kcache + off) + lane_off, kv_lds + dst);
          copy_row_pair((fresh ? vnew : vcache + off) + lane_off, kv_lds + dst + kHalfBytes);
        }
      }
    };
    for (int32_t w0 = 0; w0 < n_keys; w0 += kWindowKeys) {
      const int32_t wkeys = min(kWindowKeys, n_keys - w0);
      {
        const int32_t e = threadIdx.x;
        const int32_t key = begin + w0 + e;
        int32_t row = kRowInvalid;
        if (e < wkeys) {
          row = key_row(c, p.page_table, p.layer, b, key);
          row = key == new_pos && row != kRowInvalid ? kRowNewToken : row;
        }
        s_keyrow[e] = row;
      }
      __syncthreads();
      const int32_t n_steps = (wkeys + kStepKeys - 1) / kStepKeys;
      copy_step(0, 0);
      for (int32_t i = 0; i < n_steps; ++i) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's copies of step i
        __syncthreads();
        if (i + 1 < n_steps) copy_step(i + 1, (i + 1) % kStages);
        const int stage = i % kStages;
        const int32_t t0 = (i * kLanes + key_lane) * KT;  // first key of my tile
        TileBuf tb;
        tb.valid = 0;
#pragma unroll
        for (int kl = 0; kl < LOADS; ++kl) {
          tb.valid |= (s_keyrow[t0 + kl] != kRowInvalid ? 1u : 0u) << kl;
          tb.k[kl] = s_kv[stage][0][(key_lane * KT + kl) * LPR + cpack];
          tb.v[kl] = s_kv[stage][1][(key_lane * KT + kl) * LPR + cpack];
        }
        compute(tb);
      }
      __syncthreads();  // the table and the stages are free for the next window
    }
  } else if (my_tiles > 0 && my_tiles <= 2) {
    // A wave with one or two tiles (the sliding layers' short splits) runs
    // them straight: the pipeline below would also issue the loads of the
    // dead tiles up to the end of the chunk and wait for them before exit.
    if (prep) q_issue();
    publish(0, page_row(0, early_ok ? early_page : fetch_page(0)));
    SPLIT_MARK(2);
    TileBuf buf0, buf1;
    issue(buf0, 0, 0);
    if (!prep) q_issue();
    q_finish();
    if (my_tiles == 2) {
      issue(buf1, 0, 1);
      compute(buf0);
      SPLIT_MARK(3);
      compute(buf1);
    } else {
      compute(buf0);
      SPLIT_MARK(3);
    }
  } else if (my_tiles > 0) {
  // Software pipeline over my chunks, CT tiles each, fully unrolled inside a
  // chunk so both register buffers are static: tile t+1's loads are in flight
  // while tile t computes, and the next chunk's page-table loads are in
  // flight for a whole chunk. Every load is issued on every path, so the
  // memory wait counters stay exact.
  static_assert(CT % 2 == 0, "tiles per chunk alternate between two buffers");
    if (prep) q_issue();
    publish(0, page_row(0, early_ok ? early_page : fetch_page(0)));
    SPLIT_MARK(2);
    int32_t next_page = fetch_page(1);
    TileBuf buf0, buf1;
    issue(buf0, 0, 0);
    if (!prep) q_issue();
    q_finish();
    for (int32_t m = 0; m < my_chunks; ++m) {
#pragma unroll
      for (int t = 0; t < CT; t += 2) {
        issue(buf1, m, t + 1);
        if (m * CT + t < my_tiles) compute(buf0);
        if (m == 0 && t == 0) SPLIT_MARK(3);
        if (t + 2 < CT) {
          issue(buf0, m, t + 2);
        } else {
          publish(m + 1, page_row(m + 1, next_page));
          next_page = fetch_page(m + 2);
          issue(buf0, m + 1, 0);
        }
        if (m * CT + t + 1 < my_tiles) compute(buf1);
      }
    }
  }

  SPLIT_MARK(4);
  // ---- wave totals: l per head, acc summed over the RPL key rows
  float l_head[GW];
  gather_heads<GW, S>(reduce_sum_from<(1 << S) * GW>(l_lane), my_g, l_head);
#pragma unroll
  for (int g = 0; g < GW; ++g) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = sum_rows<LPR>(acc[g][j]);
  }

  // ---- combine the waves that share a head group (LDS)
  if (key_lanes > 1) {
    if (lane == 0) {
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        s_ml[wave][0][g] = m[g];
        s_ml[wave][1][g] = l_head[g];
      }
    }
    if (r == 0) {
      // Two 16-byte stores per head (scalar stores at this 32-byte lane
      // stride would hit the same bank eight lanes at a time).
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        float4 *dst = reinterpret_cast<float4 *>(&s_acc[wave][g][cpack * 8]);
        dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
        dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
      }
    }
    __syncthreads();
    if (key_lane == 0) {
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        float big_m = -INFINITY;
        for (int k = 0; k < key_lanes; ++k) big_m = fmaxf(big_m, s_ml[k * HG + hg][0][g]);
        const float m_ref = big_m == -INFINITY ? 0.0f : big_m;
        float big_l = 0.0f;
        float sum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int k = 0; k < key_lanes; ++k) {
          const int w = k * HG + hg;
          const float f = __builtin_amdgcn_exp2f(s_ml[w][0][g] - m_ref);
          big_l = fmaf(s_ml[w][1][g], f, big_l);
          const float4 *src = reinterpret_cast<const float4 *>(&s_acc[w][g][cpack * 8]);
          const float4 a0 = src[0], a1 = src[1];
          sum[0] = fmaf(a0.x, f, sum[0]);
          sum[1] = fmaf(a0.y, f, sum[1]);
          sum[2] = fmaf(a0.z, f, sum[2]);
          sum[3] = fmaf(a0.w, f, sum[3]);
          sum[4] = fmaf(a1.x, f, sum[4]);
          sum[5] = fmaf(a1.y, f, sum[5]);
          sum[6] = fmaf(a1.z, f, sum[6]);
          sum[7] = fmaf(a1.w, f, sum[7]);
        }
        m[g] = big_m;
        l_head[g] = big_l;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[g][j] = sum[j];
      }
    }
  }

  SPLIT_MARK(5);
  // ---- emit: the bf16 row when this split is the whole row, else partials
  const bool emitter = key_lane == 0 && r == 0;
  // With in-kernel combining, a row with one live split needs no partials.
  const bool whole_row = direct || (p.counters != nullptr && live_splits == 1);
  if (emitter) {
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      const int qh = head * G + hg * GW + g;
      const int64_t row = (int64_t)b * kQueryHeads + qh;
      if (whole_row) {
        const float inv = l_head[g] > 0.0f ? 1.0f / l_head[g] : 0.0f;
        uint4 o;
        o.x = pack_bf16x2(acc[g][0] * inv, acc[g][1] * inv);
        o.y = pack_bf16x2(acc[g][2] * inv, acc[g][3] * inv);
        o.z = pack_bf16x2(acc[g][4] * inv, acc[g][5] * inv);
        o.w = pack_bf16x2(acc[g][6] * inv, acc[g][7] * inv);
        store128(p.out + row * D + cpack * kPackElems, o);
      } else {
        const int64_t pidx = row * p.num_splits + split;
        const float m_nat = m[g] == -INFINITY ? -INFINITY : m[g] * kLn2;
        if (p.counters != nullptr) {
          // Device-coherent (sc1) stores: the combining workgroup may run on
          // another XCD, whose L2 does not see this XCD's write-back lines.
          if (cpack == 0) {
            coherent_store(p.partial_m + pidx, m_nat);
            coherent_store(p.partial_l + pidx, l_head[g]);
          }
          coherent_store8(p.partial_acc + pidx * D, cpack * 8 * 4, acc[g]);
        } else {
          if (cpack == 0) {
            p.partial_m[pidx] = m_nat;
            p.partial_l[pidx] = l_head[g];
          }
          float4 *dst = reinterpret_cast<float4 *>(p.partial_acc + pidx * D + cpack * 8);
          dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
          dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
        }
      }
    }
  }
  append_late();
  SPLIT_MARK(6);
  if (whole_row || p.counters == nullptr) return;

  // ---- in-kernel combine: the last split workgroup of (b, head) to finish
  // reduces every live split of its GQA heads. The partials went out with
  // device-coherent stores; each thread waits for its own stores to complete
  // before the workgroup counts its arrival, so the last arriver's coherent
  // loads see every split. Whole-L2 write-back/invalidate is never needed.
  __shared__ int32_t s_last;
  wait_stores_complete();
  __syncthreads();
  if (threadIdx.x == 0) {
    int32_t *counter = p.counters + (int64_t)b * c.num_heads + head;
    const int32_t arrived =
        __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = arrived == live_splits - 1;
    if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last ? 1 : 0;
  }
  __syncthreads();
  if (s_last == 0 || key_lane != 0) return;
  combine_row_group<GW, D, LPR, RPL>(p, b, head * G + hg * GW, live_splits, r, cpack);
}

// Log-sum-exp combine of the live splits of one (batch, query head) row
// (src/gemma4_flash_attention_decode.cu:880-977), as a separate launch.
// Workgroup (row, block of combine_dims dims): 256 threads = split lanes x
// groups of 4 dims (16 x 16 for 256-dim rows, 32 x 8 for 512-dim rows).
// Each thread folds its splits (s = lane, lane + lanes, ...) into a running
// (max, sum, acc) as it streams them -- the loads do not depend on the
// arithmetic, so they are all in flight together -- and the split lanes are
// merged the same way through LDS. Empty splits (l = 0) weigh 0; a row
// without a live split is zeros.
constexpr int kCombineThreads = 256;
// Dims per workgroup: 64 for 256-dim rows (16 split lanes), 32 for 512-dim
// rows (32 split lanes: the 1 x 512 layer's ~129 splits fold in shorter
// chains; 24.0 against 24.8 us per layer, while 32 dims for 256-dim rows
// measured ~1% slower on the per-layer and batch-64 legs).
template <int kDim>
constexpr int combine_dims() { return kDim == 512 ? 32 : 64; }

template <int kDim>
__global__ __launch_bounds__(kCombineThreads) void decode_combine_kernel(
    uint16_t *__restrict__ out, const float *__restrict__ partial_m,
    const float *__restrict__ partial_l, const float *__restrict__ partial_acc,
    const int32_t *__restrict__ seq_lengths, int32_t window_size,
    int32_t split_size, int32_t num_splits, const int32_t *__restrict__ gate) {
  constexpr int kCombineDims = combine_dims<kDim>();
  constexpr int kCombineLanes = kCombineThreads / (kCombineDims / 4);  // split lanes
  __shared__ float s_m[kCombineLanes], s_l[kCombineLanes];
  __shared__ float4 s_a[kCombineLanes][kCombineDims / 4];
  const int t = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int dim0 = blockIdx.y * kCombineDims;
  if (gate != nullptr && *gate != 0) {  // a failed persistent step: zeros
    if (t < kCombineDims / 4)
      *reinterpret_cast<uint2 *>(out + row * kDim + dim0 + t * 4) = make_uint2(0, 0);
    return;
  }
  const int32_t b = (int32_t)(row / kQueryHeads);
  const int32_t seq_word = seq_lengths[b];

  const int sl = t / (kCombineDims / 4);  // split lane
  const int dg = t % (kCombineDims / 4);  // 4-dim group
  const float *pm = partial_m + row * num_splits;
  const float *pl = partial_l + row * num_splits;
  const float *pa = partial_acc + row * num_splits * kDim + dim0 + dg * 4;
  float big_m = -INFINITY, big_l = 0.0f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  // Batches of kBatch split slots per thread: a batch's loads are all issued
  // before its folds, and over every slot up to num_splits, so they do not
  // wait for the length (the empty asm keeps the live-split count, derived
  // from the length, from being computed ahead of them); slots past the
  // live splits were not written this launch and are masked like empty ones.
  constexpr int kBatch = 4;
  for (int32_t s0 = sl; s0 < num_splits; s0 += kBatch * kCombineLanes) {
    float ms_b[kBatch], ls_b[kBatch];
    float4 raw_b[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int32_t s = s0 + i * kCombineLanes;
      const int32_t slot = s < num_splits ? s : s0;
      ms_b[i] = pm[slot];
      ls_b[i] = pl[slot];
      raw_b[i] = *reinterpret_cast<const float4 *>(pa + (int64_t)slot * kDim);
    }
    int32_t seq_len = seq_word;
    asm volatile("" : "+s"(seq_len));
    int32_t first = window_size > 0 ? seq_len - window_size : 0;
    first = first < 0 ? 0 : first;
    const int32_t key_count = seq_len > first ? seq_len - first : 0;
    const int32_t splits = (key_count + split_size - 1) / split_size;
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
    const int32_t s = s0 + i * kCombineLanes;
    const float ms = ms_b[i];
    const float ls = ls_b[i];
    const float4 raw = raw_b[i];
    const bool live = s < splits && s < num_splits && ls > 0.0f;
    // An empty split's acc is never used, whatever it holds.
    const float4 a = live ? raw : make_float4(0.f, 0.f, 0.f, 0.f);
    const float m_new = live ? fmaxf(big_m, ms) : big_m;
    const float f_old = big_m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((big_m - m_new) * kLog2e);
    const float f_new = live ? __builtin_amdgcn_exp2f((ms - m_new) * kLog2e) : 0.0f;
    big_l = fmaf(live ? ls : 0.0f, f_new, big_l * f_old);
    acc.x = fmaf(a.x, f_new, acc.x * f_old);
    acc.y = fmaf(a.y, f_new, acc.y * f_old);
    acc.z = fmaf(a.z, f_new, acc.z * f_old);
    acc.w = fmaf(a.w, f_new, acc.w * f_old);
    big_m = m_new;
    }
  }
  if (dg == 0) {
    s_m[sl] = big_m;
    s_l[sl] = big_l;
  }
  s_a[sl][dg] = acc;
  __syncthreads();
  if (t < kCombineDims / 4) {
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < kCombineLanes; ++k) m = fmaxf(m, s_m[k]);
    float l = 0.0f;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < kCombineLanes; ++k) {
      const float f = s_m[k] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((s_m[k] - m) * kLog2e);
      l = fmaf(s_l[k], f, l);
      const float4 v = s_a[k][t];
      a.x = fmaf(v.x, f, a.x);
      a.y = fmaf(v.y, f, a.y);
      a.z = fmaf(v.z, f, a.z);
      a.w = fmaf(v.w, f, a.w);
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    uint2 o;
    o.x = pack_bf16x2(a.x * inv, a.y * inv);
    o.y = pack_bf16x2(a.z * inv, a.w * inv);
    *reinterpret_cast<uint2 *>(out + row * kDim + dim0 + t * 4) = o;
  }
}

// (8 kv heads x 256): 2 GQA heads per wave, 8 loads -> 16-key tiles.
using SlidingShape = DecodeShape<8, 256, 2, 8, 2>;
// (1 kv head x 512): 16 GQA heads as 4 groups of 4, 8 loads -> 8-key tiles.
using GlobalRefShape = DecodeShape<1, 512, 4, 8, 4, 8>;

bool valid_decode_config(const Gemma4KvCacheConfig &c, int32_t layer) {
  const int64_t capacity = (int64_t)c.max_pages_per_seq * c.page_size;
  const int64_t rows = (int64_t)c.num_layers * c.num_pages * c.page_size;
  return layer >= 0 && layer < c.num_layers && c.num_pages > 0 && c.page_size > 0 &&
         c.max_pages_per_seq > 0 && c.batch_size > 0 && c.window_size >= 0 &&
         (c.window_size == 0 || capacity >= c.window_size) && rows < (1ll << 31);
}

}  // namespace

bool decode_geometry_ok(const Gemma4KvCacheConfig &c, int32_t layer, int32_t batch_count,
                        int32_t split_size, int32_t num_splits) {
  return batch_count > 0 && batch_count <= c.batch_size && batch_count <= 65535 &&
         num_splits > 0 && num_splits <= 65535 && split_size > 0 &&
         valid_decode_config(c, layer) &&
         ((c.num_heads == 8 && c.head_dim == 256) || (c.num_heads == 1 && c.head_dim == 512));
}

namespace {

template <class Sh>
int waves_for(int32_t split_size) {
  const int chunks = (split_size + Sh::CT * Sh::KT - 1) / (Sh::CT * Sh::KT);
  int key_lanes = 1;
  if constexpr (Sh::kStaged) return Sh::kMaxW;  // two key lanes per head group, always
  // One key lane per started chunk: a split of one chunk stays on one wave
  // (two waves on a 32-key split measured 7.4 against 6.9 us; the merge
  // costs more than the halved tile chain saves).
  while (key_lanes * 2 * Sh::HG <= Sh::kMaxW && key_lanes < chunks) key_lanes *= 2;
  return key_lanes * Sh::HG;
}

template <class Sh>
hipError_t launch_decode(const DecodeParams &p, int32_t batch_count, bool combine,
                         hipStream_t stream) {
  constexpr int D = Sh::LPR * kPackElems;
  const int waves = waves_for<Sh>(p.split_size);
  hipLaunchKernelGGL(decode_split_kernel<Sh>,
                     dim3(p.c.num_heads, p.num_splits, batch_count),
                     dim3(waves * kWave), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !combine || p.num_splits == 1 || p.counters != nullptr) return e;
  hipLaunchKernelGGL(decode_combine_kernel<D>,
                     dim3(batch_count * kQueryHeads, D / combine_dims<D>()),
                     dim3(kCombineThreads), 0, stream, p.out, p.partial_m, p.partial_l,
                     p.partial_acc, p.seq_lengths, p.c.window_size, p.split_size,
                     p.num_splits, p.gate);
  return hipGetLastError();
}

hipError_t decode_entry(uint16_t *out, float *pm, float *pl, float *pacc,
                        const uint16_t *q, uint16_t *cache_k, uint16_t *cache_v,
                        const int32_t *page_table, const int32_t *seq_lengths,
                        const int32_t *token_position, const uint16_t *new_k,
                        const uint16_t *new_v, int32_t *counters,
                        const Gemma4KvCacheConfig &c,
                        int32_t layer, float softmax_scale, int32_t split_size,
                        int32_t num_splits, int32_t batch_count, bool combine,
                        hipStream_t stream, const uint16_t *q_norm_weight = nullptr,
                        const uint16_t *k_norm_weight = nullptr, const float *cos = nullptr,
                        const float *sin = nullptr, const int32_t *gate = nullptr) {
  if (batch_count == 0) return hipSuccess;
  if (!decode_geometry_ok(c, layer, batch_count, split_size, num_splits) ||
      !(softmax_scale > 0.0f) || out == nullptr || q == nullptr ||
      cache_k == nullptr || cache_v == nullptr || page_table == nullptr ||
      seq_lengths == nullptr) {
    return hipErrorInvalidValue;
  }
  if (num_splits > 1 && (pm == nullptr || pl == nullptr || pacc == nullptr)) {
    return hipErrorInvalidValue;
  }
  DecodeParams p;
  p.out = out;
  p.partial_m = pm;
  p.partial_l = pl;
  p.partial_acc = pacc;
  p.q = q;
  p.cache_k = cache_k;
  p.cache_v = cache_v;
  p.page_table = page_table;
  p.seq_lengths = seq_lengths;
  p.token_position = token_position;
  p.counters = num_splits > 1 ? counters : nullptr;
  p.new_k = new_k;
  p.new_v = new_v;
  p.q_norm_weight = q_norm_weight;
  p.k_norm_weight = k_norm_weight;
  p.cos = cos;
  p.sin = sin;
  p.c = c;
  p.layer = layer;
  p.q_scale = softmax_scale * kLog2e;
  p.split_size = split_size;
  p.num_splits = num_splits;
  p.gate = gate;
  // Only the combined row leaves a launch that also combines: its splits may
  // be numbered by ring slot. A split-only launch hands its partials to the
  // caller in the position-numbered layout.
  p.slot_splits = combine || p.counters != nullptr ? 1 : 0;
  if (c.num_heads == 8 && c.head_dim == 256) {
    return launch_decode<SlidingShape>(p, batch_count, combine, stream);
  }
  if (c.num_heads == 1 && c.head_dim == 512) {
    return launch_decode<GlobalRefShape>(p, batch_count, combine, stream);
  }
  return hipErrorInvalidValue;
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch[kMaxDevices];  // per device: device address of `scratch`

// Device address of the current device's `scratch`, looked up once per
// device with that device current.
hipError_t noalloc_scratch(float **out) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return e;
  if (device < 0 || device >= kMaxDevices) return hipErrorNotSupported;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[device] == nullptr) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (ptr == nullptr) return hipErrorInvalidSymbol;
    g_scratch[device] = static_cast<float *>(ptr);
  }
  *out = g_scratch[device];
  return hipSuccess;
}

}  // namespace

hipError_t decode_append_gated(uint16_t *out, float *pm, float *pl, float *pacc,
                               const uint16_t *q, uint16_t *cache_k, uint16_t *cache_v,
                               const int32_t *page_table, const int32_t *seq_lengths,
                               const int32_t *token_position, const uint16_t *new_k,
                               const uint16_t *new_v, const Gemma4KvCacheConfig &c,
                               int32_t layer, float softmax_scale, int32_t split_size,
                               int32_t num_splits, int32_t batch_count, const int32_t *gate,
                               hipStream_t stream, const uint16_t *q_norm_weight,
                               const uint16_t *k_norm_weight, const float *cos,
                               const float *sin) {
  if (token_position == nullptr || new_k == nullptr || gate == nullptr) return hipErrorInvalidValue;
  return decode_entry(out, pm, pl, pacc, q, cache_k, cache_v, page_table, seq_lengths,
                      token_position, new_k, new_v, nullptr, c, layer, softmax_scale, split_size,
                      num_splits, batch_count, /*combine=*/true, stream, q_norm_weight,
                      k_norm_weight, cos, sin, gate);
}

}  // namespace gemma4

using namespace gemma4;

extern "C" {

hipError_t gemma4_flash_attention_decode_paged_bf16(
    gemma4_bf16 *d_out, float *d_partial_m, float *d_partial_l,
    float *d_partial_acc, const gemma4_bf16 *d_q, const gemma4_bf16 *d_cache_k,
    const gemma4_bf16 *d_cache_v, const int32_t *d_page_table,
    const int32_t *d_seq_lengths, Gemma4KvCacheConfig config, int32_t layer,
    float softmax_scale, int32_t split_size, int32_t num_splits,
    int32_t batch_count, hipStream_t stream) {
  return decode_entry(
      reinterpret_cast<uint16_t *>(d_out), d_partial_m, d_partial_l, d_partial_acc,
      reinterpret_cast<const uint16_t *>(d_q),
      const_cast<uint16_t *>(reinterpret_cast<const uint16_t *>(d_cache_k)),
      const_cast<uint16_t *>(reinterpret_cast<const uint16_t *>(d_cache_v)),
      d_page_table, d_seq_lengths, nullptr, nullptr, nullptr, nullptr, config, layer,
      softmax_scale, split_size, num_splits, batch_count, /*combine=*/true, stream);
}

hipError_t gemma4_flash_attention_append_decode_paged_bf16(
    gemma4_bf16 *d_out, float *d_partial_m, float *d_partial_l,
    float *d_partial_acc, const gemma4_bf16 *d_q, gemma4_bf16 *d_cache_k,
    gemma4_bf16 *d_cache_v, const int32_t *d_page_table,
    const int32_t *d_seq_lengths, const int32_t *d_token_position,
    const gemma4_bf16 *d_k, const gemma4_bf16 *d_v, int32_t *d_split_counters,
    Gemma4KvCacheConfig config, int32_t layer, float softmax_scale,
    int32_t split_size, int32_t num_splits, int32_t batch_count,
    hipStream_t stream) {
  if (d_token_position == nullptr || d_k == nullptr || d_v == nullptr) {
    return hipErrorInvalidValue;
  }
  return decode_entry(
      reinterpret_cast<uint16_t *>(d_out), d_partial_m, d_partial_l, d_partial_acc,
      reinterpret_cast<const uint16_t *>(d_q), reinterpret_cast<uint16_t *>(d_cache_k),
      reinterpret_cast<uint16_t *>(d_cache_v), d_page_table, d_seq_lengths,
      d_token_position, reinterpret_cast<const uint16_t *>(d_k),
      reinterpret_cast<const uint16_t *>(d_v), d_split_counters, config, layer,
      softmax_scale,
      split_size, num_splits, batch_count, /*combine=*/true, stream);
}

hipError_t gemma4_flash_attention_append_decode_paged_bf16_noalloc(
    gemma4_bf16 *d_out, const gemma4_bf16 *d_q, gemma4_bf16 *d_cache_k,
    gemma4_bf16 *d_cache_v, const int32_t *d_page_table, const int32_t *d_seq_lengths,
    const int32_t *d_token_position, const gemma4_bf16 *d_k, const gemma4_bf16 *d_v,
    Gemma4KvCacheConfig config, int32_t layer, float softmax_scale, int32_t split_size,
    int32_t num_splits, int32_t batch_count, hipStream_t stream) {
  if (batch_count == 0) return hipSuccess;
  // Range checks come before the scratch-size product so it cannot overflow.
  if (d_token_position == nullptr || d_k == nullptr || d_v == nullptr || batch_count < 0 ||
      batch_count > 65535 || num_splits <= 0 || num_splits > 65535 ||
      (config.head_dim != 256 && config.head_dim != 512)) {
    return hipErrorInvalidValue;
  }
  // Partials of this call: m and l [rows * splits], acc [rows * splits * D].
  const int64_t slots = (int64_t)batch_count * kQueryHeads * num_splits;
  const int64_t floats = slots * (2 + (int64_t)config.head_dim);
  if (floats * (int64_t)sizeof(float) > (int64_t)kNoAllocScratchBytes) {
    return hipErrorOutOfMemory;  // beyond the fixed scratch: use the workspace form
  }
  float *s = nullptr;
  const hipError_t e = noalloc_scratch(&s);
  if (e != hipSuccess) return e;
  // The separate combine kernel reads only the live splits this call writes,
  // so the scratch needs no clearing between calls.
  return decode_entry(
      reinterpret_cast<uint16_t *>(d_out), s, s + slots, s + 2 * slots,
      reinterpret_cast<const uint16_t *>(d_q), reinterpret_cast<uint16_t *>(d_cache_k),
      reinterpret_cast<uint16_t *>(d_cache_v), d_page_table, d_seq_lengths,
      d_token_position, reinterpret_cast<const uint16_t *>(d_k),
      reinterpret_cast<const uint16_t *>(d_v), nullptr, config, layer, softmax_scale,
      split_size, num_splits, batch_count, /*combine=*/true, stream);
}

hipError_t gemma4_flash_attention_prep_append_decode_paged_bf16(
    gemma4_bf16 *d_out, float *d_partial_m, float *d_partial_l,
    float *d_partial_acc, const gemma4_bf16 *d_q, gemma4_bf16 *d_cache_k,
    gemma4_bf16 *d_cache_v, const int32_t *d_page_table,
    const int32_t *d_seq_lengths, const int32_t *d_token_position,
    const gemma4_bf16 *d_k, const gemma4_bf16 *d_v, const gemma4_bf16 *d_q_norm_weight,
    const gemma4_bf16 *d_k_norm_weight, const float *d_cos, const float *d_sin,
    int32_t *d_split_counters, Gemma4KvCacheConfig config, int32_t layer,
    float softmax_scale, int32_t split_size, int32_t num_splits, int32_t batch_count,
    hipStream_t stream) {
  const bool global = config.num_heads == 1;
  if (d_token_position == nullptr || d_k == nullptr || (d_v == nullptr && !global) ||
      d_q_norm_weight == nullptr || d_k_norm_weight == nullptr || d_cos == nullptr ||
      d_sin == nullptr) {
    return hipErrorInvalidValue;
  }
  return decode_entry(
      reinterpret_cast<uint16_t *>(d_out), d_partial_m, d_partial_l, d_partial_acc,
      reinterpret_cast<const uint16_t *>(d_q), reinterpret_cast<uint16_t *>(d_cache_k),
      reinterpret_cast<uint16_t *>(d_cache_v), d_page_table, d_seq_lengths,
      d_token_position, reinterpret_cast<const uint16_t *>(d_k),
      global ? nullptr : reinterpret_cast<const uint16_t *>(d_v), d_split_counters, config,
      layer, softmax_scale, split_size, num_splits, batch_count, /*combine=*/true, stream,
      reinterpret_cast<const uint16_t *>(d_q_norm_weight),
      reinterpret_cast<const uint16_t *>(d_k_norm_weight), d_cos, d_sin);
}

hipError_t gemma4_flash_attention_decode_split_paged_bf16(
    gemma4_bf16 *d_out, float *d_partial_m, float *d_partial_l,
    float *d_partial_acc, const gemma4_bf16 *d_q, gemma4_bf16 *d_cache_k,
    gemma4_bf16 *d_cache_v, const int32_t *d_page_table,
    const int32_t *d_seq_lengths, const int32_t *d_token_position,
    const gemma4_bf16 *d_k, const gemma4_bf16 *d_v, Gemma4KvCacheConfig config,
    int32_t layer, float softmax_scale, int32_t split_size, int32_t num_splits,
    int32_t batch_count, hipStream_t stream) {
  if (d_token_position != nullptr && (d_k == nullptr || d_v == nullptr)) {
    return hipErrorInvalidValue;
  }
  return decode_entry(
      reinterpret_cast<uint16_t *>(d_out), d_partial_m, d_partial_l, d_partial_acc,
      reinterpret_cast<const uint16_t *>(d_q), reinterpret_cast<uint16_t *>(d_cache_k),
      reinterpret_cast<uint16_t *>(d_cache_v), d_page_table, d_seq_lengths,
      d_token_position, reinterpret_cast<const uint16_t *>(d_k),
      reinterpret_cast<const uint16_t *>(d_v), nullptr, config, layer, softmax_scale,
      split_size, num_splits, batch_count, /*combine=*/false, stream);
}

hipError_t gemma4_flash_attention_decode_combine_bf16(
    gemma4_bf16 *d_out, const float *d_partial_m, const float *d_partial_l,
    const float *d_partial_acc, const int32_t *d_seq_lengths,
    Gemma4KvCacheConfig config, int32_t split_size, int32_t num_splits,
    int32_t batch_count, hipStream_t stream) {
  if (batch_count == 0) return hipSuccess;
  if (batch_count < 0 || batch_count > 65535 || split_size <= 0 || num_splits <= 0 ||
      config.window_size < 0 || d_out == nullptr || d_partial_m == nullptr ||
      d_partial_l == nullptr || d_partial_acc == nullptr || d_seq_lengths == nullptr) {
    return hipErrorInvalidValue;
  }
  uint16_t *out = reinterpret_cast<uint16_t *>(d_out);
  const dim3 block(kCombineThreads);
  if (config.head_dim == 256) {
    hipLaunchKernelGGL(decode_combine_kernel<256>, dim3(batch_count * kQueryHeads, 256 / combine_dims<256>()),
                       block, 0, stream, out, d_partial_m, d_partial_l, d_partial_acc,
                       d_seq_lengths, config.window_size, split_size, num_splits,
                       static_cast<const int32_t *>(nullptr));
  } else if (config.head_dim == 512) {
    hipLaunchKernelGGL(decode_combine_kernel<512>, dim3(batch_count * kQueryHeads, 512 / combine_dims<512>()),
                       block, 0, stream, out, d_partial_m, d_partial_l, d_partial_acc,
                       d_seq_lengths, config.window_size, split_size, num_splits,
                       static_cast<const int32_t *>(nullptr));
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t gemma4_decode_split_plan(Gemma4KvCacheConfig config,
                                    int32_t batch_count, int32_t max_live_keys,
                                    int32_t target_workgroups,
                                    int32_t *split_size, int32_t *num_splits) {
  if (split_size == nullptr || num_splits == nullptr || batch_count <= 0 ||
      max_live_keys < 0 || config.num_heads <= 0) {
    return hipErrorInvalidValue;
  }
  int32_t tile, key_tile;
  if (config.num_heads == 8 && config.head_dim == 256) {
    tile = SlidingShape::KT * SlidingShape::CT;  // one wave's page-lookup chunk
    key_tile = SlidingShape::KT;
  } else if (config.num_heads == 1 && config.head_dim == 512) {
    // The staged kernel's granule is one LDS step (a tile per key lane):
    // 8193 keys as 171 splits of 48 run split + combine in 20.5 against
    // 21.8 us as 129 splits of 64 (32 / 80 / 96 keys: 23.7 / 23.2 / 25.2).
    tile = (GlobalRefShape::kMaxW / GlobalRefShape::HG) * GlobalRefShape::KT;
    key_tile = GlobalRefShape::KT;
  } else {
    return hipErrorInvalidValue;
  }
  // Default: one split workgroup per CU for one sequence (measured on 8193,
  // 16384 and 131072 keys: fewer, longer splits stream as fast and make the
  // combine cheaper; counts that are not a multiple of the CU count leave a
  // tail). A batch is sized by its longest sequence, so shorter ones leave
  // workgroups idle: 32 per CU then (measured best on 64 sequences of 512 to
  // 32768 keys).
  const bool planned = target_workgroups <= 0;
  if (planned) target_workgroups = batch_count > 1 ? 8192 : 256;
  const int64_t keys = (int64_t)std::max(max_live_keys, 1);
  const int64_t heads = (int64_t)batch_count * config.num_heads;
  int64_t splits_per_seq = (target_workgroups + heads - 1) / heads;
  if (splits_per_seq < 1) splits_per_seq = 1;
  int64_t size = (keys + splits_per_seq - 1) / splits_per_seq;
  size = ((size + tile - 1) / tile) * tile;
  if (size < tile) size = tile;
  // One sequence whose splits come out at two tiles or fewer (a sliding
  // layer's 1024-key window): the split is a dependent chain of tile
  // latencies, so one tile per workgroup, as long as that stays within two
  // workgroups per CU (1024 keys: 8.5 against 9.4 us per layer with the
  // combine, 512 against 256 workgroups).
  if (planned && batch_count == 1 && size <= 2 * key_tile &&
      heads * ((keys + key_tile - 1) / key_tile) <= 2 * target_workgroups) {
    size = key_tile;
  }
  *split_size = (int32_t)size;
  *num_splits = (int32_t)((keys + size - 1) / size);
  return hipSuccess;
}

}  // extern "C"
