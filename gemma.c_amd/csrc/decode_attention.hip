// Paged split-K decode attention for gfx950 (flash decoding), with an
// optional fused K/V append. Replaces the decode-attention phases of
// src/gemma4_flash_attention_decode.cu (phase_decode_paged_grouped_split,
// phase_decode_paged_reduce, phase_decode_q_paged_kv_norm_rope's cache write).
//
// Work decomposition
//   workgroup (split, kv_head, batch)   grid = (num_splits, num_heads, batch)
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

#include "gemma4_flash_attention.h"

#include <algorithm>
#include <math.h>

namespace gemma4 {
namespace {

constexpr int kMaxWaves = 4;
constexpr int kRowInvalid = -1;   // key outside the split or unmapped page
constexpr int kRowNewToken = -2;  // key being appended in this launch

struct DecodeParams {
  uint16_t *out;
  float *partial_m;
  float *partial_l;
  float *partial_acc;
  const uint16_t *q;
  uint16_t *cache_k;  // written only by the fused append
  uint16_t *cache_v;
  const int32_t *page_table;
  const int32_t *seq_lengths;
  const int32_t *token_position;  // null: no append
  const uint16_t *new_k;
  const uint16_t *new_v;
  Gemma4KvCacheConfig c;
  int32_t layer;
  float q_scale;  // softmax_scale * log2(e)
  int32_t split_size;
  int32_t num_splits;
};

template <int kHeads, int kDim, int kHeadsPerWave, int kLoads>
struct DecodeShape {
  static constexpr int G = kQueryHeads / kHeads;          // GQA group
  static constexpr int GW = kHeadsPerWave;                // heads per wave
  static constexpr int HG = G / GW;                       // head groups per kv head
  static constexpr int LPR = kDim / kPackElems;           // lanes per key row
  static constexpr int RPL = kWave / LPR;                 // rows per load
  static constexpr int LOADS = kLoads;                    // loads per lane per tile
  static constexpr int KT = RPL * kLoads;                 // keys per tile
  static constexpr int NP = kLoads * GW;                  // partial dots per lane
  static constexpr int S = __builtin_ctz(LPR / NP);       // duplicate-lane bits
  static constexpr int GB = __builtin_ctz(GW);            // head-select bits
  static constexpr int kRowElems = kHeads * kDim;
  static_assert(G % GW == 0, "heads per wave must divide the GQA group");
  static_assert(NP <= LPR, "one reduced score per lane at most");
  static_assert((NP & (NP - 1)) == 0 && (GW & (GW - 1)) == 0, "powers of two");
  static_assert(KT <= kWave, "one page lookup per lane per tile");
  static_assert(RPL * NP <= kWave, "probability slot holds one tile");
};

// Value-splitting butterfly: N partial values per lane are summed over the
// lanes that differ in bits [log2(O*2/N).. log2(O)] of the lane id; after the
// split steps every lane carries one value, and remaining offsets are plain
// all-reduce steps (the value then repeats across those lanes).
template <int N, int O>
__device__ __forceinline__ void split_butterfly(float *v, int lane) {
  if constexpr (N > 1) {
    const bool hi = (lane & O) != 0;
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const float send = hi ? v[i] : v[i + N / 2];
      const float keep = hi ? v[i + N / 2] : v[i];
      v[i] = keep + xor_lane(send, O);
    }
    split_butterfly<N / 2, O / 2>(v, lane);
  } else if constexpr (O >= 1) {
    v[0] += xor_lane(v[0], O);
    split_butterfly<1, O / 2>(v, lane);
  }
}

// Max / sum of one value over all lanes whose bit pattern differs only at
// offsets >= kFrom (lanes below kFrom carry duplicates or another head).
template <int kFrom>
__device__ __forceinline__ float reduce_max_from(float v) {
#pragma unroll
  for (int o = kFrom; o < kWave; o <<= 1) v = fmaxf(v, xor_lane(v, o));
  return v;
}
template <int kFrom>
__device__ __forceinline__ float reduce_sum_from(float v) {
#pragma unroll
  for (int o = kFrom; o < kWave; o <<= 1) v += xor_lane(v, o);
  return v;
}

// Collect a per-head value held by the lanes of head `my_g` into out[g] for
// every head g of the wave (lanes of head g differ in bits [S, S+GB)).
template <int GW, int S>
__device__ __forceinline__ void gather_heads(float mine, int my_g, float (&out)[GW]) {
  float other[GW];
  other[0] = mine;
#pragma unroll
  for (int d = 1; d < GW; ++d) other[d] = xor_lane(mine, d << S);
#pragma unroll
  for (int g = 0; g < GW; ++g) {
    const int d = my_g ^ g;
    float v = other[0];
#pragma unroll
    for (int dd = 1; dd < GW; ++dd) v = (d == dd) ? other[dd] : v;
    out[g] = v;
  }
}

__device__ __forceinline__ void wave_lds_sync() {
  // LDS operations of one wave complete in issue order; this only stops the
  // compiler from moving LDS accesses across the exchange point.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Cache row index of `key` for sequence `b`, or kRowInvalid for an unmapped
// page (src/gemma4_flash_attention_decode.cu:791-805).
__device__ __forceinline__ int32_t key_row(const Gemma4KvCacheConfig &c,
                                           const int32_t *__restrict__ page_table,
                                           int32_t layer, int32_t b, int32_t key) {
  const int32_t logical_page = key / c.page_size;
  const int32_t slot = logical_page % c.max_pages_per_seq;
  const int32_t physical = page_table[b * c.max_pages_per_seq + slot];
  if (physical < 0 || physical >= c.num_pages) return kRowInvalid;
  const int32_t page_offset = key - logical_page * c.page_size;
  return ((int32_t)layer * c.num_pages + physical) * c.page_size + page_offset;
}

// Cache row the fused append writes for (b, position), or -1 when the
// reference skip rules drop it (src/gemma4_kv_cache.cu:25-34).
__device__ __forceinline__ int32_t append_row(const Gemma4KvCacheConfig &c,
                                              const int32_t *__restrict__ page_table,
                                              int32_t layer, int32_t b, int32_t position) {
  if (position < 0 || b >= c.batch_size) return -1;
  const int32_t logical_page = position / c.page_size;
  if (c.window_size == 0 && logical_page >= c.max_pages_per_seq) return -1;
  return key_row(c, page_table, layer, b, position);
}

template <class Sh>
__global__ __launch_bounds__(kMaxWaves * kWave) void decode_split_kernel(DecodeParams p) {
  constexpr int G = Sh::G, GW = Sh::GW, HG = Sh::HG, LPR = Sh::LPR, RPL = Sh::RPL;
  constexpr int LOADS = Sh::LOADS, KT = Sh::KT, NP = Sh::NP, S = Sh::S;
  constexpr int D = LPR * kPackElems;

  __shared__ int32_t s_rows[kMaxWaves][kWave];
  __shared__ float s_prob[kMaxWaves][kWave];
  __shared__ float s_ml[kMaxWaves][2][GW];
  __shared__ float s_acc[kMaxWaves][GW][D];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  const int hg = wave % HG;                 // head group of this wave
  const int key_lane = wave / HG;           // key-tile slot among same-group waves
  const int key_lanes = waves / HG;
  const int r = lane / LPR;                 // key row within a load
  const int cpack = lane % LPR;             // 16-byte pack within the row

  const int32_t split = blockIdx.x;
  const int32_t head = blockIdx.y;
  const int32_t b = blockIdx.z;
  const Gemma4KvCacheConfig &c = p.c;

  const int32_t seq_len = wave_uniform(p.seq_lengths[b]);
  int32_t first = c.window_size > 0 ? seq_len - c.window_size : 0;
  first = first < 0 ? 0 : first;
  const int32_t key_count = seq_len > first ? seq_len - first : 0;
  const int32_t live_splits = (key_count + p.split_size - 1) / p.split_size;
  const bool direct = p.num_splits == 1;

  // ---- fused append of the current token (one split per (b, head) owns it)
  int32_t new_pos = -1, new_row = -1;
  if (p.token_position != nullptr) {
    new_pos = wave_uniform(p.token_position[b]);
    new_row = wave_uniform(append_row(c, p.page_table, p.layer, b, new_pos));
    const bool in_live = new_pos >= first && new_pos < seq_len;
    const int32_t owner = in_live ? (new_pos - first) / p.split_size : 0;
    if (split == owner && new_row >= 0 && threadIdx.x < LPR) {
      const int64_t src = ((int64_t)b * c.num_heads + head) * D + threadIdx.x * kPackElems;
      const int64_t dst = (int64_t)new_row * Sh::kRowElems + (int64_t)head * D +
                          threadIdx.x * kPackElems;
      store128(p.cache_k + dst, load128(p.new_k + src));
      store128(p.cache_v + dst, load128(p.new_v + src));
    }
    if (!in_live || new_row < 0) new_pos = -1;  // attention reads it from the cache path only if live
  }

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
    return;
  }
  if (split >= live_splits) return;

  const int32_t begin = first + split * p.split_size;
  const int32_t end = min(seq_len, begin + p.split_size);

  // ---- Q for the GW heads of this wave, 8 dims per lane, pre-scaled
  float qf[GW][8];
#pragma unroll
  for (int g = 0; g < GW; ++g) {
    const int qh = head * G + hg * GW + g;
    const uint4 qp = load128(p.q + ((int64_t)b * kQueryHeads + qh) * D + cpack * kPackElems);
    unpack8(qp, qf[g]);
#pragma unroll
    for (int j = 0; j < 8; ++j) qf[g][j] *= p.q_scale;
  }

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

  const int32_t n_tiles = (end - begin + KT - 1) / KT;
  auto lookup = [&](int32_t tile) -> int32_t {
    const int32_t key = begin + tile * KT + lane;
    if (lane >= KT || tile >= n_tiles || key >= end) return kRowInvalid;
    if (key == new_pos) return kRowNewToken;
    return key_row(c, p.page_table, p.layer, b, key);
  };

  int32_t next_row = lookup(key_lane);
  for (int32_t tile = key_lane; tile < n_tiles; tile += key_lanes) {
    // Publish this tile's rows (lane l holds key l) in load order.
    {
      const int l = lane;
      if (l < KT) s_rows[wave][(l % RPL) * LOADS + l / RPL] = next_row;
    }
    wave_lds_sync();
    int32_t rows[LOADS];
#pragma unroll
    for (int kl = 0; kl < LOADS; ++kl) rows[kl] = s_rows[wave][r * LOADS + kl];
    next_row = lookup(tile + key_lanes);  // overlaps with this tile's loads

    uint4 kraw[LOADS], vraw[LOADS];
    uint32_t valid_mask = 0;
#pragma unroll
    for (int kl = 0; kl < LOADS; ++kl) {
      kraw[kl] = make_uint4(0, 0, 0, 0);
      vraw[kl] = make_uint4(0, 0, 0, 0);
      const int32_t row = rows[kl];
      if (row != kRowInvalid) {
        valid_mask |= 1u << kl;
        const uint16_t *kp = row == kRowNewToken ? p.new_k + new_off
                                                 : kbase + (int64_t)row * Sh::kRowElems;
        const uint16_t *vp = row == kRowNewToken ? p.new_v + new_off
                                                 : vbase + (int64_t)row * Sh::kRowElems;
        kraw[kl] = load128(kp);
        vraw[kl] = load128(vp);
      }
    }

    // Partial Q·K over this lane's 8 dims: part[kl * GW + g].
    float part[NP];
#pragma unroll
    for (int kl = 0; kl < LOADS; ++kl) {
      float kf[8];
      unpack8(kraw[kl], kf);
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) s = fmaf(qf[g][j], kf[j], s);
        part[kl * GW + g] = s;
      }
    }
    split_butterfly<NP, LPR / 2>(part, lane);
    const bool valid = (valid_mask >> my_kl) & 1u;
    const float score = valid ? part[0] : -INFINITY;

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
      const float4 t = *reinterpret_cast<const float4 *>(&s_prob[wave][r * NP + i]);
      pv[i] = t.x; pv[i + 1] = t.y; pv[i + 2] = t.z; pv[i + 3] = t.w;
    }

#pragma unroll
    for (int g = 0; g < GW; ++g) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] *= alpha[g];
    }
#pragma unroll
    for (int kl = 0; kl < LOADS; ++kl) {
      float vf[8];
      unpack8(vraw[kl], vf);
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        const float w = pv[kl * GW + g];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[g][j] = fmaf(w, vf[j], acc[g][j]);
      }
    }
  }

  // ---- wave totals: l per head, acc summed over the RPL key rows
  float l_head[GW];
  gather_heads<GW, S>(reduce_sum_from<(1 << S) * GW>(l_lane), my_g, l_head);
#pragma unroll
  for (int o = LPR; o < kWave; o <<= 1) {
#pragma unroll
    for (int g = 0; g < GW; ++g) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] += xor_lane(acc[g][j], o);
    }
  }

  // ---- combine the waves that share a head group (LDS), then emit
  if (key_lanes > 1) {
    if (lane == 0) {
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        s_ml[wave][0][g] = m[g];
        s_ml[wave][1][g] = l_head[g];
      }
    }
    if (r == 0) {
#pragma unroll
      for (int g = 0; g < GW; ++g) {
#pragma unroll
        for (int j = 0; j < 8; ++j) s_acc[wave][g][cpack * 8 + j] = acc[g][j];
      }
    }
    __syncthreads();
    if (key_lane != 0) return;
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
#pragma unroll
        for (int j = 0; j < 8; ++j) sum[j] = fmaf(s_acc[w][g][cpack * 8 + j], f, sum[j]);
      }
      m[g] = big_m;
      l_head[g] = big_l;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] = sum[j];
    }
  }

  if (r != 0) return;
#pragma unroll
  for (int g = 0; g < GW; ++g) {
    const int qh = head * G + hg * GW + g;
    const int64_t row = (int64_t)b * kQueryHeads + qh;
    if (direct) {
      const float inv = l_head[g] > 0.0f ? 1.0f / l_head[g] : 0.0f;
      uint4 o;
      o.x = pack_bf16x2(acc[g][0] * inv, acc[g][1] * inv);
      o.y = pack_bf16x2(acc[g][2] * inv, acc[g][3] * inv);
      o.z = pack_bf16x2(acc[g][4] * inv, acc[g][5] * inv);
      o.w = pack_bf16x2(acc[g][6] * inv, acc[g][7] * inv);
      store128(p.out + row * D + cpack * kPackElems, o);
    } else {
      const int64_t pidx = row * p.num_splits + split;
      if (cpack == 0) {
        p.partial_m[pidx] = m[g] == -INFINITY ? -INFINITY : m[g] * kLn2;
        p.partial_l[pidx] = l_head[g];
      }
      float4 *dst = reinterpret_cast<float4 *>(p.partial_acc + pidx * D + cpack * 8);
      dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
      dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
    }
  }
}

// Log-sum-exp combine of the live splits of one (batch, query head) row
// (src/gemma4_flash_attention_decode.cu:880-977). One wave per row; each lane
// owns D/64 consecutive dims.
template <int kDim>
__global__ __launch_bounds__(kWave) void decode_combine_kernel(
    uint16_t *__restrict__ out, const float *__restrict__ partial_m,
    const float *__restrict__ partial_l, const float *__restrict__ partial_acc,
    const int32_t *__restrict__ seq_lengths, int32_t window_size,
    int32_t split_size, int32_t num_splits) {
  constexpr int kDimsPerLane = kDim / kWave;  // 4 or 8
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int32_t b = (int32_t)(row / kQueryHeads);
  const int32_t seq_len = wave_uniform(seq_lengths[b]);
  int32_t first = window_size > 0 ? seq_len - window_size : 0;
  first = first < 0 ? 0 : first;
  const int32_t key_count = seq_len > first ? seq_len - first : 0;
  int32_t splits = (key_count + split_size - 1) / split_size;
  splits = splits < num_splits ? splits : num_splits;

  const float *pm = partial_m + row * num_splits;
  const float *pl = partial_l + row * num_splits;
  float big_m = -INFINITY;
  for (int32_t s = lane; s < splits; s += kWave) big_m = fmaxf(big_m, pm[s]);
  big_m = reduce_max_from<1>(big_m);
  float big_l = 0.0f;
  for (int32_t s = lane; s < splits; s += kWave) {
    const float ls = pl[s];
    if (ls > 0.0f) big_l = fmaf(ls, __builtin_amdgcn_exp2f((pm[s] - big_m) * kLog2e), big_l);
  }
  big_l = reduce_sum_from<1>(big_l);

  float acc[kDimsPerLane];
#pragma unroll
  for (int j = 0; j < kDimsPerLane; ++j) acc[j] = 0.0f;
  const float *pa = partial_acc + row * num_splits * kDim + lane * kDimsPerLane;
#pragma unroll 4
  for (int32_t s = 0; s < splits; ++s) {
    const float ls = pl[s];
    const float w = ls > 0.0f ? __builtin_amdgcn_exp2f((pm[s] - big_m) * kLog2e) : 0.0f;
#pragma unroll
    for (int j = 0; j < kDimsPerLane; j += 4) {
      const float4 a = *reinterpret_cast<const float4 *>(pa + (int64_t)s * kDim + j);
      acc[j] = fmaf(a.x, w, acc[j]);
      acc[j + 1] = fmaf(a.y, w, acc[j + 1]);
      acc[j + 2] = fmaf(a.z, w, acc[j + 2]);
      acc[j + 3] = fmaf(a.w, w, acc[j + 3]);
    }
  }
  const float inv = (splits > 0 && big_l > 0.0f) ? 1.0f / big_l : 0.0f;
  uint16_t *o = out + row * kDim + lane * kDimsPerLane;
#pragma unroll
  for (int j = 0; j < kDimsPerLane; j += 4) {
    uint2 w;
    w.x = pack_bf16x2(acc[j] * inv, acc[j + 1] * inv);
    w.y = pack_bf16x2(acc[j + 2] * inv, acc[j + 3] * inv);
    *reinterpret_cast<uint2 *>(o + j) = w;
  }
}

// (8 kv heads x 256): 2 GQA heads per wave, 16 loads -> 32-key tiles.
using SlidingShape = DecodeShape<8, 256, 2, 16>;
// (1 kv head x 512): 16 GQA heads as 4 groups of 4, 8 loads -> 8-key tiles.
using GlobalRefShape = DecodeShape<1, 512, 4, 8>;

bool valid_decode_config(const Gemma4KvCacheConfig &c, int32_t layer) {
  const int64_t capacity = (int64_t)c.max_pages_per_seq * c.page_size;
  const int64_t rows = (int64_t)c.num_layers * c.num_pages * c.page_size;
  return layer >= 0 && layer < c.num_layers && c.num_pages > 0 && c.page_size > 0 &&
         c.max_pages_per_seq > 0 && c.batch_size > 0 && c.window_size >= 0 &&
         (c.window_size == 0 || capacity >= c.window_size) && rows < (1ll << 31);
}

template <class Sh>
int waves_for(int32_t split_size) {
  const int tiles = (split_size + Sh::KT - 1) / Sh::KT;
  int key_lanes = 1;
  while (key_lanes * 2 * Sh::HG <= kMaxWaves && key_lanes < tiles) key_lanes *= 2;
  return key_lanes * Sh::HG;
}

template <class Sh>
hipError_t launch_decode(const DecodeParams &p, int32_t batch_count,
                         hipStream_t stream) {
  constexpr int D = Sh::LPR * kPackElems;
  const int waves = waves_for<Sh>(p.split_size);
  hipLaunchKernelGGL(decode_split_kernel<Sh>,
                     dim3(p.num_splits, p.c.num_heads, batch_count),
                     dim3(waves * kWave), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.num_splits == 1) return e;
  hipLaunchKernelGGL(decode_combine_kernel<D>, dim3(batch_count * kQueryHeads),
                     dim3(kWave), 0, stream, p.out, p.partial_m, p.partial_l,
                     p.partial_acc, p.seq_lengths, p.c.window_size, p.split_size,
                     p.num_splits);
  return hipGetLastError();
}

hipError_t decode_entry(uint16_t *out, float *pm, float *pl, float *pacc,
                        const uint16_t *q, uint16_t *cache_k, uint16_t *cache_v,
                        const int32_t *page_table, const int32_t *seq_lengths,
                        const int32_t *token_position, const uint16_t *new_k,
                        const uint16_t *new_v, const Gemma4KvCacheConfig &c,
                        int32_t layer, float softmax_scale, int32_t split_size,
                        int32_t num_splits, int32_t batch_count,
                        hipStream_t stream) {
  if (batch_count == 0) return hipSuccess;
  if (batch_count < 0 || batch_count > c.batch_size || batch_count > 65535 ||
      !valid_decode_config(c, layer) || !(softmax_scale > 0.0f) ||
      split_size <= 0 || num_splits <= 0 || out == nullptr || q == nullptr ||
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
  p.new_k = new_k;
  p.new_v = new_v;
  p.c = c;
  p.layer = layer;
  p.q_scale = softmax_scale * kLog2e;
  p.split_size = split_size;
  p.num_splits = num_splits;
  if (c.num_heads == 8 && c.head_dim == 256) {
    return launch_decode<SlidingShape>(p, batch_count, stream);
  }
  if (c.num_heads == 1 && c.head_dim == 512) {
    return launch_decode<GlobalRefShape>(p, batch_count, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace
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
      d_page_table, d_seq_lengths, nullptr, nullptr, nullptr, config, layer,
      softmax_scale, split_size, num_splits, batch_count, stream);
}

hipError_t gemma4_flash_attention_append_decode_paged_bf16(
    gemma4_bf16 *d_out, float *d_partial_m, float *d_partial_l,
    float *d_partial_acc, const gemma4_bf16 *d_q, gemma4_bf16 *d_cache_k,
    gemma4_bf16 *d_cache_v, const int32_t *d_page_table,
    const int32_t *d_seq_lengths, const int32_t *d_token_position,
    const gemma4_bf16 *d_k, const gemma4_bf16 *d_v, Gemma4KvCacheConfig config,
    int32_t layer, float softmax_scale, int32_t split_size, int32_t num_splits,
    int32_t batch_count, hipStream_t stream) {
  if (d_token_position == nullptr || d_k == nullptr || d_v == nullptr) {
    return hipErrorInvalidValue;
  }
  return decode_entry(
      reinterpret_cast<uint16_t *>(d_out), d_partial_m, d_partial_l, d_partial_acc,
      reinterpret_cast<const uint16_t *>(d_q), reinterpret_cast<uint16_t *>(d_cache_k),
      reinterpret_cast<uint16_t *>(d_cache_v), d_page_table, d_seq_lengths,
      d_token_position, reinterpret_cast<const uint16_t *>(d_k),
      reinterpret_cast<const uint16_t *>(d_v), config, layer, softmax_scale,
      split_size, num_splits, batch_count, stream);
}

hipError_t gemma4_decode_split_plan(Gemma4KvCacheConfig config,
                                    int32_t batch_count, int32_t max_live_keys,
                                    int32_t target_workgroups,
                                    int32_t *split_size, int32_t *num_splits) {
  if (split_size == nullptr || num_splits == nullptr || batch_count <= 0 ||
      max_live_keys < 0 || config.num_heads <= 0) {
    return hipErrorInvalidValue;
  }
  int32_t tile;
  if (config.num_heads == 8 && config.head_dim == 256) {
    tile = SlidingShape::KT;
  } else if (config.num_heads == 1 && config.head_dim == 512) {
    tile = GlobalRefShape::KT;
  } else {
    return hipErrorInvalidValue;
  }
  if (target_workgroups <= 0) target_workgroups = 512;  // two per CU on 256 CUs
  const int64_t keys = (int64_t)std::max(max_live_keys, 1);
  const int64_t heads = (int64_t)batch_count * config.num_heads;
  int64_t splits_per_seq = (target_workgroups + heads - 1) / heads;
  if (splits_per_seq < 1) splits_per_seq = 1;
  int64_t size = (keys + splits_per_seq - 1) / splits_per_seq;
  size = ((size + tile - 1) / tile) * tile;
  if (size < tile) size = tile;
  *split_size = (int32_t)size;
  *num_splits = (int32_t)((keys + size - 1) / size);
  return hipSuccess;
}

}  // extern "C"
