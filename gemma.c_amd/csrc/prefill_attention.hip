// Causal (optionally sliding-window) GQA prefill attention for gfx950 with
// bf16 MFMA, over a chunk of new rows whose earlier keys may live in the paged
// cache. Replaces the FA2 forward kernel of gemma.c
// (src/gemma4_flash_attention_prefill.cu:767-954: Q tile staged once, K/V
// blocks streamed, S = QK^T by tensor-core MMA, masked online softmax, P·V,
// normalise) and extends it to seqlen_k > seqlen_q with the prior keys read
// through the page table (the mask is the reference's,
// src/gemma4_flash_attention_prefill.cu:524-535).
//
// Formulation: the kernel computes S^T = K·Q^T and O^T = V^T·P^T with
// v_mfma_f32_32x32x16_bf16. In the 32x32 accumulator layout lane l holds
// column n = l % 32 (one query row) and 16 key/dim entries, so
//   * a query row's softmax max needs one cross-lane exchange (lane ^ 32),
//   * the online-softmax rescale is a per-lane scalar,
//   * P^T feeds the second MFMA straight from registers (the contraction's
//     key order is permuted to match, and V^T is read in that order).
// Workgroup = (kv head, 64 chunk rows), 4 waves; wave w owns rows
// [16w, 16w+16) for both GQA heads of the kv head (32 MFMA columns). K tiles
// (32 keys) are staged row-major and V tiles transposed into LDS, double
// buffered, with the next tile's global loads in flight during the current
// tile's MFMAs. Blocks are ordered head-fastest so the workgroups of one kv
// head land on one XCD and share its L2 as they stream the same keys.
#include "gemma4_device.hpp"

#include "gemma4_flash_attention.h"

#include <math.h>

namespace gemma4 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kPrefillThreads = 256;
constexpr int kPrefillRows = 64;     // chunk rows per workgroup
constexpr int kKeyTile = 32;         // keys per K/V tile
constexpr int kKPad = 8;             // bf16 pad per K row (bank spread)
constexpr int kVPad = 8;             // bf16 pad per V^T row

struct PrefillParams {
  uint16_t *out;             // [B][Lq][16][D]
  const uint16_t *q;         // [B][Lq][16][D]
  const uint16_t *k;         // [B][Lq][Hk][D] chunk keys
  const uint16_t *v;
  const uint16_t *cache_k;   // paged prior keys (may be null when no prior)
  const uint16_t *cache_v;
  const int32_t *page_table;
  const int32_t *prior;      // [B] keys already in the cache (null: 0)
  Gemma4KvCacheConfig c;
  int32_t layer;
  int32_t chunk_len;
  int32_t window;            // 0: global (causal only)
  float q_scale;             // softmax_scale * log2(e)
};

__device__ __forceinline__ f32x16_t mfma32(uint4 a, uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

template <int D>
struct PrefillSmem {
  uint16_t k[2][kKeyTile][D + kKPad];
  uint16_t vt[2][D][kKeyTile + kVPad];
  alignas(16) int32_t valid[2][kKeyTile];
};

template <int D>
__global__ __launch_bounds__(kPrefillThreads, 1) void prefill_chunk_kernel(PrefillParams p) {
  static_assert(D == 256, "tile shapes are sized for head_dim 256");
  constexpr int KS = D / 16;        // k-steps of S^T (dims)
  constexpr int DB = D / 32;        // 32-dim blocks of O^T
  constexpr int KCH = kKeyTile * D / 8 / kPrefillThreads;  // 16-B K chunks per thread per tile
  __shared__ PrefillSmem<D> sm;

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = wave_uniform(t >> 6);
  const int half = lane >> 5;       // lane / 32
  const int n = lane & 31;          // MFMA column = query row of this lane
  const int Hk = p.c.num_heads;
  const int head = blockIdx.x % Hk;
  const int q0 = (blockIdx.x / Hk) * kPrefillRows;
  const int b = blockIdx.y;
  const int Lq = p.chunk_len;
  const int prior = p.prior != nullptr ? p.prior[b] : 0;

  // Rows of this lane: chunk row r = q0 + 16*wave + n % 16, q head 2*head + n / 16
  // (G = 2 for 16 query heads over 8 kv heads).
  const int G = kQueryHeads / Hk;
  const int r_local = n % 16;
  const int g = n / 16;
  const int row = q0 + 16 * wave + r_local;
  const bool row_ok = row < Lq && g < G;
  const int qh = head * G + g;
  const int qpos = prior + row;  // absolute position of this query row

  // Q^T operand: lane holds Q[row][16s + 8*half .. +8] for every k-step s.
  uint4 qreg[KS];
  {
    const uint16_t *qrow = p.q + (((int64_t)b * Lq + (row_ok ? row : 0)) * kQueryHeads + qh) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qreg[s] = row_ok ? load128(qrow + 16 * s + 8 * half) : make_uint4(0, 0, 0, 0);
    }
  }

  // Key range of the workgroup (absolute positions), tile-aligned start.
  const int wg_last = prior + min(q0 + kPrefillRows, Lq) - 1;  // last visible key of any row
  int kstart = p.window > 0 ? prior + q0 - p.window + 1 : 0;
  kstart = kstart < 0 ? 0 : kstart;
  const int tile0 = (kstart / kKeyTile) * kKeyTile;
  const int n_tiles = wg_last < tile0 ? 0 : (wg_last - tile0) / kKeyTile + 1;

  // Staging assignment. K: thread t copies 16-B part (t % 32) of keys
  // t/32 + 8i. V: thread t transposes keys 4*(t%8)..+3 x dims 8*(t/8)..+7.
  // Thread-local key j (0..3 for K, 4..7 for V) of a tile at kt:
  const int kpart = t % 32;
  const int vkg = t % 8;
  const int vdg = t / 8;
  auto tile_key = [&](int j) { return j < 4 ? t / 32 + 8 * j : 4 * vkg + (j - 4); };

  // Page lookups run two tiles ahead of the MFMAs: fetch_pages issues the
  // page-table loads of a tile's prior keys; issue_tile turns them into
  // source rows and issues the K/V loads of the next tile. Every load is
  // unconditional (a harmless in-bounds word / dummy row when there is
  // nothing to read) so no divergent branch disturbs the wait counters.
  const Gemma4KvCacheConfig &c = p.c;
  const bool paged = p.page_table != nullptr && prior > 0;
  const float inv_page = 1.0f / (float)c.page_size;
  auto page_of = [&](int kp) {  // kp / page_size for 0 <= kp < 2^24
    int lp = (int)((float)kp * inv_page);
    lp += (lp + 1) * c.page_size <= kp ? 1 : 0;
    lp -= lp * c.page_size > kp ? 1 : 0;
    return lp;
  };
  const int32_t *pt_row = paged ? p.page_table + b * c.max_pages_per_seq
                                : reinterpret_cast<const int32_t *>(p.q);
  const int pt_mod = paged ? c.max_pages_per_seq : 1;
  auto fetch_pages = [&](int kt, int32_t (&pg)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int kp = kt + tile_key(j);
      kp = kp < prior ? kp : prior - 1;  // chunk keys: any in-bounds slot
      kp = kp < 0 ? 0 : kp;
      pg[j] = pt_row[page_of(kp) % pt_mod];
    }
  };
  // Element offset of one key's row for this head, or -1 when the key is out
  // of the workgroup's range or on an unmapped page; cache rows carry bit 62.
  constexpr int64_t kCacheBit = 1ll << 62;
  auto key_off = [&](int kp, int phys) -> int64_t {
    const int64_t chunk_off = (((int64_t)b * Lq + (kp - prior)) * Hk + head) * D;
    const int lp = page_of(kp < 0 ? 0 : kp);
    const int64_t crow = ((int64_t)p.layer * c.num_pages + phys) * c.page_size + (kp - lp * c.page_size);
    const int64_t cache_off = ((crow * Hk + head) * D) | kCacheBit;
    const bool in_range = kp >= 0 && kp <= wg_last;
    const bool cached_ok = paged && phys >= 0 && phys < c.num_pages;
    const int64_t off = kp >= prior ? chunk_off : (cached_ok ? cache_off : -1);
    return in_range ? off : -1;
  };
  auto src_of = [&](int64_t off, const uint16_t *cache, const uint16_t *chunk) {
    const uint16_t *base = (off & kCacheBit) ? cache : chunk;
    return off < 0 ? chunk : base + (off & ~kCacheBit);  // invalid: dummy row, masked later
  };

  struct Stage {
    uint4 k[KCH];
    uint4 v[4];
    uint32_t valid;  // bit i: K key t/32 + 8i valid; bit 4+i: V key 4*(t%8)+i valid
  };
  auto issue_tile = [&](Stage &st, int kt, const int32_t (&pg)[8]) {
    st.valid = 0;
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int64_t off = key_off(kt + tile_key(i), pg[i]);
      st.valid |= (off >= 0 ? 1u : 0u) << i;
      st.k[i] = load128(src_of(off, p.cache_k, p.k) + kpart * 8);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t off = key_off(kt + tile_key(4 + i), pg[4 + i]);
      st.valid |= (off >= 0 ? 1u : 0u) << (4 + i);
      st.v[i] = load128(src_of(off, p.cache_v, p.v) + vdg * 8);
    }
  };
  auto store_tile = [&](const Stage &st, int buf) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const bool ok = (st.valid >> i) & 1u;
      store128(&sm.k[buf][t / 32 + 8 * i][kpart * 8], ok ? st.k[i] : make_uint4(0, 0, 0, 0));
      if (kpart == 0) sm.valid[buf][t / 32 + 8 * i] = ok ? 1 : 0;
    }
    uint32_t w[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 vv = ((st.valid >> (4 + i)) & 1u) ? st.v[i] : make_uint4(0, 0, 0, 0);
      w[i][0] = vv.x; w[i][1] = vv.y; w[i][2] = vv.z; w[i][3] = vv.w;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
      uint2 pair;
      pair.x = __builtin_amdgcn_perm(w[1][e / 2], w[0][e / 2], sel);
      pair.y = __builtin_amdgcn_perm(w[3][e / 2], w[2][e / 2], sel);
      *reinterpret_cast<uint2 *>(&sm.vt[buf][vdg * 8 + e][4 * vkg]) = pair;
    }
  };

  // Online softmax state: lane's row; lanes l and l^32 share a row.
  float m_run = -INFINITY;
  float l_run = 0.0f;
  f32x16_t acc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) acc[d] = f32x16_t{};

  Stage st;
  int32_t pages[8];
  if (n_tiles > 0) {
    fetch_pages(tile0, pages);
    issue_tile(st, tile0, pages);
    fetch_pages(tile0 + kKeyTile, pages);
    store_tile(st, 0);
  }
  __syncthreads();

  for (int it = 0; it < n_tiles; ++it) {
    const int buf = it & 1;
    const int kt = tile0 + it * kKeyTile;
    const bool more = it + 1 < n_tiles;
    if (more) {
      issue_tile(st, kt + kKeyTile, pages);              // in flight during the MFMAs
      fetch_pages(kt + 2 * kKeyTile, pages);             // two tiles ahead
    }

    // S^T[key m][row n] = sum_d K[m][d] Q[n][d], as two independent chains.
    f32x16_t s_even = f32x16_t{}, s_odd = f32x16_t{};
#pragma unroll
    for (int s = 0; s < KS; s += 2) {
      const uint4 k0 = *reinterpret_cast<const uint4 *>(&sm.k[buf][n][16 * s + 8 * half]);
      const uint4 k1 = *reinterpret_cast<const uint4 *>(&sm.k[buf][n][16 * s + 16 + 8 * half]);
      s_even = mfma32(k0, qreg[s], s_even);
      s_odd = mfma32(k1, qreg[s + 1], s_odd);
    }
    const f32x16_t s_acc = s_even + s_odd;
    // Lane holds keys m = (i/4)*8 + 4*half + i%4, i = 0..15, of row n.
    int flags[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int4 f = *reinterpret_cast<const int4 *>(&sm.valid[buf][8 * j + 4 * half]);
      flags[4 * j] = f.x; flags[4 * j + 1] = f.y; flags[4 * j + 2] = f.z; flags[4 * j + 3] = f.w;
    }
    const int win_lo = p.window > 0 ? qpos - p.window : -1;  // visible: win_lo < kp <= qpos
    float sc[16];
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kp = kt + (i / 4) * 8 + 4 * half + (i % 4);
      const bool vis = row_ok & (flags[i] != 0) & (kp <= qpos) & (kp > win_lo);
      sc[i] = vis ? s_acc[i] * p.q_scale : -INFINITY;
      tmax = fmaxf(tmax, sc[i]);
    }
    tmax = fmaxf(tmax, lane_xor<32>(tmax));
    const float m_new = fmaxf(m_run, tmax);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    // Rescale only when some row's maximum moved (exactly; alpha == 1 else).
    if (__builtin_amdgcn_ballot_w64(m_new > m_run) != 0) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DB; ++d) acc[d] *= alpha;
    }
    m_run = m_new;
    uint32_t pw[8];
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = __builtin_amdgcn_exp2f(sc[i] - m_use);
      const float p1 = __builtin_amdgcn_exp2f(sc[i + 1] - m_use);
      l_run += p0 + p1;
      pw[i / 2] = pack_bf16x2(p0, p1);
    }
    // O^T[dim][row] += sum over keys V^T[dim][key] P^T[key][row]; k-step s2
    // covers keys 16*s2 + {4h..4h+3, 8+4h..8+4h+3} for lane half h.
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const uint4 pb = make_uint4(pw[4 * s2], pw[4 * s2 + 1], pw[4 * s2 + 2], pw[4 * s2 + 3]);
      uint4 vf[DB];  // all fragments of this k-step first: one LDS wait, then DB MFMAs
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        const uint16_t *vrow = &sm.vt[buf][32 * d + n][16 * s2 + 4 * half];
        const uint2 lo = *reinterpret_cast<const uint2 *>(vrow);
        const uint2 hi = *reinterpret_cast<const uint2 *>(vrow + 8);
        vf[d] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
#pragma unroll
      for (int d = 0; d < DB; ++d) acc[d] = mfma32(vf[d], pb, acc[d]);
    }
    if (more) store_tile(st, buf ^ 1);
    __syncthreads();
  }

  // Normalise and store: lane holds dims 32d + (i/4)*8 + 4*half + i%4 of row n.
  l_run += lane_xor<32>(l_run);
  if (!row_ok) return;
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  uint16_t *orow = p.out + (((int64_t)b * Lq + row) * kQueryHeads + qh) * D;
#pragma unroll
  for (int d = 0; d < DB; ++d) {
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      uint2 o;
      o.x = pack_bf16x2(acc[d][i] * inv, acc[d][i + 1] * inv);
      o.y = pack_bf16x2(acc[d][i + 2] * inv, acc[d][i + 3] * inv);
      *reinterpret_cast<uint2 *>(orow + 32 * d + (i / 4) * 8 + 4 * half) = o;
    }
  }
}

}  // namespace
}  // namespace gemma4

using namespace gemma4;

extern "C" hipError_t gemma4_flash_attention_prefill_chunk_paged_bf16(
    gemma4_bf16 *d_out, const gemma4_bf16 *d_q, const gemma4_bf16 *d_k,
    const gemma4_bf16 *d_v, const gemma4_bf16 *d_cache_k, const gemma4_bf16 *d_cache_v,
    const int32_t *d_page_table, const int32_t *d_prior_lengths, Gemma4KvCacheConfig config,
    int32_t layer, int32_t batch_size, int32_t chunk_len, float softmax_scale,
    hipStream_t stream) {
  if (batch_size == 0 || chunk_len == 0) return hipSuccess;
  const bool paged = d_prior_lengths != nullptr;
  if (batch_size < 0 || chunk_len < 0 || batch_size > 65535 || !(softmax_scale > 0.0f) ||
      d_out == nullptr || d_q == nullptr || d_k == nullptr || d_v == nullptr ||
      config.num_heads != 8 || config.head_dim != 256 || config.window_size < 0) {
    return hipErrorInvalidValue;
  }
  if (paged && (d_cache_k == nullptr || d_cache_v == nullptr || d_page_table == nullptr ||
                layer < 0 || layer >= config.num_layers || config.page_size <= 0 ||
                config.max_pages_per_seq <= 0 || config.num_pages <= 0 ||
                batch_size > config.batch_size)) {
    return hipErrorInvalidValue;
  }
  PrefillParams p;
  p.out = reinterpret_cast<uint16_t *>(d_out);
  p.q = reinterpret_cast<const uint16_t *>(d_q);
  p.k = reinterpret_cast<const uint16_t *>(d_k);
  p.v = reinterpret_cast<const uint16_t *>(d_v);
  p.cache_k = paged ? reinterpret_cast<const uint16_t *>(d_cache_k) : nullptr;
  p.cache_v = paged ? reinterpret_cast<const uint16_t *>(d_cache_v) : nullptr;
  p.page_table = paged ? d_page_table : nullptr;
  p.prior = d_prior_lengths;
  p.c = config;
  p.layer = layer;
  p.chunk_len = chunk_len;
  p.window = config.window_size;
  p.q_scale = softmax_scale * kLog2e;
  const int blocks = config.num_heads * ((chunk_len + kPrefillRows - 1) / kPrefillRows);
  hipLaunchKernelGGL(prefill_chunk_kernel<256>, dim3(blocks, batch_size),
                     dim3(kPrefillThreads), 0, stream, p);
  return hipGetLastError();
}
