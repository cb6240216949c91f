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
//
// Workgroup = (kv head, 64 chunk rows), 4 waves, one per SIMD; wave w owns
// rows [16w, 16w+16) for both GQA heads of the kv head (32 MFMA columns).
// Keys stream in tiles of 64 through two LDS stages. Each tile's K and V rows
// are copied into LDS by the waves themselves with global_load_lds (no
// register staging): wave w copies keys [16w, 16w+16) of the tile, one 1 KiB
// instruction per key pair, from addresses its lanes resolved through the
// page table one tile earlier. The rows land XOR-swizzled in 16-byte chunks:
//   * K row k, chunk c sits at chunk c ^ (k & 15): the 16 lanes of one
//     ds_read_b128 pass read 16 keys at one logical chunk without bank
//     conflicts;
//   * V row k, chunk c sits at chunk c ^ ((k & 3) << 2): ds_read_b64_tr_b16
//     hands lane i of a 16-lane group V[k0 + e][n0 + i] (e = 0..3) from four
//     rows x 32 bytes, which this layout spreads over all banks. The
//     transposing read turns row-major V into the V^T operand directly.
// Tile t+1 is copied while tile t is computed; one barrier per tile. The
// copies are issued between block 1's score MFMAs (inline asm, so the
// compiler neither serialises them nor waits on them; each wave waits for
// its own copies right before the barrier), the next tile's row addresses
// are resolved between block 0's score MFMAs, and the page-table entries
// those need arrive in LDS by a 4-byte copy issued two tiles ahead.
// Each score block first issues all 16 of its K-fragment reads (into AGPRs),
// then its MFMA chain, so LDS latency is paid once per block. The MFMAs use
// the VGPR accumulator form (a build flag for this file): with AGPR
// accumulators the rarely taken rescale path made the compiler copy all 128
// accumulators between register files on every tile.
// Softmax maxima are updated lazily: the running max moves (and the
// accumulators are rescaled) only when a row's new maximum exceeds it by
// more than 8 in log2 units, so exp2 arguments stay <= 8 and the result is
// unchanged up to rounding. Blocks of 32 keys that no row of a wave sees
// skip their MFMAs (not their share of the copies), and blocks every row
// sees skip the mask. Blocks are ordered head-fastest so the workgroups of
// one kv head land on one XCD and share its L2 as they stream the same keys.
#include "gemma4_device.hpp"
#include "lds_copy.hpp"

#include "gemma4_flash_attention.h"

#include <math.h>

#include <type_traits>

namespace gemma4 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr int kPrefillThreads = 256;
constexpr int kPrefillWaves = kPrefillThreads / kWave;
constexpr int kPrefillRows = 64;                 // chunk rows per workgroup
constexpr int kDim = 256;                        // head_dim of the supported geometry
constexpr int kRowBytes = kDim * 2;              // one bf16 K or V row of a head
constexpr int kTileKeys = 64;                    // keys per LDS stage
constexpr int kTileBytes = kTileKeys * kRowBytes;  // 32 KiB per stage and operand
constexpr int kCopyKeys = kTileKeys / kPrefillWaves;  // keys each wave copies per tile
constexpr float kRescaleSlack = 8.0f;           // log2 headroom of the lazy max

struct PrefillParams {
  uint16_t *out;             // [B][Lq][16][D]
  const uint16_t *q;         // [B][Lq][16][D]
  const uint16_t *k;         // [B][Lq][Hk][D] chunk keys
  const uint16_t *v;
  const uint16_t *cache_k;   // paged prior keys (null when no prior)
  const uint16_t *cache_v;
  const int32_t *page_table;
  const int32_t *prior;      // [B] keys already in the cache (null: 0)
  Gemma4KvCacheConfig c;
  int32_t layer;
  int32_t chunk_len;
  int32_t window;            // 0: global (causal only)
  float q_scale;             // softmax_scale * log2(e)
  // Balanced global chunks (n_pairs > 0): row blocks j and nb-1-j form a
  // pair served by two workgroups with equal key work; the one row block a
  // pair splits meets in its slot of the workspace.
  int32_t n_pairs;
  char *ws;
};

constexpr int kPartialFloats = 130;  // per thread: 128 accumulators, max, sum
// Workspace slot s at s * kSlotBytes: the arrival counter (256-byte
// aligned), then the two halves' partials (kPartialFloats x 256 floats
// each, element-major). A slot sits at the same place for every chunk
// length, so calls of different sizes can share a workspace.
constexpr int64_t kSlotCounterBytes = 256;
constexpr int64_t kSlotBytes = kSlotCounterBytes + 2LL * kPartialFloats * kPrefillThreads * 4;

__device__ __forceinline__ f32x16_t mfma32(uint4 a, uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Two fp32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  const f32x2_t f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

// floor(n / d) for 0 <= n < 2^24 and d >= 1, from the fp32 reciprocal plus
// one correction step each way.
__device__ __forceinline__ int div_small(int n, int d, float inv_d) {
  int q = (int)((float)n * inv_d);
  q += (q + 1) * d <= n ? 1 : 0;
  q -= q * d > n ? 1 : 0;
  return q;
}

typedef unsigned u32x4v_t __attribute__((ext_vector_type(4)));

// Issues the 16 K-fragment reads of one S^T block (32 keys x 256 dims) so
// that all are in flight before the first MFMA; the fragments land in AGPRs.
// k_addr is the LDS byte address of k-step 0 for this lane; k-step s sits at
// k_addr ^ (s << 5) (the XOR swizzle of the K rows, see the kernel comment),
// plus kImm for the stage and block. The swizzle changes chunk bits 0..3
// only, so k-step s + 8 sits 256 bytes after k-step s: the reads go out in
// pairs (s, s + 8) from one XORed address, in issue order 0, 8, 1, 9, ...
// (kFragOrder). The reads are invisible to the compiler's counters: fragment
// s is consumed only after kfrag_ready(s).
template <int kImm>
__device__ __forceinline__ void read_kfrags(uint32_t k_addr, u32x4v_t (&kf)[16]) {
  uint32_t t0, t1;
  asm volatile(
      "s_waitcnt lgkmcnt(0)\n\t"
      "v_xor_b32 %[t0], 0, %[ka]\n\t"
      "ds_read_b128 %[f0], %[t0] offset:%[imm]\n\t"
      "ds_read_b128 %[f8], %[t0] offset:%[imm2]\n\t"
      "v_xor_b32 %[t1], 32, %[ka]\n\t"
      "ds_read_b128 %[f1], %[t1] offset:%[imm]\n\t"
      "ds_read_b128 %[f9], %[t1] offset:%[imm2]\n\t"
      "v_xor_b32 %[t0], 64, %[ka]\n\t"
      "ds_read_b128 %[f2], %[t0] offset:%[imm]\n\t"
      "ds_read_b128 %[f10], %[t0] offset:%[imm2]\n\t"
      "v_xor_b32 %[t1], 96, %[ka]\n\t"
      "ds_read_b128 %[f3], %[t1] offset:%[imm]\n\t"
      "ds_read_b128 %[f11], %[t1] offset:%[imm2]\n\t"
      "v_xor_b32 %[t0], 128, %[ka]\n\t"
      "ds_read_b128 %[f4], %[t0] offset:%[imm]\n\t"
      "ds_read_b128 %[f12], %[t0] offset:%[imm2]\n\t"
      "v_xor_b32 %[t1], 160, %[ka]\n\t"
      "ds_read_b128 %[f5], %[t1] offset:%[imm]\n\t"
      "ds_read_b128 %[f13], %[t1] offset:%[imm2]\n\t"
      "v_xor_b32 %[t0], 192, %[ka]\n\t"
      "ds_read_b128 %[f6], %[t0] offset:%[imm]\n\t"
      "ds_read_b128 %[f14], %[t0] offset:%[imm2]\n\t"
      "v_xor_b32 %[t1], 224, %[ka]\n\t"
      "ds_read_b128 %[f7], %[t1] offset:%[imm]\n\t"
      "ds_read_b128 %[f15], %[t1] offset:%[imm2]"
      : [t0] "=&v"(t0), [t1] "=&v"(t1),
        [f0] "=&a"(kf[0]), [f1] "=&a"(kf[1]), [f2] "=&a"(kf[2]), [f3] "=&a"(kf[3]), [f4]
        "=&a"(kf[4]), [f5] "=&a"(kf[5]), [f6] "=&a"(kf[6]), [f7] "=&a"(kf[7]), [f8]
        "=&a"(kf[8]), [f9] "=&a"(kf[9]), [f10] "=&a"(kf[10]), [f11] "=&a"(kf[11]), [f12]
        "=&a"(kf[12]), [f13] "=&a"(kf[13]), [f14] "=&a"(kf[14]), [f15] "=&a"(kf[15])
      : [ka] "v"(k_addr), [imm] "i"(kImm), [imm2] "i"(kImm + 256));
}

// Issue position p of read_kfrags reads k-step kFragOrder(p).
constexpr int kFragOrder(int p) { return (p >> 1) + 8 * (p & 1); }
// Issue position of k-step s.
constexpr int kFragPos(int s) { return s < 8 ? 2 * s : 2 * (s - 8) + 1; }

// Waits until fragment kStep of read_kfrags has landed (LDS returns in
// order, so at most 15 - kFragPos(kStep) of the block's reads may still be
// pending; any other LDS or scalar load in flight only makes the wait
// stricter).
template <int kStep>
__device__ __forceinline__ void kfrag_ready(u32x4v_t &f) {
  asm volatile("s_waitcnt lgkmcnt(%[n])" : "+a"(f) : [n] "i"(15 - kFragPos(kStep)));
}

// f(integral_constant<int, I>) for I = kBegin .. kEnd-1, unrolled.
template <int kBegin, int kEnd, class F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (kBegin < kEnd) {
    f(std::integral_constant<int, kBegin>{});
    static_for<kBegin + 1, kEnd>(f);
  }
}

template <int kSt>
using Stage = std::integral_constant<int, kSt>;

template <bool kPaired>
__global__ __launch_bounds__(kPrefillThreads, 1) void prefill_chunk_kernel(PrefillParams p) {
  constexpr int KS = kDim / 16;        // k-steps of S^T (dims)
  constexpr int DB = kDim / 32;        // 32-dim blocks of O^T
  // One LDS object with a fixed layout. V stages come first: the
  // transposing reads address them with a 16-bit immediate offset, which
  // reaches only the first 64 KiB. K stages are read by read_kfrags (inline
  // asm, base in a register); their 512-byte alignment keeps the XOR
  // swizzle out of the base address. All LDS copies are inline asm, so the
  // compiler needs no per-object aliasing to keep them apart from its reads.
  struct Lds {
    uint4 v[2][kTileBytes / 16];
    uint4 k[2][kTileBytes / 16];
    uint32_t valid[2][kPrefillWaves];      // bit j: key 16w + j of the stage is readable
    uint4 rows[kPrefillWaves][kCopyKeys];  // {K address, V address} per copied key
    int32_t pages[2][kPrefillWaves][kWave];  // page-table entry per copied key (lane % 16)
  };
  __shared__ __attribute__((aligned(1024))) Lds lds;
  uint4 *const s_v0 = lds.v[0];
  uint4 *const s_v1 = lds.v[1];
  auto &s_k = lds.k;
  auto &s_valid = lds.valid;
  auto &s_rows = lds.rows;
  auto &s_pages = lds.pages;

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = wave_uniform(t >> 6);
  const int half = lane >> 5;       // lane / 32
  const int n = lane & 31;          // MFMA column = query row of this lane
  const int Hk = p.c.num_heads;
  const int head = blockIdx.x % Hk;
  const int b = blockIdx.y;
  const int Lq = p.chunk_len;
  const int prior = p.prior != nullptr ? wave_uniform(p.prior[b]) : 0;

  // ---- work units: (row block, tile range, split slot) -------------------
  // Plain: one row block per workgroup. Balanced (global chunks): row
  // blocks j and J = nb-1-j need T(j) + T(J) key tiles together; workgroup
  // A takes block j and the first x tiles of block J, workgroup B the other
  // T(J) - x, with x chosen so both get half. A split block's two halves
  // merge through the workspace.
  // The (at most two) units are named values, not an array indexed by a
  // runtime count, so they stay in registers (no scratch).
  struct Unit {
    int q0, t_lo, t_hi, slot, part;
  };
  constexpr int kAllTiles = 1 << 30;
  Unit unit0 = {0, 0, 0, -1, 0}, unit1 = {0, 0, 0, -1, 0};
  int n_units = 0;
  if constexpr (kPaired) {
    const int rest = blockIdx.x / Hk;
    const int pair = rest >> 1, side = rest & 1;
    const int nb = (Lq + kPrefillRows - 1) / kPrefillRows;
    const int j = pair, J = nb - 1 - pair;
    auto tiles_of = [&](int blk) {  // causal, no window: tiles 0 .. last key
      return (prior + min(kPrefillRows * (blk + 1), Lq) - 1) / kTileKeys + 1;
    };
    if (j == J) {
      if (side == 0) {
        unit0 = {kPrefillRows * j, 0, kAllTiles, -1, 0};
        n_units = 1;
      }
    } else if (j < J) {
      const int tj = tiles_of(j), tJ = tiles_of(J);
      int x = (tj + tJ) / 2 - tj;
      x = x < 0 ? 0 : (x > tJ ? tJ : x);
      const int slot = (b * Hk + head) * p.n_pairs + pair;
      if (side == 0) {
        unit0 = {kPrefillRows * j, 0, kAllTiles, -1, 0};
        n_units = 1;
        if (x > 0) {
          unit1 = {kPrefillRows * J, 0, x, x < tJ ? slot : -1, 0};
          n_units = 2;
        }
      } else if (x < tJ) {
        unit0 = {kPrefillRows * J, x, kAllTiles, x > 0 ? slot : -1, 1};
        n_units = 1;
      }
    }
  } else {
    unit0 = {(int)(blockIdx.x / Hk) * kPrefillRows, 0, kAllTiles, -1, 0};
    n_units = 1;
  }
  __shared__ int s_last;

  for (int u = 0; u < n_units; ++u) {
  const Unit &cur = u == 0 ? unit0 : unit1;
  const int q0 = wave_uniform(cur.q0);
  const int unit_lo = wave_uniform(cur.t_lo);
  const int unit_hi = wave_uniform(cur.t_hi);
  const int unit_slot = wave_uniform(cur.slot);
  const int unit_part = wave_uniform(cur.part);

  // Rows of this lane: chunk row r = q0 + 16*wave + n % 16, q head 2*head + n / 16
  // (G = 2 for 16 query heads over 8 kv heads).
  const int G = kQueryHeads / Hk;
  const int g = n / 16;
  const int row = q0 + 16 * wave + n % 16;
  const bool row_ok = row < Lq && g < G;
  const int qh = head * G + g;
  const int qpos = prior + row;  // absolute position of this query row
  const int win_lo = p.window > 0 ? qpos - p.window : -1;  // visible: win_lo < kp <= qpos
  // Wave-uniform row span for the block skip / no-mask tests.
  const int wave_row0 = q0 + 16 * wave;
  const bool wave_has_rows = wave_row0 < Lq;
  const bool wave_rows_full = wave_row0 + 15 < Lq;
  const int wave_qmin = prior + wave_row0;
  const int wave_qmax = prior + min(wave_row0 + 15, Lq - 1);

  // Q^T operand: lane holds Q[row][16s + 8*half .. +8] for every k-step s.
  u32x4v_t qreg[KS];
  {
    const uint16_t *qrow =
        p.q + (((int64_t)b * Lq + (row_ok ? row : 0)) * kQueryHeads + qh) * kDim;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint4 x = row_ok ? load128(qrow + 16 * s + 8 * half) : make_uint4(0, 0, 0, 0);
      qreg[s] = u32x4v_t{x.x, x.y, x.z, x.w};
    }
  }

  // Key range of the workgroup (absolute positions), tile-aligned start.
  const int wg_last = prior + min(q0 + kPrefillRows, Lq) - 1;  // last visible key of any row
  int kstart = p.window > 0 ? prior + q0 - p.window + 1 : 0;
  kstart = kstart < 0 ? 0 : kstart;
  const int tile0_rows = (kstart / kTileKeys) * kTileKeys;
  const int n_tiles_rows = (wg_last - tile0_rows) / kTileKeys + 1;
  // This unit's tiles of the row block.
  const int tile0 = tile0_rows + unit_lo * kTileKeys;
  const int n_tiles = min(n_tiles_rows, unit_hi) - unit_lo;

  // ---- key rows: page lookup one tile ahead, addresses at copy time ------
  // Lane j (= lane % 16) of wave w resolves key tile + 16w + j.
  const Gemma4KvCacheConfig &c = p.c;
  const bool paged = p.page_table != nullptr && prior > 0;
  const float inv_page = 1.0f / (float)c.page_size;
  const float inv_pages = 1.0f / (float)c.max_pages_per_seq;
  const int32_t *pt_row = paged ? p.page_table + (int64_t)b * c.max_pages_per_seq
                                : reinterpret_cast<const int32_t *>(p.q);
  const int key_lane = lane & (kCopyKeys - 1);
  // Address of the page-table entry of key kt + 16w + lane % 16.
  auto page_entry = [&](int kt) __attribute__((always_inline)) -> const int32_t * {
    int kp = kt + kCopyKeys * wave + key_lane;
    kp = kp < prior ? kp : prior - 1;  // chunk keys: any in-bounds slot
    kp = kp < 0 ? 0 : kp;
    // Without a prior context page_size = max_pages = 1 and pt_row is any
    // readable word, so the arithmetic needs no branch.
    const int lp = div_small(kp, c.page_size, inv_page);
    const int slot = lp - div_small(lp, c.max_pages_per_seq, inv_pages) * c.max_pages_per_seq;
    return pt_row + (paged ? slot : 0);
  };
  // Row r of this head starts at base + (r << kRowShift) bytes in both the
  // chunk tensor ([B][Lq][Hk][D], base = row 0 of sequence b) and the cache
  // layer ([pages * page_size][Hk][D], base = row 0 of the layer).
  constexpr int kRowShift = 12;  // log2(Hk * D * 2) for Hk = 8, D = 256
  const uint64_t chunk_k = reinterpret_cast<uint64_t>(p.k + ((int64_t)b * Lq * Hk + head) * kDim);
  const uint64_t chunk_v = reinterpret_cast<uint64_t>(p.v + ((int64_t)b * Lq * Hk + head) * kDim);
  const int64_t layer_elems = (int64_t)p.layer * c.num_pages * c.page_size * Hk * kDim;
  const uint64_t cache_k =
      paged ? reinterpret_cast<uint64_t>(p.cache_k + layer_elems + head * kDim) : chunk_k;
  const uint64_t cache_v =
      paged ? reinterpret_cast<uint64_t>(p.cache_v + layer_elems + head * kDim) : chunk_v;
  // Byte addresses of one key's K and V rows for this head, and whether the
  // key can be read (in range, on a mapped page). Unreadable keys point at
  // the first chunk row, which always exists, and are masked later. Written
  // without branches so the compiler can interleave it with MFMAs.
  auto resolve = [&](int kt, int32_t phys, uint4 &rows_out) __attribute__((always_inline)) -> bool {
    const int kp = kt + kCopyKeys * wave + key_lane;
    const bool is_chunk = kp >= prior;
    const int lp = div_small(kp, c.page_size, inv_page);
    const bool cache_ok = paged & (phys >= 0) & (phys < c.num_pages);
    const bool ok = (is_chunk & (kp <= wg_last)) | (!is_chunk & cache_ok);
    const uint32_t crow = (uint32_t)(phys * c.page_size + (kp - lp * c.page_size));
    const uint32_t row = ok ? (is_chunk ? (uint32_t)(kp - prior) : crow) : 0u;
    const bool use_cache = ok & !is_chunk;
    const uint64_t off = (uint64_t)row << kRowShift;
    const uint64_t ka = (use_cache ? cache_k : chunk_k) + off;
    const uint64_t va = (use_cache ? cache_v : chunk_v) + off;
    rows_out = make_uint4((uint32_t)ka, (uint32_t)(ka >> 32), (uint32_t)va, (uint32_t)(va >> 32));
    return ok;
  };

  // Source chunk of each copy lane: instruction a of a wave copies keys
  // 16w + 2a (lanes 0..31) and 16w + 2a + 1 (lanes 32..63); lane l fills
  // LDS chunk l % 32 of its key with the swizzled source chunk.
  auto src_k = [&](int a) __attribute__((always_inline)) {
    return (n ^ ((2 * a + half) & 15)) * 16;  // key index mod 16 (16w is a multiple of 16)
  };
  auto src_v = [&](int a) __attribute__((always_inline)) {
    return (n ^ (((2 * a + half) & 3) << 2)) * 16;
  };

  // Row addresses of the next tile: lane j < 16 resolves key 16w + j and
  // publishes {K row, V row} in the wave's row table and the stage's validity
  // bits; lane l then fetches key 16w + 2a + l/32 of copy a and adds its
  // swizzled source chunk.
  auto prepare_copy = [&](auto st, int kt, int32_t phys, uint64_t (&ksrc)[kCopyKeys / 2],
                          uint64_t (&vsrc)[kCopyKeys / 2]) __attribute__((always_inline)) {
    constexpr int S = decltype(st)::value;
    uint4 rows;
    const bool ok = resolve(kt, phys, rows);
    const uint32_t ok_bits = (uint32_t)__builtin_amdgcn_ballot_w64(ok) & 0xFFFFu;
    // Lanes with equal lane % 16 hold equal rows, so every lane stores
    // (no divergent branch in the way of instruction scheduling).
    s_rows[wave][key_lane] = rows;
    s_valid[S][wave] = ok_bits;
    uint4 rr[kCopyKeys / 2];
#pragma unroll
    for (int a = 0; a < kCopyKeys / 2; ++a) rr[a] = s_rows[wave][2 * a + half];
#pragma unroll
    for (int a = 0; a < kCopyKeys / 2; ++a) {
      ksrc[a] = (((uint64_t)rr[a].y << 32) | rr[a].x) + src_k(a);
      vsrc[a] = (((uint64_t)rr[a].w << 32) | rr[a].z) + src_v(a);
    }
  };
  // LDS byte address of this wave's copy destination in each stage.
  auto lds_addr = [](const void *ptr) __attribute__((always_inline)) -> uint32_t {
    return (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char *)ptr);
  };
  const int copy_row0 = kCopyKeys * wave * (kRowBytes / 16);
  const uint32_t k_dst[2] = {(uint32_t)wave_uniform(lds_addr(&s_k[0][copy_row0])),
                             (uint32_t)wave_uniform(lds_addr(&s_k[1][copy_row0]))};
  const uint32_t v_dst[2] = {(uint32_t)wave_uniform(lds_addr(&s_v0[copy_row0])),
                             (uint32_t)wave_uniform(lds_addr(&s_v1[copy_row0]))};

  // ---- LDS read offsets (bytes within a stage) ----------------------------
  // K operand of S^T k-step s: key 32*blk + n, logical chunk 2s + half.
  const uint32_t k_addr =
      (uint32_t)reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint4 *)&s_k[0][0]) +
      n * kRowBytes + ((half ^ (n & 15)) << 4);
  // V^T operand of dim block d: lane i of 16-lane group gsel reads key
  // k0 + j, dims 32d + 16 gsel + 4q (j = (lane % 16) / 4, q = lane % 4),
  // k0 = 32*blk + 16*s2 + 8*r + 4*half.
  const int vj = (lane & 15) >> 2;
  const int vq = lane & 3;
  const int vg = (lane >> 4) & 1;
  int voff[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
    voff[d] = (4 * half + vj) * kRowBytes + (((4 * (d ^ vj) + 2 * vg + (vq >> 1)) << 4) |
                                             ((vq & 1) << 3));

  // Online softmax state: lane's row; lanes l and l^32 share a row.
  float m_run = -INFINITY;
  float l_run = 0.0f;
  f32x16_t acc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) acc[d] = f32x16_t{};

  // One block of 32 keys: S^T, masked softmax, O^T += V^T P^T.
  // Next-tile work rides on the two blocks of a tile: the row addresses
  // are resolved (next_rows) while block 0's score MFMAs run, and the 16
  // copies are issued between block 1's score MFMAs. Both happen even when
  // a block itself is skipped.
  uint64_t ksrc[kCopyKeys / 2], vsrc[kCopyKeys / 2];
  auto issue_copies = [&](auto st) __attribute__((always_inline)) {
    constexpr int S = decltype(st)::value;
#pragma unroll
    for (int c = 0; c < kCopyKeys / 2; ++c) {
      copy_row_pair(ksrc[c], k_dst[S ^ 1] + c * 2 * kRowBytes);
      copy_row_pair(vsrc[c], v_dst[S ^ 1] + c * 2 * kRowBytes);
    }
  };
  auto attend_block = [&](auto st, auto blk, const char *vbase, int kb_lo, uint32_t valid32,
                          bool copy, auto &&next_rows) __attribute__((always_inline)) {
    constexpr int S = decltype(st)::value;
    constexpr int kBlk = decltype(blk)::value;
    constexpr int kImm = S * kTileBytes + kBlk * 32 * kRowBytes;
    const int kb_hi = kb_lo + 31;
    if (!wave_has_rows || kb_lo > wave_qmax || (p.window > 0 && kb_hi <= wave_qmin - p.window)) {
      if (copy) {
        if constexpr (kBlk == 0) {
          next_rows();
        } else {
          issue_copies(st);
        }
      }
      return;
    }
    const bool full = wave_rows_full && valid32 == 0xFFFFFFFFu && kb_hi <= wave_qmin &&
                      (p.window == 0 || kb_lo > wave_qmax - p.window);
    // S^T[key m][row n] = sum_d K[m][d] Q[n][d].
    u32x4v_t kf[KS];
    read_kfrags<kImm>(k_addr, kf);
    f32x16_t s_acc = f32x16_t{};
    // The k-steps in the order their fragments arrive (kFragOrder).
    auto step_s = [&](auto pc) __attribute__((always_inline)) {
      constexpr int pos = decltype(pc)::value;
      constexpr int s = kFragOrder(pos);
      kfrag_ready<s>(kf[s]);
      s_acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf[s]),
                                                      __builtin_bit_cast(bf16x8_t, qreg[s]), s_acc,
                                                      0, 0, 0);
      if constexpr (kBlk == 1) {
        if (copy) {
          if constexpr (pos % 2 == 0) {
            copy_row_pair(ksrc[pos / 2], k_dst[S ^ 1] + (pos / 2) * 2 * kRowBytes);
          } else {
            copy_row_pair(vsrc[pos / 2], v_dst[S ^ 1] + (pos / 2) * 2 * kRowBytes);
          }
        }
        // Each fragment's wait stays right before its MFMA (the scheduler
        // otherwise clusters the waits and the reads stop overlapping).
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    static_for<0, KS>(step_s);
    if constexpr (kBlk == 0) {
      if (copy) next_rows();
      // Interleave the address work with the score MFMAs.
      static_for<0, KS>([](auto) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // 3 VALU
      });
    }
    // Lane holds keys m = (i/4)*8 + 4*half + i%4, i = 0..15, of row n. The
    // maximum is taken over the raw scores (q_scale > 0) and the scale is
    // folded into the exp2 argument.
    float sc[16];
    if (full) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sc[i] = s_acc[i];
    } else {
      // Visible keys of this row as a 32-bit mask over the block: readable,
      // at or before the row, and inside its window.
      const int hi = qpos - kb_lo;        // last visible key index
      const int lo = win_lo + 1 - kb_lo;  // first visible key index
      const uint32_t below = hi < 0 ? 0u : (hi >= 31 ? 0xFFFFFFFFu : (2u << hi) - 1u);
      const uint32_t above = lo <= 0 ? 0xFFFFFFFFu : (lo > 31 ? 0u : 0xFFFFFFFFu << lo);
      const uint32_t vis = (row_ok ? valid32 & below & above : 0u) >> (4 * half);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int m = (i / 4) * 8 + (i % 4);
        sc[i] = (vis >> m) & 1u ? s_acc[i] : -INFINITY;
      }
    }
    float tmax = fmaxf(fmaxf(sc[0], sc[1]), sc[2]);
#pragma unroll
    for (int i = 3; i < 15; i += 2) tmax = fmaxf(fmaxf(tmax, sc[i]), sc[i + 1]);
    tmax = fmaxf(tmax, sc[15]);
    tmax = xor_max<32>(tmax) * p.q_scale;
    // Lazy maximum: move it (and rescale) only when a row outgrew it by more
    // than the slack; otherwise exp2 arguments stay below the slack.
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + kRescaleSlack) != 0) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DB; ++d) acc[d] *= alpha;
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    uint32_t pw[8];
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[i], p.q_scale, -m_use));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[i + 1], p.q_scale, -m_use));
      l_run += p0 + p1;
      pw[i / 2] = cvt_pk_bf16(p0, p1);
    }
    // O^T[dim][row] += sum over keys V^T[dim][key] P^T[key][row]; k-step s2
    // covers keys 16*s2 + {4h..4h+3, 8+4h..8+4h+3} for lane half h, the two
    // groups of four read by one transposing load each.
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const uint4 pb = make_uint4(pw[4 * s2], pw[4 * s2 + 1], pw[4 * s2 + 2], pw[4 * s2 + 3]);
      uint4 vf[DB];
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
        const char *base = vbase + (16 * s2) * kRowBytes + voff[d];
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4 *)(__attribute__((address_space(3))) char *)(base));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4 *)(__attribute__((address_space(3))) char *)(base + 8 * kRowBytes));
        const uint2 l2 = __builtin_bit_cast(uint2, lo);
        const uint2 h2 = __builtin_bit_cast(uint2, hi);
        vf[d] = make_uint4(l2.x, l2.y, h2.x, h2.y);
      }
#pragma unroll
      for (int d = 0; d < DB; ++d) acc[d] = mfma32(vf[d], pb, acc[d]);
    }
    // The block's 32 transposing V reads run two MFMAs ahead of its 16 P.V
    // MFMAs (the compiler's own order waits on each MFMA's reads right before
    // it; measured against 2 to 6 MFMAs of lead: 5-6% faster at this one).
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // 4 DS reads
    static_for<0, 14>([](auto) __attribute__((always_inline)) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // 2 DS reads
    });
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  };

  // ---- pipeline: copy tile i+1 and look up tile i+2 while computing i -----
  // The page-table entries of tile t land in s_pages[t & 1] by LDS copy,
  // issued two tiles ahead, so no vector register waits on them.
  const uint32_t page_dst[2] = {(uint32_t)wave_uniform(lds_addr(&s_pages[0][wave][0])),
                                (uint32_t)wave_uniform(lds_addr(&s_pages[1][wave][0]))};
  prepare_copy(Stage<0>{}, tile0, *page_entry(tile0), ksrc, vsrc);
  issue_copies(Stage<1>{});  // into stage 0
  copy_dwords(page_entry(tile0 + kTileKeys), page_dst[1]);
  auto step = [&](auto st, int it) __attribute__((always_inline)) {
    constexpr int S = decltype(st)::value;
    const int kt = tile0 + it * kTileKeys;
    // Tile it copied: each wave waits for its own copies, the barrier for all.
    // Every wave has also finished tile it-1, so stage S^1 is free.
    wait_copies();
    __syncthreads();
    // The copy after the last tile reads keys past the workgroup's range,
    // which resolve to the (always readable) first chunk row: the loop has
    // no branches around its copies.
    constexpr bool copy = true;
    const int32_t next_phys = s_pages[S ^ 1][wave][lane];
    auto next_rows = [&]() __attribute__((always_inline)) {
      prepare_copy(Stage<S ^ 1>{}, kt + kTileKeys, next_phys, ksrc, vsrc);
      copy_dwords(page_entry(kt + 2 * kTileKeys), page_dst[S]);
    };
    const char *vbase = reinterpret_cast<const char *>(S == 0 ? s_v0 : s_v1);
    const uint4 vw = *reinterpret_cast<const uint4 *>(&s_valid[S][0]);
    attend_block(st, std::integral_constant<int, 0>{}, vbase, kt, vw.x | (vw.y << 16), copy,
                 next_rows);
    attend_block(st, std::integral_constant<int, 1>{}, vbase + 32 * kRowBytes, kt + 32,
                 vw.z | (vw.w << 16), copy, next_rows);
  };
  for (int it = 0; it < n_tiles; it += 2) {
    step(Stage<0>{}, it);
    if (it + 1 < n_tiles) step(Stage<1>{}, it + 1);
  }
  wait_copies();  // no copy may still be writing LDS when the unit ends

  // A split row block: store this half's partial (device-coherent: the
  // other half may run on another XCD), count the arrival, and let the
  // second arriver merge both halves and write the rows.
  bool emit = true;
  if (unit_slot >= 0) {
    char *slot = p.ws + (int64_t)unit_slot * kSlotBytes;
    float *part = reinterpret_cast<float *>(slot + kSlotCounterBytes);
    float *mine = part + unit_part * kPartialFloats * kPrefillThreads;
    const float *other = part + (unit_part ^ 1) * kPartialFloats * kPrefillThreads;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        __hip_atomic_store(mine + (d * 16 + i) * kPrefillThreads + t, acc[d][i], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    __hip_atomic_store(mine + 128 * kPrefillThreads + t, m_run, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(mine + 129 * kPrefillThreads + t, l_run, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
    __syncthreads();
    if (t == 0) {
      // Release: the workgroup's partial stores (complete at the barrier)
      // are ordered before the arrival; acquire: the first arriver's partial
      // is visible to the second arriver.
      int32_t *counter = reinterpret_cast<int32_t *>(slot);
      const int32_t arrived =
          __hip_atomic_fetch_add(counter, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      if (arrived == 1) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = arrived == 1 ? 1 : 0;
    }
    __syncthreads();
    emit = s_last != 0;
    if (emit) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      const float mo = __hip_atomic_load(other + 128 * kPrefillThreads + t, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
      const float lo = __hip_atomic_load(other + 129 * kPrefillThreads + t, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
      const float mm = fmaxf(m_run, mo);
      const float fa = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - mm);
      const float fb = mo == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mo - mm);
      l_run = l_run * fa + lo * fb;
#pragma unroll
      for (int d = 0; d < DB; ++d) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float ao = __hip_atomic_load(other + (d * 16 + i) * kPrefillThreads + t,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          acc[d][i] = acc[d][i] * fa + ao * fb;
        }
      }
      m_run = mm;
    }
  }

  if (emit) {
    // Normalise and store: lane holds dims 32d + (i/4)*8 + 4*half + i%4 of row n.
    l_run = xor_sum<32>(l_run);
    if (row_ok) {
      const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
      uint16_t *orow = p.out + (((int64_t)b * Lq + row) * kQueryHeads + qh) * kDim;
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
  }
  if constexpr (kPaired) __syncthreads();  // the next unit reuses the LDS stages and tables
  }  // units
}

}  // namespace
}  // namespace gemma4

using namespace gemma4;

namespace {

// Balanced-mode geometry of a chunk: row-block pairs per (sequence, head) and
// the workspace bytes (one slot per pair).
int prefill_pairs(int32_t chunk_len) {
  const int nb = (chunk_len + kPrefillRows - 1) / kPrefillRows;
  return nb < 2 ? 0 : (nb + 1) / 2;
}
size_t prefill_workspace_bytes(int32_t batch_size, int32_t chunk_len, int32_t heads) {
  if (batch_size <= 0 || chunk_len <= 0 || heads <= 0) return 0;
  const int64_t slots = (int64_t)batch_size * heads * prefill_pairs(chunk_len);
  return (size_t)(slots * kSlotBytes);
}

hipError_t prefill_chunk_launch(gemma4_bf16 *d_out, const gemma4_bf16 *d_q, const gemma4_bf16 *d_k,
                                const gemma4_bf16 *d_v, const gemma4_bf16 *d_cache_k,
                                const gemma4_bf16 *d_cache_v, const int32_t *d_page_table,
                                const int32_t *d_prior_lengths, Gemma4KvCacheConfig config,
                                int32_t layer, int32_t batch_size, int32_t chunk_len,
                                float softmax_scale, void *d_workspace, size_t workspace_bytes,
                                bool balanced, hipStream_t stream) {
  if (batch_size == 0 || chunk_len == 0) return hipSuccess;
  const bool paged = d_prior_lengths != nullptr;
  if (batch_size < 0 || chunk_len < 0 || batch_size > 65535 || !(softmax_scale > 0.0f) ||
      d_out == nullptr || d_q == nullptr || d_k == nullptr || d_v == nullptr ||
      config.num_heads != 8 || config.head_dim != kDim || config.window_size < 0) {
    return hipErrorInvalidValue;
  }
  if (paged && (d_cache_k == nullptr || d_cache_v == nullptr || d_page_table == nullptr ||
                layer < 0 || layer >= config.num_layers || config.page_size <= 0 ||
                config.max_pages_per_seq <= 0 || config.num_pages <= 0 ||
                batch_size > config.batch_size)) {
    return hipErrorInvalidValue;
  }
  const size_t need = prefill_workspace_bytes(batch_size, chunk_len, config.num_heads);
  if (balanced && (d_workspace == nullptr || workspace_bytes < need ||
                   (reinterpret_cast<uintptr_t>(d_workspace) & 255) != 0)) {
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
  if (!paged) {
    // Without a prior context no page is read; keep the divisors valid.
    p.c.page_size = 1;
    p.c.max_pages_per_seq = 1;
  }
  p.layer = paged ? layer : 0;
  p.chunk_len = chunk_len;
  p.window = config.window_size;
  p.q_scale = softmax_scale * kLog2e;
  // Sliding chunks already carry equal work per row block; only causal
  // (global) chunks of two or more row blocks are paired.
  p.n_pairs = balanced && config.window_size == 0 ? prefill_pairs(chunk_len) : 0;
  p.ws = p.n_pairs > 0 ? static_cast<char *>(d_workspace) : nullptr;
  int blocks = config.num_heads * ((chunk_len + kPrefillRows - 1) / kPrefillRows);
  if (p.n_pairs > 0) blocks = config.num_heads * 2 * p.n_pairs;
  if (p.n_pairs > 0) {
    hipLaunchKernelGGL(prefill_chunk_kernel<true>, dim3(blocks, batch_size),
                       dim3(kPrefillThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL(prefill_chunk_kernel<false>, dim3(blocks, batch_size),
                       dim3(kPrefillThreads), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace

extern "C" hipError_t gemma4_flash_attention_prefill_chunk_paged_bf16(
    gemma4_bf16 *d_out, const gemma4_bf16 *d_q, const gemma4_bf16 *d_k,
    const gemma4_bf16 *d_v, const gemma4_bf16 *d_cache_k, const gemma4_bf16 *d_cache_v,
    const int32_t *d_page_table, const int32_t *d_prior_lengths, Gemma4KvCacheConfig config,
    int32_t layer, int32_t batch_size, int32_t chunk_len, float softmax_scale,
    hipStream_t stream) {
  return prefill_chunk_launch(d_out, d_q, d_k, d_v, d_cache_k, d_cache_v, d_page_table,
                              d_prior_lengths, config, layer, batch_size, chunk_len,
                              softmax_scale, nullptr, 0, false, stream);
}

extern "C" size_t gemma4_flash_attention_prefill_chunk_workspace_bytes(
    int32_t batch_size, int32_t chunk_len, Gemma4KvCacheConfig config) {
  return config.window_size == 0 ? prefill_workspace_bytes(batch_size, chunk_len, config.num_heads)
                                 : 0;
}

extern "C" hipError_t gemma4_flash_attention_prefill_chunk_paged_bf16_ws(
    gemma4_bf16 *d_out, const gemma4_bf16 *d_q, const gemma4_bf16 *d_k,
    const gemma4_bf16 *d_v, const gemma4_bf16 *d_cache_k, const gemma4_bf16 *d_cache_v,
    const int32_t *d_page_table, const int32_t *d_prior_lengths, Gemma4KvCacheConfig config,
    int32_t layer, int32_t batch_size, int32_t chunk_len, float softmax_scale,
    void *d_workspace, size_t workspace_bytes, hipStream_t stream) {
  const bool balanced = config.window_size == 0 && prefill_pairs(chunk_len) > 0;
  return prefill_chunk_launch(d_out, d_q, d_k, d_v, d_cache_k, d_cache_v, d_page_table,
                              d_prior_lengths, config, layer, batch_size, chunk_len,
                              softmax_scale, d_workspace, workspace_bytes, balanced, stream);
}
