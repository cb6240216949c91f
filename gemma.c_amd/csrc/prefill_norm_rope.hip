// Prefill self-attention launchers with Q/K/V preparation, gfx950: the drop-in
// for gemma4_flash_attention_{sliding,global}_fwd_bf16_norm_rope
// (src/gemma4_flash_attention.cuh:9-45, src/gemma4_flash_attention_prefill.cu:1110-1257).
// Each launcher runs two kernels on the caller's stream:
//   1. prefill_prep_kernel: per (token row, kv head) Q and K get learned
//      RMSNorm + split-half RoPE at the row's absolute position, V gets
//      scale-free RMSNorm (the 1x512 geometry derives V from the raw K), into
//      the caller's q/k/v_prepared buffers
//      (src/gemma4_flash_attention_prefill.cu:1023-1101);
//   2. causal attention over the prepared rows (seqlen_q == seqlen_k):
//      the 8x256 geometry reuses the chunk kernel (no prior context), the
//      1x512 geometry runs prefill_d512_kernel below.
//
// prefill_d512_kernel: 16 query heads share one 512-dim KV head. A wave owns
// one query row and all 16 heads (16 MFMA columns) on
// v_mfma_f32_16x16x32_bf16, computing S^T = K Q^T (16 keys x 16 heads per
// block, 16 k-steps of 32 dims) and O^T = V^T P^T (32 dim blocks of 16). In
// the 16x16 accumulator lane l holds head l % 16 and four keys (or dims)
// 4 (l/16) + i, so P^T feeds the second MFMA from registers when its 32-key
// contraction order is permuted to {4g..4g+3, 16+4g..16+4g+3} for lane
// group g, and V^T is read in that order by two ds_read_b64_tr_b16 per
// operand. O^T is 128 fp32 per lane (VGPR accumulator form, a build flag
// for this file), Q^T 64 registers held in AGPRs. A workgroup is four
// consecutive rows that share 32-key K/V tiles copied into two LDS stages
// with global_load_lds (tile t+1 in flight while tile t is computed; K chunk
// c of key k at c ^ (k & 15), V chunk c at c ^ ((k & 7) << 1), 16-byte
// chunks, so the operand reads are bank-conflict free). Scheduling: each
// score block issues its 16 K-fragment reads into AGPRs before its first
// MFMA (one counter wait per MFMA, two accumulator chains), and the P.V
// phase keeps its transposing V reads four MFMAs ahead. The lazy online
// softmax of the chunk kernel (maximum moved only when it grows by more than
// 8 in log2 units). Per 32-key tile a wave reads 64 KiB of K and V from LDS
// for 16 query columns, so the kernel is bound by LDS reads, not MFMA.
#include "gemma4_device.hpp"
#include "lds_copy.hpp"
#include "prep_common.hpp"

#include "gemma4_flash_attention.h"

#include <math.h>
#include <type_traits>

namespace gemma4 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));

struct PrefillPrepParams {
  uint16_t *q_prepared;  // [rows][16][D]
  uint16_t *k_prepared;  // [rows][Hk][D]
  uint16_t *v_prepared;
  const uint16_t *q;
  const uint16_t *k;
  const uint16_t *v;     // null for the 1x512 geometry (V from K)
  const uint16_t *q_norm_weight;
  const uint16_t *k_norm_weight;
  const float *cos;
  const float *sin;
  const int32_t *token_position;  // [rows]
};

// Workgroup (block of kPrepRows token rows, kv head), one wave per prepared
// head; a wave first loads its head of all kPrepRows rows, then prepares
// and stores them one by one, so the row loads overlap. A negative
// position skips the row (src/gemma4_flash_attention_prefill.cu:1049-1051).
// Two rows per workgroup: more, smaller workgroups measured faster for
// 2048 rows (launchers 8x256 / 1x512: 8 rows 67.5 / 164 us, 4 rows 64.5 /
// 157.3 us, 2 rows 63.5 / 157.4 us, 1 row 63.2 / 157.2 us, 16 rows 69.7 /
// 183.6 us).
constexpr int kPrepRows = 2;

template <int kHeads, int kDim, int kRotary, bool kHasV>
__global__ __launch_bounds__((prep_waves<kHeads, kHasV>() * kWave)) void prefill_prep_kernel(
    PrefillPrepParams p, int64_t rows) {
  constexpr int kGroup = kQueryHeads / kHeads;
  constexpr int kPer = kDim / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = wave_uniform(threadIdx.x / kWave);
  const int head = blockIdx.y;
  const int64_t row0 = (int64_t)blockIdx.x * kPrepRows;
  int32_t position[kPrepRows];
#pragma unroll
  for (int r = 0; r < kPrepRows; ++r)
    position[r] = row0 + r < rows ? wave_uniform(p.token_position[row0 + r]) : -1;
  float x[kPrepRows][kPer];
  // Loads the given tensor's head of every row of the block.
  auto load_rows = [&](const uint16_t *base, int heads_per_row, int h) {
#pragma unroll
    for (int r = 0; r < kPrepRows; ++r) {
      const int64_t rr = row0 + r < rows ? row0 + r : row0;
      load_head<kDim>(base + (rr * heads_per_row + h) * kDim, x[r], lane);
    }
  };
  if (wave < kGroup) {
    const int qh = head * kGroup + wave;
    load_rows(p.q, kQueryHeads, qh);
#pragma unroll
    for (int r = 0; r < kPrepRows; ++r) {
      if (position[r] < 0) continue;
      store_weighted_rope<kDim, kRotary>(
          p.q_prepared + ((row0 + r) * kQueryHeads + qh) * kDim, x[r], p.q_norm_weight,
          p.cos + (int64_t)position[r] * (kRotary / 2), p.sin + (int64_t)position[r] * (kRotary / 2),
          lane);
    }
    if (kHasV || wave != 0) return;
  }
  const bool k_wave = kHasV ? wave == kGroup : wave == 0;
  load_rows(k_wave ? p.k : p.v, kHeads, head);
#pragma unroll
  for (int r = 0; r < kPrepRows; ++r) {
    if (position[r] < 0) continue;
    const int64_t off = ((row0 + r) * kHeads + head) * kDim;
    if (k_wave) {
      store_weighted_rope<kDim, kRotary>(p.k_prepared + off, x[r], p.k_norm_weight,
                                         p.cos + (int64_t)position[r] * (kRotary / 2),
                                         p.sin + (int64_t)position[r] * (kRotary / 2), lane);
      if constexpr (!kHasV) store_scale_free<kDim>(p.v_prepared + off, x[r], lane);
    } else {
      store_scale_free<kDim>(p.v_prepared + off, x[r], lane);
    }
  }
}

// ---- 1x512 causal self-attention ---------------------------------------
constexpr int kD512 = 512;
constexpr int kD512Rows = 4;          // query rows (one per wave) per workgroup
constexpr int kD512Threads = kD512Rows * kWave;
constexpr int kD512Tile = 32;         // keys per LDS tile
constexpr int kD512RowBytes = kD512 * 2;
constexpr int kD512Chunks = kD512RowBytes / 16;  // 16-byte chunks per row
constexpr float kD512Slack = 8.0f;
constexpr int kD512VLead = 4;         // P.V MFMAs the V reads run ahead

struct D512Params {
  uint16_t *out;        // [B][L][16][512]
  const uint16_t *q;    // [B][L][16][512]
  const uint16_t *k;    // [B][L][1][512]
  const uint16_t *v;
  int32_t seq_len;
  float q_scale;        // softmax_scale * log2(e)
};

__device__ __forceinline__ f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

typedef unsigned u32x4v_t __attribute__((ext_vector_type(4)));

// The 16 K-fragment reads of one 16-key score block into AGPRs, all in
// flight before the first MFMA. For lane key k (k & 15 = lane & 15) and lane
// group g, k-step s sits at chunk (4s + g) ^ (k & 15) of the key's row: bits
// 0-1 of the chunk are g ^ (k & 3), bits 2-3 are (s & 3) ^ ((k >> 2) & 3)
// and bits 4+ are s >> 2. So with base = the address of k-step 0, k-step s
// is at (base ^ (64 (s & 3))) + 256 (s >> 2): four XORed addresses, four
// immediate offsets each. Issue position p = 4 (s & 3) + (s >> 2).
template <int kImm>
__device__ __forceinline__ void d512_read_kfrags(uint32_t k_addr, u32x4v_t (&kf)[16]) {
  uint32_t t0, t1;
  asm volatile(
      "s_waitcnt lgkmcnt(0)\n\t"
      "v_xor_b32 %[t0], 0, %[ka]\n\t"
      "ds_read_b128 %[f0], %[t0] offset:%[i0]\n\t"
      "ds_read_b128 %[f4], %[t0] offset:%[i1]\n\t"
      "ds_read_b128 %[f8], %[t0] offset:%[i2]\n\t"
      "ds_read_b128 %[f12], %[t0] offset:%[i3]\n\t"
      "v_xor_b32 %[t1], 64, %[ka]\n\t"
      "ds_read_b128 %[f1], %[t1] offset:%[i0]\n\t"
      "ds_read_b128 %[f5], %[t1] offset:%[i1]\n\t"
      "ds_read_b128 %[f9], %[t1] offset:%[i2]\n\t"
      "ds_read_b128 %[f13], %[t1] offset:%[i3]\n\t"
      "v_xor_b32 %[t0], 128, %[ka]\n\t"
      "ds_read_b128 %[f2], %[t0] offset:%[i0]\n\t"
      "ds_read_b128 %[f6], %[t0] offset:%[i1]\n\t"
      "ds_read_b128 %[f10], %[t0] offset:%[i2]\n\t"
      "ds_read_b128 %[f14], %[t0] offset:%[i3]\n\t"
      "v_xor_b32 %[t1], 192, %[ka]\n\t"
      "ds_read_b128 %[f3], %[t1] offset:%[i0]\n\t"
      "ds_read_b128 %[f7], %[t1] offset:%[i1]\n\t"
      "ds_read_b128 %[f11], %[t1] offset:%[i2]\n\t"
      "ds_read_b128 %[f15], %[t1] offset:%[i3]"
      : [t0] "=&v"(t0), [t1] "=&v"(t1),
        [f0] "=&a"(kf[0]), [f1] "=&a"(kf[1]), [f2] "=&a"(kf[2]), [f3] "=&a"(kf[3]), [f4]
        "=&a"(kf[4]), [f5] "=&a"(kf[5]), [f6] "=&a"(kf[6]), [f7] "=&a"(kf[7]), [f8]
        "=&a"(kf[8]), [f9] "=&a"(kf[9]), [f10] "=&a"(kf[10]), [f11] "=&a"(kf[11]), [f12]
        "=&a"(kf[12]), [f13] "=&a"(kf[13]), [f14] "=&a"(kf[14]), [f15] "=&a"(kf[15])
      : [ka] "v"(k_addr), [i0] "i"(kImm), [i1] "i"(kImm + 256), [i2] "i"(kImm + 512),
        [i3] "i"(kImm + 768));
}
// Issue position of k-step s in d512_read_kfrags.
constexpr int d512FragPos(int s) { return 4 * (s & 3) + (s >> 2); }
template <int kStep>
__device__ __forceinline__ void d512_kfrag_ready(u32x4v_t &f) {
  asm volatile("s_waitcnt lgkmcnt(%[n])" : "+a"(f) : [n] "i"(15 - d512FragPos(kStep)));
}
template <int kBegin, int kEnd, class F>
__device__ __forceinline__ void d512_static_for(F &&f) {
  if constexpr (kBegin < kEnd) {
    f(std::integral_constant<int, kBegin>{});
    d512_static_for<kBegin + 1, kEnd>(f);
  }
}

__global__ __launch_bounds__(kD512Threads, 1) void prefill_d512_kernel(D512Params p) {
  constexpr int KS = kD512 / 32;  // 32-dim k-steps of S^T
  constexpr int DB = kD512 / 16;  // 16-dim blocks of O^T
  // Two stages of K and V tiles (32 keys x 1 KiB each).
  struct Lds {
    uint4 k[2][kD512Tile * kD512Chunks];
    uint4 v[2][kD512Tile * kD512Chunks];
  };
  __shared__ __attribute__((aligned(1024))) Lds lds;

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = wave_uniform(t >> 6);
  const int head = lane & 15;   // MFMA column
  const int g = lane >> 4;      // lane group: keys / dims 4g..4g+3 of the accumulator
  const int b = blockIdx.y;
  const int L = p.seq_len;
  // Causal work grows with the row: the last rows are dispatched first, so
  // the workgroups of the first rows fill the CUs that free up early
  // (longest-first order; one workgroup per CU at a time).
  const int r0 = (gridDim.x - 1 - blockIdx.x) * kD512Rows;
  const int row = r0 + wave;
  const bool row_ok = row < L;
  const int last_key = min(r0 + kD512Rows, L) - 1;  // last key any row of the workgroup sees

  // Q^T operand: lane holds Q[row][head][32 s + 8 g .. +8] for k-step s.
  uint4 qreg[KS];
  {
    const uint16_t *qrow = p.q + (((int64_t)b * L + (row_ok ? row : 0)) * kQueryHeads + head) * kD512;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qreg[s] = row_ok ? load128(qrow + 32 * s + 8 * g) : make_uint4(0, 0, 0, 0);
    // Q lives in AGPRs (an MFMA operand may be an AGPR); all loads are
    // issued before the first constraint forces a wait.
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4v_t t4 = {qreg[s].x, qreg[s].y, qreg[s].z, qreg[s].w};
      asm volatile("" : "+a"(t4));
      qreg[s] = make_uint4(t4.x, t4.y, t4.z, t4.w);
    }
  }

  float m_run = -INFINITY, l_run = 0.0f;
  f32x4_t acc[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) acc[d] = f32x4_t{};

  const uint16_t *kseq = p.k + (int64_t)b * L * kD512;
  const uint16_t *vseq = p.v + (int64_t)b * L * kD512;
  const int n_tiles = last_key / kD512Tile + 1;
  // Copy of a tile into a stage: wave w copies keys 8w .. 8w+7, one 1 KiB
  // row per copy; lane l fills LDS chunk l with the swizzled source chunk.
  constexpr int kCopyRows = kD512Tile / (kD512Threads / kWave);
  auto copy_tile = [&](int kt, int stage) {
#pragma unroll
    for (int i = 0; i < kCopyRows; ++i) {
      const int key = kCopyRows * wave + i;
      const int64_t src_row = (int64_t)min(kt + key, L - 1) * kD512;  // past the end: masked
      const uint32_t dk = lds_address(&lds.k[stage][key * kD512Chunks]);
      const uint32_t dv = lds_address(&lds.v[stage][key * kD512Chunks]);
      copy_row_pair(reinterpret_cast<uint64_t>(kseq + src_row + 8 * (lane ^ (key & 15))),
                    wave_uniform(dk));
      copy_row_pair(reinterpret_cast<uint64_t>(vseq + src_row + 8 * (lane ^ ((key & 7) << 1))),
                    wave_uniform(dv));
    }
  };
  const int k15 = lane & 15;
  const uint32_t k_base = lds_address(&lds.k[0][0]) + k15 * kD512RowBytes +
                          16 * (g ^ (k15 & 3)) + 64 * ((k15 >> 2) & 3);
  constexpr int kStageBytes = kD512Tile * kD512RowBytes;
  copy_tile(0, 0);
  for (int tile = 0; tile < n_tiles; ++tile) {
    const int kt = tile * kD512Tile;
    const int stage = tile & 1;
    // Tile `tile` copied (each wave waits for its own copies, the barrier for
    // all); every wave is done with tile-1, so the other stage is free.
    wait_copies();
    __syncthreads();
    if (tile + 1 < n_tiles) copy_tile(kt + kD512Tile, stage ^ 1);
    if (!row_ok || kt > row) continue;  // uniform per wave
    const uint4 *s_v = lds.v[stage];

    // Scores of the two 16-key blocks: lane holds head `head`, keys
    // 16 blk + 4 g + i.
    f32x4_t sblk[2];
    auto score_block = [&](auto st, auto bl) __attribute__((always_inline)) {
      constexpr int kImm =
          decltype(st)::value * kStageBytes + decltype(bl)::value * 16 * kD512RowBytes;
      u32x4v_t kf[16];
      d512_read_kfrags<kImm>(k_base, kf);
      f32x4_t s2[2] = {f32x4_t{}, f32x4_t{}};
      d512_static_for<0, 16>([&](auto pc) __attribute__((always_inline)) {
        constexpr int pos = decltype(pc)::value;
        constexpr int s = 4 * (pos & 3) + (pos >> 2);  // k-step at issue position pos
        d512_kfrag_ready<s>(kf[s]);
        s2[pos & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8_t, kf[s]), __builtin_bit_cast(bf16x8_t, qreg[s]),
            s2[pos & 1], 0, 0, 0);
        // Keep each fragment's wait right before its MFMA: without this
        // fence the scheduler issued all sixteen waits first, one
        // lgkmcnt(0) in effect, and the reads no longer overlapped the
        // MFMAs.
        __builtin_amdgcn_sched_barrier(0);
      });
      return s2[0] + s2[1];
    };
    if (stage == 0) {
      sblk[0] = score_block(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
      sblk[1] = score_block(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{});
    } else {
      sblk[0] = score_block(std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{});
      sblk[1] = score_block(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
    }
    float sc[8];
    float tmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int kp = kt + 16 * (j / 4) + 4 * g + (j % 4);
      const float x = sblk[j / 4][j % 4];
      sc[j] = kp <= row ? x : -INFINITY;
      tmax = fmaxf(tmax, sc[j]);
    }
    tmax = xor_max<16>(tmax);
    tmax = xor_max<32>(tmax) * p.q_scale;
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + kD512Slack) != 0) {
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int d = 0; d < DB; ++d) acc[d] *= alpha;
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    uint32_t pw[4];
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      const float p0 = __builtin_amdgcn_exp2f(fmaf(sc[j], p.q_scale, -m_use));
      const float p1 = __builtin_amdgcn_exp2f(fmaf(sc[j + 1], p.q_scale, -m_use));
      l_run += p0 + p1;
      pw[j / 2] = pack_bf16x2(p0, p1);
    }
    const uint4 pb = make_uint4(pw[0], pw[1], pw[2], pw[3]);
    // V^T operand of dim block d: lane i of group g reads rows k0 + j,
    // dims 16 d + 4 q (j = (lane % 16) / 4, q = lane % 4) with k0 = 4 g
    // and 16 + 4 g.
    const int vj = (lane & 15) >> 2;
    const int vq = lane & 3;
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      uint2 half_op[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int vrow = 16 * r + 4 * g + vj;
        const int c = 2 * d + (vq >> 1);
        const char *addr = reinterpret_cast<const char *>(s_v) + vrow * kD512RowBytes +
                           ((c ^ ((vrow & 7) << 1)) << 4) + ((vq & 1) << 3);
        typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;
        const i16x4_t tr = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_i16x4 *)(__attribute__((address_space(3))) const char *)(addr));
        half_op[r] = __builtin_bit_cast(uint2, tr);
      }
      acc[d] = mfma16(make_uint4(half_op[0].x, half_op[0].y, half_op[1].x, half_op[1].y), pb,
                      acc[d]);
    }
    // Keep the transposing V reads kD512VLead MFMAs ahead of their MFMA
    // (measured: 2 ahead 171 us, 4 ahead 164 us, 6 ahead 164.7 us for the
    // 2048-row launcher).
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kD512VLead, 1);
#pragma unroll
    for (int i = 0; i < DB - kD512VLead; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // 1 MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);  // its successor's 2 reads
    }
    __builtin_amdgcn_sched_group_barrier(0x008, kD512VLead, 1);
  }

  wait_copies();  // no copy may still be writing LDS when the workgroup exits

  // Normalise and store: lane holds head `head`, dims 16 d + 4 g + i.
  l_run = xor_sum<16>(l_run);
  l_run = xor_sum<32>(l_run);
  if (!row_ok) return;
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  uint16_t *orow = p.out + (((int64_t)b * L + row) * kQueryHeads + head) * kD512;
#pragma unroll
  for (int d = 0; d < DB; ++d) {
    uint2 o;
    o.x = pack_bf16x2(acc[d][0] * inv, acc[d][1] * inv);
    o.y = pack_bf16x2(acc[d][2] * inv, acc[d][3] * inv);
    *reinterpret_cast<uint2 *>(orow + 16 * d + 4 * g) = o;
  }
}

bool prefill_args_ok(const void *out, const void *qp, const void *kp, const void *vp,
                     const void *q, const void *k, const void *position, int batch_size,
                     int seqlen_q, int seqlen_k) {
  // src/gemma4_flash_attention_prefill.cu:1131-1138, 1199-1205
  return batch_size > 0 && seqlen_q > 0 && seqlen_q == seqlen_k && out != nullptr &&
         qp != nullptr && kp != nullptr && vp != nullptr && q != nullptr && k != nullptr &&
         position != nullptr && (int64_t)batch_size * seqlen_q <= 0x7fffffff;
}

}  // namespace
}  // namespace gemma4

using namespace gemma4;

extern "C" hipError_t gemma4_flash_attention_sliding_fwd_bf16_norm_rope(
    gemma4_bf16 *d_out, gemma4_bf16 *d_q_prepared, gemma4_bf16 *d_k_prepared,
    gemma4_bf16 *d_v_prepared, const gemma4_bf16 *d_q, const gemma4_bf16 *d_k,
    const gemma4_bf16 *d_v, const gemma4_bf16 *d_q_norm_weight,
    const gemma4_bf16 *d_k_norm_weight, const float *d_cos, const float *d_sin,
    const int32_t *d_token_position, int batch_size, int seqlen_q, int seqlen_k, int window_size,
    float softmax_scale, hipStream_t stream) {
  if (!prefill_args_ok(d_out, d_q_prepared, d_k_prepared, d_v_prepared, d_q, d_k,
                       d_token_position, batch_size, seqlen_q, seqlen_k) ||
      window_size <= 0 || d_v == nullptr || d_q_norm_weight == nullptr ||
      d_k_norm_weight == nullptr || d_cos == nullptr || d_sin == nullptr) {
    return hipErrorInvalidValue;
  }
  PrefillPrepParams pp{};
  pp.q_prepared = reinterpret_cast<uint16_t *>(d_q_prepared);
  pp.k_prepared = reinterpret_cast<uint16_t *>(d_k_prepared);
  pp.v_prepared = reinterpret_cast<uint16_t *>(d_v_prepared);
  pp.q = reinterpret_cast<const uint16_t *>(d_q);
  pp.k = reinterpret_cast<const uint16_t *>(d_k);
  pp.v = reinterpret_cast<const uint16_t *>(d_v);
  pp.q_norm_weight = reinterpret_cast<const uint16_t *>(d_q_norm_weight);
  pp.k_norm_weight = reinterpret_cast<const uint16_t *>(d_k_norm_weight);
  pp.cos = d_cos;
  pp.sin = d_sin;
  pp.token_position = d_token_position;
  // 8x256 geometry: RoPE over the whole head, V projection present.
  const int64_t rows = (int64_t)batch_size * seqlen_q;
  hipLaunchKernelGGL((prefill_prep_kernel<8, 256, 256, true>),
                     dim3((rows + kPrepRows - 1) / kPrepRows, 8),
                     dim3(prep_waves<8, true>() * kWave), 0, stream, pp, rows);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  // Attention over the prepared rows: the chunk kernel without a prior
  // context (only num_heads, head_dim and window_size of the config are read).
  Gemma4KvCacheConfig c{};
  c.num_layers = 1;
  c.num_heads = 8;
  c.head_dim = 256;
  c.window_size = window_size;
  return gemma4_flash_attention_prefill_chunk_paged_bf16(
      d_out, d_q_prepared, d_k_prepared, d_v_prepared, nullptr, nullptr, nullptr, nullptr, c, 0,
      batch_size, seqlen_q, softmax_scale, stream);
}

extern "C" hipError_t gemma4_flash_attention_global_fwd_bf16_norm_rope(
    gemma4_bf16 *d_out, gemma4_bf16 *d_q_prepared, gemma4_bf16 *d_k_prepared,
    gemma4_bf16 *d_v_prepared, const gemma4_bf16 *d_q, const gemma4_bf16 *d_k,
    const gemma4_bf16 *d_q_norm_weight, const gemma4_bf16 *d_k_norm_weight, const float *d_cos,
    const float *d_sin, const int32_t *d_token_position, int batch_size, int seqlen_q,
    int seqlen_k, float softmax_scale, hipStream_t stream) {
  if (!prefill_args_ok(d_out, d_q_prepared, d_k_prepared, d_v_prepared, d_q, d_k,
                       d_token_position, batch_size, seqlen_q, seqlen_k) ||
      d_q_norm_weight == nullptr || d_k_norm_weight == nullptr || d_cos == nullptr ||
      d_sin == nullptr || batch_size > 65535 || !(softmax_scale > 0.0f)) {
    return hipErrorInvalidValue;
  }
  PrefillPrepParams pp{};
  pp.q_prepared = reinterpret_cast<uint16_t *>(d_q_prepared);
  pp.k_prepared = reinterpret_cast<uint16_t *>(d_k_prepared);
  pp.v_prepared = reinterpret_cast<uint16_t *>(d_v_prepared);
  pp.q = reinterpret_cast<const uint16_t *>(d_q);
  pp.k = reinterpret_cast<const uint16_t *>(d_k);
  pp.v = nullptr;
  pp.q_norm_weight = reinterpret_cast<const uint16_t *>(d_q_norm_weight);
  pp.k_norm_weight = reinterpret_cast<const uint16_t *>(d_k_norm_weight);
  pp.cos = d_cos;
  pp.sin = d_sin;
  pp.token_position = d_token_position;
  // 1x512 geometry: RoPE over a quarter of the head, V from the raw K.
  const int64_t rows = (int64_t)batch_size * seqlen_q;
  hipLaunchKernelGGL((prefill_prep_kernel<1, 512, 128, false>),
                     dim3((rows + kPrepRows - 1) / kPrepRows, 1),
                     dim3(prep_waves<1, false>() * kWave), 0, stream, pp, rows);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  D512Params ap{};
  ap.out = reinterpret_cast<uint16_t *>(d_out);
  ap.q = reinterpret_cast<const uint16_t *>(d_q_prepared);
  ap.k = reinterpret_cast<const uint16_t *>(d_k_prepared);
  ap.v = reinterpret_cast<const uint16_t *>(d_v_prepared);
  ap.seq_len = seqlen_q;
  ap.q_scale = softmax_scale * kLog2e;
  hipLaunchKernelGGL(prefill_d512_kernel,
                     dim3((seqlen_q + kD512Rows - 1) / kD512Rows, batch_size),
                     dim3(kD512Threads), 0, stream, ap);
  return hipGetLastError();
}
