// Attention output projection + post-attention RMSNorm + residual (gfx950).
// Follows project_attention_out_post_attention
// (src/gemma4_flash_attention_decode.cu:34-129): a GEMV of the attention row
// (16 query heads x head_dim) against the column-major O weights
// ([3840][width]), the learned RMSNorm of the bf16 result
// (src/gemma4_rmsnorm.cu:28-85) and the residual add
// (src/gemma4_cuda_utils.cuh:105-122).
//
// The weights (31.5 MiB for width 4096, 63 MiB for 8192) are read once per
// launch; that stream is the roofline (HBM). A few rows run on v_dot2, more
// on bf16 MFMA (exact products, fp32 sums), so a batch of decode rows costs
// little more than one row. The norm needs the whole 3840-wide row, so a second small kernel
// (one workgroup per row) applies it and the residual add.
#include "gemma4_attention_output.h"
#include "gemma4_device.hpp"
#include "prep_common.hpp"

namespace gemma4 {
namespace {

constexpr int kHidden = GEMMA4_ATTENTION_OUTPUT_HIDDEN;
constexpr int kNormThreads = 512;
constexpr int kHiddenPacks = kHidden / kPackElems;  // 480
static_assert(kHiddenPacks <= kNormThreads, "one pack per norm thread");

// Few rows (below kMfmaRows): v_dot2 GEMV. A wave owns kCols hidden columns
// and holds all of their weights in registers (32 16-byte packs per lane,
// each load instruction reading 1 KiB of one column's contiguous weights),
// then runs each row against them: lane l dots packs l, l + 64, ... (exact
// bf16 products, one rounding per pair) and a wave sum finishes each column.
constexpr int kRowWaves = 4;

template <int kWidth>
struct RowShape {
  static constexpr int kPacks = kWidth / (kPackElems * kWave);  // per lane per column
  static constexpr int kCols = 32 / kPacks;                     // 32 packs in flight per lane
  static constexpr int kColsPerGroup = kCols * kRowWaves;
  static constexpr int kGroups = kHidden / kColsPerGroup;
  static_assert(kWidth % (kPackElems * kWave) == 0 && 32 % kPacks == 0, "width");
  static_assert(kHidden % kColsPerGroup == 0, "whole column groups");
};

template <int kWidth>
__global__ __launch_bounds__(kRowWaves *kWave) void o_projection_rows_kernel(
    const uint16_t *__restrict__ attn, const uint16_t *__restrict__ w,
    uint16_t *__restrict__ residual, int32_t rows) {
  using S = RowShape<kWidth>;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = wave_uniform(threadIdx.x / kWave);
  const int col0 = (blockIdx.x * kRowWaves + wave) * S::kCols;
  uint4 wp[S::kCols][S::kPacks];
#pragma unroll
  for (int c = 0; c < S::kCols; ++c)
#pragma unroll
    for (int i = 0; i < S::kPacks; ++i)
      wp[c][i] = load128_stream(w + (int64_t)(col0 + c) * kWidth + (i * kWave + lane) * kPackElems);
  for (int32_t r = 0; r < rows; ++r) {
    const uint16_t *a = attn + (int64_t)r * kWidth;
    uint4 ap[S::kPacks];
#pragma unroll
    for (int i = 0; i < S::kPacks; ++i) ap[i] = load128(a + (i * kWave + lane) * kPackElems);
    float sum[S::kCols];
#pragma unroll
    for (int c = 0; c < S::kCols; ++c) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < S::kPacks; ++i) {
        s = dot2_bf16(ap[i].x, wp[c][i].x, s);
        s = dot2_bf16(ap[i].y, wp[c][i].y, s);
        s = dot2_bf16(ap[i].z, wp[c][i].z, s);
        s = dot2_bf16(ap[i].w, wp[c][i].w, s);
      }
      sum[c] = wave_sum(s);
    }
    if (lane == 0) {
      uint16_t *out = residual + (int64_t)r * kHidden + col0;
      if constexpr (S::kCols == 4) {
        *reinterpret_cast<uint2 *>(out) =
            make_uint2(pack_bf16x2(sum[0], sum[1]), pack_bf16x2(sum[2], sum[3]));
      } else {
        *reinterpret_cast<uint32_t *>(out) = pack_bf16x2(sum[0], sum[1]);
      }
    }
  }
}

// kMfmaRows rows and more: D[row][col] = sum_k attn[row][k] * W[col][k] on
// v_mfma_f32_16x16x32_bf16. A workgroup owns 16 hidden columns; its kSplit =
// 8 waves split k into slices of width / 8 (16 or 32 MFMA steps each). In a
// step lane l supplies A = attn[row block + l % 16][k0 + 8 (l / 16) ..] and
// B = W[col0 + l % 16][k0 + 8 (l / 16) ..], each one 16-byte pack (W's
// column-major rows make B a contiguous read), and the 16x16 fp32 result
// holds column l % 16, rows 4 (l / 16) + 0..3. Each weight pack is loaded
// once and used for up to kBlocks row blocks of 16; partial sums of the k
// slices meet in LDS. 240 workgroups of 8 waves.
constexpr int kColsPerGroup = 16;
constexpr int kSplit = 8;  // waves per workgroup, one k slice each
constexpr int kGroups = kHidden / kColsPerGroup;
constexpr int kMaxBlocks = 4;  // row blocks per pass (64 rows)
// From this many rows on the MFMA kernel is faster (measured crossover: at
// one row the dot2 kernel's 1 KiB-contiguous weight reads win; at eight the
// dot2 kernel's VALU work has caught up with the weight stream).
constexpr int kMfmaRows = 8;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

template <int kWidth, int kBlocks>
__global__ __launch_bounds__(kSplit *kWave) void o_projection_kernel(
    const uint16_t *__restrict__ attn, const uint16_t *__restrict__ w,
    uint16_t *__restrict__ residual, int32_t rows) {
  constexpr int kSliceK = kWidth / kSplit;
  constexpr int kSteps = kSliceK / 32;
  __shared__ f32x4_t partial[kSplit][kBlocks][kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = wave_uniform(threadIdx.x / kWave);
  const int col0 = blockIdx.x * kColsPerGroup;
  const int k0 = wave * kSliceK + 8 * (lane / 16);
  const uint16_t *wl = w + (int64_t)(col0 + lane % 16) * kWidth + k0;
  uint4 wp[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s) wp[s] = load128_stream(wl + 32 * s);
  for (int32_t row0 = 0; row0 < rows; row0 += 16 * kBlocks) {
    f32x4_t acc[kBlocks];
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) {
      acc[b] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      const int32_t row = row0 + 16 * b + lane % 16;
      const bool live = row < rows;
      const uint16_t *al = attn + (int64_t)(live ? row : 0) * kWidth + k0;
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
        uint4 ap = load128(al + 32 * s);
        if (!live) ap = make_uint4(0, 0, 0, 0);
        acc[b] = mfma16(ap, wp[s], acc[b]);
      }
    }
#pragma unroll
    for (int b = 0; b < kBlocks; ++b) partial[wave][b][lane] = acc[b];
    __syncthreads();
    if (threadIdx.x < kBlocks * kWave) {
      const int b = threadIdx.x / kWave;
      f32x4_t sum = partial[0][b][lane];
#pragma unroll
      for (int k = 1; k < kSplit; ++k) sum += partial[k][b][lane];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int32_t row = row0 + 16 * b + 4 * (lane / 16) + i;
        if (row < rows)
          residual[(int64_t)row * kHidden + col0 + lane % 16] =
              (uint16_t)f32_to_bf16_bits(sum[i]);
      }
    }
    __syncthreads();
  }
}

// One workgroup per row: thread t < 480 owns pack t of the hidden row.
__global__ __launch_bounds__(kNormThreads) void post_attention_norm_kernel(
    const uint16_t *__restrict__ residual, const uint16_t *__restrict__ weight,
    const uint16_t *__restrict__ x, uint16_t *__restrict__ normed, uint16_t *__restrict__ ffn) {
  __shared__ float wave_sums[kNormThreads / kWave];
  const int t = threadIdx.x;
  const int64_t off = (int64_t)blockIdx.x * kHidden + t * kPackElems;
  const bool owner = t < kHiddenPacks;
  float v[kPackElems] = {};
  if (owner) unpack8(load128(residual + off), v);
  float sq = 0.0f;
#pragma unroll
  for (int i = 0; i < kPackElems; ++i) sq = fmaf(v[i], v[i], sq);
  sq = wave_sum(sq);
  if ((t & (kWave - 1)) == 0) wave_sums[t / kWave] = sq;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kNormThreads / kWave; ++i) total += wave_sums[i];
  if (!owner) return;
  const float scale = 1.0f / sqrtf(total / (float)kHidden + kRmsEps);
  float g[kPackElems], xi[kPackElems];
  unpack8(load128(weight + t * kPackElems), g);
  unpack8(load128(x + off), xi);
  float n[kPackElems], f[kPackElems];
#pragma unroll
  for (int i = 0; i < kPackElems; ++i) {
    n[i] = v[i] * scale * g[i];
    // The residual adds the bf16-rounded normed value.
    n[i] = __uint_as_float(f32_to_bf16_bits(n[i]) << 16);
    f[i] = xi[i] + n[i];
  }
  store128(normed + off, make_uint4(pack_bf16x2(n[0], n[1]), pack_bf16x2(n[2], n[3]),
                                    pack_bf16x2(n[4], n[5]), pack_bf16x2(n[6], n[7])));
  store128(ffn + off, make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]),
                                 pack_bf16x2(f[4], f[5]), pack_bf16x2(f[6], f[7])));
}

template <int kWidth, int kBlocks>
hipError_t launch_projection_blocks(const uint16_t *attn, const uint16_t *w, uint16_t *residual,
                                    int32_t rows, hipStream_t stream) {
  hipLaunchKernelGGL((o_projection_kernel<kWidth, kBlocks>), dim3(kGroups),
                     dim3(kSplit * kWave), 0, stream, attn, w, residual, rows);
  return hipGetLastError();
}

// Row blocks per pass: as many as the rows need, up to kMaxBlocks (more rows
// take several passes over the weights held in registers).
template <int kWidth>
hipError_t launch_projection(const uint16_t *attn, const uint16_t *w, uint16_t *residual,
                             int32_t rows, hipStream_t stream) {
  if (rows < kMfmaRows) {
    using S = RowShape<kWidth>;
    hipLaunchKernelGGL(o_projection_rows_kernel<kWidth>, dim3(S::kGroups), dim3(kRowWaves * kWave),
                       0, stream, attn, w, residual, rows);
    return hipGetLastError();
  }
  if (rows <= 16) return launch_projection_blocks<kWidth, 1>(attn, w, residual, rows, stream);
  if (rows <= 32) return launch_projection_blocks<kWidth, 2>(attn, w, residual, rows, stream);
  return launch_projection_blocks<kWidth, kMaxBlocks>(attn, w, residual, rows, stream);
}

}  // namespace
}  // namespace gemma4

extern "C" hipError_t gemma4_attention_o_projection_post_norm_bf16(
    gemma4_bf16 *residual_out, gemma4_bf16 *normed_out, gemma4_bf16 *ffn_residual,
    const gemma4_bf16 *attention_out, const gemma4_bf16 *o_proj_col_major,
    const gemma4_bf16 *post_norm_weight, const gemma4_bf16 *attention_x, int32_t rows,
    int32_t attention_width, hipStream_t stream) {
  using namespace gemma4;
  if (residual_out == nullptr || normed_out == nullptr || ffn_residual == nullptr ||
      attention_out == nullptr || o_proj_col_major == nullptr || post_norm_weight == nullptr ||
      attention_x == nullptr || rows < 0 || (attention_width != 4096 && attention_width != 8192)) {
    return hipErrorInvalidValue;
  }
  if (rows == 0) return hipSuccess;
  auto *res = reinterpret_cast<uint16_t *>(residual_out);
  const auto *attn = reinterpret_cast<const uint16_t *>(attention_out);
  const auto *w = reinterpret_cast<const uint16_t *>(o_proj_col_major);
  const hipError_t e = attention_width == 4096 ? launch_projection<4096>(attn, w, res, rows, stream)
                                               : launch_projection<8192>(attn, w, res, rows, stream);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(post_attention_norm_kernel, dim3(rows), dim3(kNormThreads), 0, stream, res,
                     reinterpret_cast<const uint16_t *>(post_norm_weight),
                     reinterpret_cast<const uint16_t *>(attention_x),
                     reinterpret_cast<uint16_t *>(normed_out),
                     reinterpret_cast<uint16_t *>(ffn_residual));
  return hipGetLastError();
}
