// Persistent decode step for gfx950: one launch of one workgroup per CU walks
// a run of consecutive model layers, and for each layer appends the current token's
// K/V and runs split-K GQA decode attention with its log-sum-exp combine.
// Replaces the per-layer launches of the reference decode loop
// (src/gemma4_decode_megakernel.cu:172-183 calling
// gemma4_decode_megakernel_flash_attention_layer_bf16, whose append and
// attention phases are src/gemma4_flash_attention_decode.cu:979-1067, with
// grid.sync() between them).
//
// Layer order is a real data dependence: layer i's q and new K/V rows are
// read only after every attention output row of layer i-1 has been
// published, exactly as if layer i's projections consumed layer i-1's
// output. What may run early is what does not depend on the previous layer:
// the page-table lookups and the first K/V tiles of layer i (cache rows of
// older tokens) are loaded into registers while layer i-1 is still being
// combined, so the per-layer critical path is flag → q → math on resident
// tiles → partial → combine → flag, and HBM streaming of the next layer
// overlaps it.
//
// Decomposition (8 KV heads x 256 dims, 16 query heads, GQA group 2)
//   One workgroup per CU (256), placed by the hardware round-robin over the
//   8 XCDs. Each workgroup reads its XCD id and takes a ticket t (0..31)
//   from that XCD's counter; the workgroups of XCD x serve KV head x of
//   every sequence: sequence b = t % batch, split s = t / batch, with
//   splits = 32 / batch per (sequence, head) "unit". All splits of a unit
//   therefore share one L2, and their partials are exchanged through it.
//   compute waves 0..7: 8-key tiles t = wave, wave+8, ... of the split
//   control wave 8:     waits for the previous layer, stages the layer's q
//                       and appended K/V rows in LDS, then combines the
//                       unit's splits for its own 8-dim output chunks
//                       (c = s, s + splits, ...) and signals
//   prefetch wave 9:    DMAs the next global layer's tiles 16..31 of the
//                       split into LDS (global_load_lds), a few per barrier
//                       interval over the 4 layers before it
// A tile is 8 keys x 256 dims of K and V: lane (r, c) loads the 16-byte pack
// c of key rows 4r..4r+3 (rows 0-3 for lanes 0-31, 4-7 for lanes 32-63).
// Compute waves wait only for their own tile loads (q and the appended rows
// come through LDS), so tiles prefetched long ahead never hold them up.
//
// Exchange between workgroups
//   * split records (XCD-local): per (unit, split), 32 chunks of 8 output
//     dims holding acc[8], m, l for each head of the pair, written with
//     ordinary stores (they reach the XCD's L2) and read with sc0|nt loads,
//     which skip the L1 and are served from the L2 the writer shares.
//     Empty dwords hold a signalling-NaN sentinel that arithmetic never
//     produces, so readers poll the data itself; the one reader of a chunk
//     empties it again before it signals the layer complete.
//   * layer completion: each workgroup stores its output chunks
//     device-coherently, waits for them, then sets its XCD-local flag; the
//     XCD's ticket-0 workgroup collects the 32 local flags and sets the XCD's
//     device-coherent flag. Ticket 0 polls all 8 XCD flags and then raises
//     the XCD's go flag in its L2; the other 31 workgroups poll that (an L2
//     round trip, so they start the next layer together) before reading the
//     next layer's q. Flags hold the launch epoch
//     (1 + the value the previous launch left in the workspace header), so
//     they never need clearing.
// The XCD mapping needs exactly 32 workgroups per XCD, one per CU;
// workspace initialisation checks that once by a probe launch of this kernel
// and otherwise reports the entry point unsupported.
// Every wait is bounded by the real-time clock. The steps are ordinary
// launches that rely on all 256 workgroups being resident together (each
// takes a whole CU's LDS), which holds while no other kernel occupies CUs.
// If a wait gives up, the wave stops waiting, writes zeros for the output
// chunks it owns from that layer on, and records the error code and the
// launch's epoch in the workspace header. The error is sticky: every later
// launch on the workspace sees it at entry, writes zeros to all its outputs,
// touches no cache and exits, until the workspace is initialised again.
#include "gemma4_device.hpp"
#include "decode_common.hpp"
#include "prep_common.hpp"

#include "gemma4_flash_attention.h"

#include <math.h>

#include <atomic>


namespace gemma4 {
namespace {

// Model layer cadence (src/gemma4.h:105-108): every 6th layer and the last
// one are global.
constexpr int32_t kNumModelLayers = 48;
constexpr int32_t kGlobalPeriod = 6;
constexpr int kSHeads = 8, kSDim = 256, kSGroup = 2;
// Eight compute waves, two per SIMD (163 VGPRs each, three waves on two of
// the SIMDs with the control and prefetch waves): 382 against 392 us per
// config-2 step with four, mostly from the global layers' tile compute.
constexpr int kComputeWaves = 8;
constexpr int kControlWave = kComputeWaves;      // wave 8
constexpr int kPrefetchWave = kComputeWaves + 1; // wave 9
constexpr int kStepThreads = (kComputeWaves + 2) * kWave;
constexpr int kStepWorkgroups = 256;  // one workgroup per CU
constexpr int kLPR = kSDim / kPackElems;      // 32 lanes per key row
constexpr int kTileLoads = 4;                 // rows per lane per tile
constexpr int kTileKeys = 2 * kTileLoads;     // 8 keys per tile
constexpr int kNP = kTileLoads * kSGroup;     // partial dots per lane
constexpr int kSBits = 2;                     // log2(kLPR / kNP)
constexpr int kWaveKeys = 128;                // row-table entries per wave
constexpr int kMaxSplitKeys = kComputeWaves * kWaveKeys;
constexpr int kRowElems = kSHeads * kSDim;
// A split record is 32 chunks of 8 dims; a chunk holds, per head g of the
// pair, acc[8] then (m, l) and 2 pad floats, so the reader of one chunk
// finds everything it needs (and empties) in 96 contiguous bytes.
constexpr int kChunks = kSDim / kPackElems;
constexpr int kHalfChunk = kPackElems + 4;
constexpr int kChunkFloats = 2 * kHalfChunk;
constexpr int kRecordFloats = kChunks * kChunkFloats;
constexpr int kXcds = 8;                      // XCDs of an MI355X
constexpr int kXcdSlots = 32;                 // workgroups (CUs) per XCD
constexpr int kMaxBatch = 8;                  // at least 4 splits per unit
constexpr int32_t kMaxWalkSteps = 0xffff;     // iterations of one walk (flag stamps)
constexpr uint32_t kSentinel = 0x7fa5a5a5u;   // signalling NaN
constexpr int kHeaderInts = 64;               // epoch, error, ..., pad
// Header words: launch epoch; error code (0 ok, 1 a wait gave up, 2 a split
// longer than the row tables); the epoch of the launch that set the error;
// and a fault-injection hook for tests (stall layer + 1, its wait limit in
// ticks, and a word the host never sets).
constexpr int kHeaderEpoch = 0, kHeaderError = 1, kHeaderErrorEpoch = 2;
constexpr int kHeaderStallLayer = 3, kHeaderStallTicks = 4, kHeaderNeverSet = 5;
constexpr int kTicketStride = 32;             // ints between the XCD ticket counters
constexpr int kGlobalFlagStride = 16;         // ints per layer: one flag per XCD
constexpr uint64_t kWaitTicks = 100ull * 1000 * 1000 / 5;  // 0.2 s at 100 MHz
constexpr int kPrefetchTiles = 16 / kComputeWaves;  // register tile buffers per wave
// Global-layer tiles staged in LDS ahead of time by the prefetch wave: the
// split's tiles 16..31 (after the 16 held in compute-wave registers, two
// per wave). 16 x 8 KiB = 128 KiB of dynamic LDS (with the 29 KiB of static
// arrays, all of a CU's 160 KiB), which also keeps the hardware to one
// workgroup per CU.
constexpr int kLdsSlots = 16;
constexpr int kRegTiles = kComputeWaves * kPrefetchTiles;  // tiles 0..15 of a split: registers
constexpr int kLdsLead = 4;                    // layers of lead for the LDS prefetch
constexpr int kSlotsPerInterval = 2;           // slots requested between two barriers
constexpr size_t kPadLds = (size_t)kLdsSlots * 2 * kTileLoads * kWave * 16;

struct StepParams {
  uint16_t *out;
  const uint16_t *q;
  const uint16_t *new_k;
  const uint16_t *new_v;
  uint16_t *cache_k[2];  // [0] sliding, [1] global
  uint16_t *cache_v[2];
  const int32_t *page_table[2];
  Gemma4KvCacheConfig c[2];
  const int32_t *seq_lengths;
  const int32_t *token_position;
  // Optional preparation of the layers' raw projections (all null: q/k/v
  // are already prepared): learned RMSNorm weights per launch layer
  // [layer_count][256] for Q and K, and RoPE tables [position][128] per cache
  // kind ([0] sliding, [1] global).
  const uint16_t *q_norm_w;
  const uint16_t *k_norm_w;
  const float *rope_cos[2];
  const float *rope_sin[2];
  int32_t *header;
  uint32_t *tickets;      // [xcd * kTicketStride]
  int32_t *local_flags;   // [layer][xcd][slot]
  int32_t *global_flags;  // [layer][kGlobalFlagStride]
  int32_t *go_flags;      // [layer][xcd][16]: XCD-local copy of "layer complete"
  float *records;
  int32_t *probe;         // non-null: only report each workgroup's XCD id
  uint64_t *trace;        // STEP_TRACE builds: [workgroup][layer][10] real-time stamps
  int32_t batch;
  int32_t first_layer;
  int32_t layer_count;
  int32_t walk_layer;     // walks: the cache layer every iteration uses
  int32_t units;
  int32_t splits;
  float q_scale;
};

__device__ __forceinline__ bool model_layer_global(int32_t layer) {
  return layer == kNumModelLayers - 1 || (layer + 1) % kGlobalPeriod == 0;
}
// Index of `layer` among the cache layers of its own kind.
__device__ __forceinline__ int32_t cache_layer_of(int32_t layer) {
  const bool global = model_layer_global(layer);
  int32_t index = 0;
  for (int32_t l = 0; l < layer; ++l) index += model_layer_global(l) == global ? 1 : 0;
  return index;
}

// Workgroup barrier of the step kernel. The step's barriers order LDS traffic only: each wave's LDS operations
// complete, then s_barrier (inline asm, so the compiler adds no wait for
// vector memory operations). Tile loads and LDS DMA stay in flight across
// it; global-memory ordering the step needs is explicit (the prefetch
// wave's DMA wait before a global layer, the control wave's store wait
// before its flag, a walk's append wait). With __syncthreads every wave
// first waited for all of its outstanding loads: 383.4-383.8 against
// 376.5 us per config-2 step. Walks keep __syncthreads (4.44 against 4.54
// us per step).
template <bool kLdsOnly>
__device__ __forceinline__ void step_barrier() {
  if constexpr (kLdsOnly) {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  } else {
    __syncthreads();
  }
}

__device__ __forceinline__ uint64_t now_ticks() { return __builtin_amdgcn_s_memrealtime(); }

// Development builds only (-DSTEP_TRACE=1): real-time stamps of the layer
// phases, [workgroup (xcd * 32 + ticket)][layer][10], in the workspace.
#ifndef STEP_TRACE
#define STEP_TRACE 0
#endif
#if STEP_TRACE
#define STEP_MARK(e)                                                                     \
  do {                                                                                   \
    if (lane == 0 && (wave == kControlWave || wave == 0) && i < kNumModelLayers)        \
      p.trace[((int64_t)(xcd * kXcdSlots + ticket) * kNumModelLayers + i) * 10 + (e)] = \
          now_ticks();                                                                   \
  } while (0)
#else
#define STEP_MARK(e) \
  do {               \
  } while (0)
#endif

// Development builds only (-DSTEP_FLOOR=n): the same launch with parts of
// the work taken out, to price the per-layer handoffs on their own.
//   1: no K/V bytes -- no cache tiles, no LDS DMA, no appended row; every
//      exchange stays (q read, split records, combine, output rows, flags)
//   2: also no split records, combine or output rows: per layer only the q
//      read and the device-wide completion handoff
//   3: the device-wide handoff alone
//   4: the math on register contents, no K/V loads or LDS DMA
//   5: the K/V loads and DMA, no math (each tile only waited for)
//   6: every XCD's global-layer reads go to KV head 0's columns (results
//      wrong; prices eight XCDs streaming the same bytes)
#ifndef STEP_FLOOR
#define STEP_FLOOR 0
#endif
constexpr int kFloor = STEP_FLOOR;


// Id of the XCD (and so of the L2) this wave runs on.
__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v;
}
// The CU this wave runs on within its XCD: HW_ID bits 8..15 (CU id, SH id,
// SE id).
__device__ __forceinline__ uint32_t hw_cu_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(v));
  return (v >> 8) & 0xff;
}
// Reads of data another workgroup of the same XCD wrote with ordinary
// stores. sc0|nt loads skip the CU's L1 (an sc0 load alone can still hit a
// stale L1 line) and are served by the XCD's L2, clean or dirty, so a poll
// costs an L2 round trip; device-scope (sc1) loads would go to memory for
// every line the L2 holds clean.
constexpr int kLocalLoadAux = 1 | 2;

__device__ __forceinline__ int32_t coherent_load_i32(const int32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void coherent_store_i32(int32_t *p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
using u32x2 = __attribute__((ext_vector_type(2))) unsigned;
// Device-coherent buffer accesses at a per-lane byte offset from a
// wave-uniform base (a per-lane base would force a loop over lanes).
using BufferRsrc = decltype(__builtin_amdgcn_make_buffer_rsrc((void *)nullptr, 0, 0, 0));
__device__ __forceinline__ BufferRsrc buffer_of(const void *base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0,
                                           (int32_t)min<int64_t>(bytes, 0x7fffffff), 0x00020000);
}
// Ordinary store: written through the CU's L1 into the XCD's L2, where the
// other workgroups of the XCD read it.
__device__ __forceinline__ void local_store2(BufferRsrc r, int32_t off, float a, float b) {
  const u32x2 v = {__float_as_uint(a), __float_as_uint(b)};
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 0);
}

// Preparation of one 256-dim row held by a 32-lane half, lane c owning dims
// [8c, 8c + 8): RMSNorm, then (weighted) the learned weight and split-half
// RoPE over all 256 dims with the position's cos/sin row (c's dims and their
// partners, 16 lanes away, share the table entries [8c mod 128, +8)).
// The per-layer preparation's arithmetic with its own reduction order for
// the sum of squares (src/gemma4_flash_attention_decode.cu:233-283).
__device__ __forceinline__ uint4 prep_row(uint4 raw, uint4 weight, bool weighted,
                                          const float (&cs)[kPackElems],
                                          const float (&sn)[kPackElems], int c) {
  float x[8];
  unpack8(raw, x);
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss = fmaf(x[j], x[j], ss);
  // Sum over the row's 32 lanes, all exchanges on the VALU (DPP row ops and
  // a 16-lane row swap).
  ss += lane_pair<1>(ss);
  ss += lane_pair<2>(ss);
  ss += lane_pair<4>(ss);
  ss += lane_pair<8>(ss);
  ss = xor_sum<16>(ss);
  const float scale = 1.0f / sqrtf(ss / (float)kSDim + kRmsEps);
  float w[8];
  unpack8(weight, w);
  float y[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = weighted ? x[j] * scale * w[j] : x[j] * scale;
  float partner[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) partner[j] = xor_lane16(y[j]);
  const float sign = c < 16 ? -1.0f : 1.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = weighted ? fmaf(sign * partner[j], sn[j], y[j] * cs[j]) : y[j];
  // Round to bf16 (nearest even) with the hardware pair conversion.
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x2_t pr = {(__bf16)y[2 * j], (__bf16)y[2 * j + 1]};
    o[j] = __builtin_bit_cast(uint32_t, pr);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// Everything a compute wave needs about one layer of its split.
// All fields are wave-uniform.
struct LayerView {
  int32_t kind;           // 0 sliding cache, 1 global cache
  int32_t new_row;        // cache row this wave appends the new token to, or -1
  int32_t n_tiles;        // tiles of this wave
  bool owner;             // this wave attends over the new token
  int32_t new_j;          // owner: wave-local tile of the new token (else -1)
  int32_t new_r, new_kl;  // owner: its row half and load index in that tile
  bool lds;               // tiles 16 .. 16 + kLdsSlots - 1 of the split are in LDS
  int par;                // row table: s_rows[par]
};

// kWalk = false: iteration i is model layer first_layer + i of one decode
// step (the sliding or global cache by the model's layer cadence).
// kWalk = true: iteration i is decode step i of one layer (cache layer
// walk_layer of cache 0): the sequences' lengths grow by one per iteration
// and each iteration appends its token before attending, so later
// iterations read rows that other workgroups appended in this launch.
template <bool kWalk>
__global__ __launch_bounds__(kStepThreads) void decode_step_kernel(StepParams p) {
  __shared__ int4 s_rows[2][kComputeWaves][kWaveKeys / 4];  // [layer parity][wave]
  __shared__ float s_prob[kComputeWaves][kWave];
  __shared__ float s_ml[kComputeWaves][kSGroup][2];
  __shared__ float s_acc[kComputeWaves][kSGroup][kSDim];
  __shared__ uint4 s_q[kWave];    // q rows of the unit: [g][pack]
  __shared__ uint4 s_new[kWave];  // appended rows of the unit: [K pack | V pack]
  __shared__ int32_t s_ticket;
  __shared__ int32_t s_failed, s_epoch, s_stall_layer, s_stall_ticks;
  __shared__ int4 s_lds_rows[kLdsSlots * kTileKeys / 4];  // cache rows of the LDS tiles
  extern __shared__ uint4 s_tiles[];  // [slot][K 0..3 | V 0..3][lane]

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = wave_uniform(threadIdx.x / kWave);
  const int32_t xcd = (int32_t)(xcc_id() & 0xf);
  if (p.probe != nullptr) {
    // XCD id and the CU's place in it (HW_ID bits 8..15: CU, SH, SE).
    if (threadIdx.x == 0) p.probe[blockIdx.x] = xcd | (int32_t)(hw_cu_id() << 8);
    return;
  }
  if (threadIdx.x == kControlWave * kWave) {
    // Tickets count up forever; every launch takes exactly 32 per XCD.
    s_ticket = (int32_t)(__hip_atomic_fetch_add(p.tickets + xcd * kTicketStride, 1u,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) %
                         kXcdSlots);
    // Header words 0..7 in one device-coherent load. A failed earlier
    // launch (error recorded under another epoch) turns this launch into a
    // no-op that writes zeros.
    const BufferRsrc hdr = buffer_of(p.header, 32);
    const u32x4 h0 = __builtin_amdgcn_raw_buffer_load_b128(hdr, 0, 0, kCoherentAux);
    const u32x4 h1 = __builtin_amdgcn_raw_buffer_load_b128(hdr, 16, 0, kCoherentAux);
    const int32_t ep = (int32_t)h0[kHeaderEpoch] + 1;
    s_epoch = ep;
    s_failed = h0[kHeaderError] != 0 && (int32_t)h0[kHeaderErrorEpoch] != ep;
    s_stall_layer = (int32_t)h0[kHeaderStallLayer] - 1;
    s_stall_ticks = (int32_t)h1[kHeaderStallTicks - 4];
  }
  step_barrier<!kWalk>();
  const int32_t ticket = wave_uniform(s_ticket);
  const bool active = ticket < p.batch * p.splits;
  const int32_t b = active ? ticket % p.batch : 0;
  const int32_t split = active ? ticket / p.batch : p.splits;  // inactive: no keys
  const int32_t head = xcd;
  const int32_t u = b * kSHeads + head;
  // Step: the lengths and token positions as prepared for this step. Walk:
  // the lengths before the walk; iteration i appends position len + i and
  // attends over len + i + 1 keys.
  const int32_t seq_len = wave_uniform(kWalk ? p.seq_lengths[b] + 1 : p.seq_lengths[b]);
  const int32_t new_pos = wave_uniform(kWalk ? p.seq_lengths[b] : p.token_position[b]);
  auto seq_at = [&](int32_t i) { return kWalk ? seq_len + i : seq_len; };
  auto pos_at = [&](int32_t i) { return kWalk ? new_pos + i : new_pos; };
  const int64_t q_stride = (int64_t)p.units * kSGroup * kSDim;  // per layer
  const int64_t kv_stride = (int64_t)p.units * kSDim;
  // Split records: one buffer over the whole region, addressed in bytes.
  const BufferRsrc rec_buf = buffer_of(p.records, (int64_t)p.units * p.splits * kRecordFloats * 4);
  auto record = [&](int32_t s) -> int32_t {  // byte offset of split s's record
    return (u * p.splits + s) * (kRecordFloats * 4);
  };
  const int32_t epoch = wave_uniform(s_epoch);
  auto is_global_i = [&](int32_t i) { return !kWalk && model_layer_global(p.first_layer + i); };
  // Flag words of iteration i and the value that marks it complete. A step
  // uses one flag row per model layer and marks it with the launch epoch; a
  // walk cycles four rows and marks iteration i with (epoch, i) in one word
  // (an iteration's row is rewritten only after every workgroup is past it).
  auto fslot = [&](int32_t i) { return kWalk ? (i & 3) : i; };
  auto stamp = [&](int32_t i) {
    return kWalk ? (int32_t)(((uint32_t)epoch << 16) | ((uint32_t)i & 0xffffu)) : epoch;
  };
  // Zeros for the output chunks this workgroup owns (those it combines:
  // c = split, split + splits, ... of both rows of unit u), layers from..end.
  auto zero_own_chunks = [&](int32_t from) {
    const int g = lane >> 5;
    const int32_t c = split + (lane & 31) * p.splits;
    if (!active || c >= kChunks) return;
    for (int32_t i = from; i < p.layer_count; ++i) {
      uint4 *dst = reinterpret_cast<uint4 *>(p.out + i * q_stride + (u * kSGroup + g) * kSDim +
                                             c * kPackElems);
      *dst = make_uint4(0, 0, 0, 0);
    }
  };
  if (wave_uniform(s_failed)) {
    if (wave == kControlWave) zero_own_chunks(0);
    return;
  }

  // Wave-local tile j of a split is tile t = wave + kComputeWaves * j; tiles
  // 0 .. kRegTiles - 1 are prefetched into compute-wave registers, tiles
  // kRegTiles .. kRegTiles + kLdsSlots - 1 of a global layer come from LDS
  // slot t - kRegTiles, later ones are streamed.
  if (wave == kPrefetchWave) {
    // ----------------------------------------------------------- prefetch
    // The LDS tiles of the next global layer are requested a few slots at a
    // time over the kLdsLead layers before it, so the DMA traffic never
    // arrives as one burst on the critical path of a layer. This wave waits
    // only for its own DMA, so its outstanding loads hold nobody up.
    auto next_global = [&](int32_t from) {
      for (int32_t l = from; l < p.layer_count; ++l)
        if (is_global_i(l)) return l;
      return (int32_t)-1;
    };
    const int r = lane / kLPR;
    const int64_t col = (int64_t)(kFloor == 6 ? 0 : head) * kSDim + (lane % kLPR) * kPackElems;
    const uint16_t *kb = p.cache_k[1] + col;
    const uint16_t *vb = p.cache_v[1] + col;
    int32_t target = -1, slots = 0, filled = 0;
    auto plan = [&](int32_t gi) {
      // Cache rows of the slot keys: entry e = slot * 8 + key.
      const Gemma4KvCacheConfig &c = p.c[1];
      const int32_t cache_layer = wave_uniform(cache_layer_of(p.first_layer + gi));
      const int32_t split_size = (seq_len + p.splits - 1) / p.splits;
      const int32_t k0 = split * split_size;
      const int32_t k1 = active ? min(seq_len, k0 + split_size) : k0;
      const bool live_new = new_pos >= 0 && new_pos < seq_len;
      const int32_t *pt = p.page_table[1] + b * c.max_pages_per_seq;
      int32_t *tab = reinterpret_cast<int32_t *>(s_lds_rows);
      for (int e = lane; e < kLdsSlots * kTileKeys; e += kWave) {
        const int32_t key = k0 + (kRegTiles + e / kTileKeys) * kTileKeys + e % kTileKeys;
        const int32_t logical = key / c.page_size;
        const int32_t physical = pt[logical % c.max_pages_per_seq];
        const bool ok = key < k1 && !(live_new && key == new_pos) && physical >= 0 &&
                        physical < c.num_pages;
        tab[e] = ok ? (cache_layer * c.num_pages + physical) * c.page_size +
                          (key - logical * c.page_size)
                    : kRowInvalid;
      }
      wave_lds_sync();
      const int32_t tiles = k1 > k0 ? (k1 - k0 + kTileKeys - 1) / kTileKeys : 0;
      target = gi;
      slots = (kFloor >= 1 && kFloor <= 4) ? 0
                                           : wave_uniform(max(0, min(kLdsSlots, tiles - kRegTiles)));
      filled = 0;
    };
    auto request = [&](int count) {
      for (int n = 0; n < count && filled < slots; ++n, ++filled) {
        const int4 rr = s_lds_rows[filled * 2 + r];
        const int32_t rows[4] = {rr.x, rr.y, rr.z, rr.w};
#pragma unroll
        for (int kl = 0; kl < kTileLoads; ++kl) {
          const int64_t off = (int64_t)(rows[kl] < 0 ? 0 : rows[kl]) * kRowElems;
          // cache policy 2 = nontemporal: streamed once, keep L2 for the records
          __builtin_amdgcn_global_load_lds(kb + off, s_tiles + (filled * 8 + kl) * kWave, 16, 0,
                                           2);
          __builtin_amdgcn_global_load_lds(vb + off, s_tiles + (filled * 8 + 4 + kl) * kWave, 16,
                                           0, 2);
        }
      }
    };
    auto maybe_plan = [&](int32_t i) {  // at layer i: start the next global layer?
      if (target > i) return;           // still filling for a later layer
      const int32_t g = next_global(i + 1);
      if (g >= 0 && g - i <= kLdsLead) plan(g);
    };
    maybe_plan(-1);
    for (int32_t i = 0; i < p.layer_count; ++i) {
      if (target == i) {
        // Everything of this global layer requested and landed before its
        // compute starts.
        request(kLdsSlots);
        wait_stores_complete();
      }
      step_barrier<!kWalk>();  // A
      if (target > i) request(kSlotsPerInterval);
      step_barrier<!kWalk>();  // B
      if (target > i) request(kSlotsPerInterval);
      step_barrier<!kWalk>();  // C
      maybe_plan(i);
      if (target > i) request(kSlotsPerInterval);
    }
    return;
  }

  if (wave == kControlWave) {
    // ------------------------------------------------------------ control
    // The control wave carries the per-layer chain (flags, inputs, combine):
    // it issues ahead of the compute wave sharing its SIMD (measured 1.3%
    // off the step; raising the compute waves over the prefetch wave too
    // changed nothing).
    __builtin_amdgcn_s_setprio(3);
    bool abort = false;
    // Records an error under this launch's epoch; a wait that gives up also
    // stops every later wait of this wave.
    auto fail = [&](int32_t code) {
      abort = true;
      if (lane == 0) {
        coherent_store_i32(p.header + kHeaderErrorEpoch, epoch);
        coherent_store_i32(p.header + kHeaderError, code);
      }
    };
    // A split longer than the row tables hold would drop keys: report it.
    // Only the kinds of cache this launch reads (a run of sliding layers
    // never reads the global cache).
    bool uses[2] = {false, false};
    for (int32_t l = 0; l < p.layer_count; ++l) uses[is_global_i(l) ? 1 : 0] = true;
    for (int kind = 0; kind < (kWalk ? 1 : 2); ++kind) {
      if (!uses[kind]) continue;
      const Gemma4KvCacheConfig &c = p.c[kind];
      const int32_t last_len = seq_at(p.layer_count - 1);  // the longest iteration
      int32_t first = c.window_size > 0 ? last_len - c.window_size : 0;
      first = first < 0 ? 0 : first;
      const int32_t n_keys = last_len > first ? last_len - first : 0;
      if ((n_keys + p.splits - 1) / p.splits > kMaxSplitKeys) fail(2);
    }
    // Fault injection for tests: at layer stall_layer - 1, ticket 0 of XCD 0
    // waits, with the given limit, for a header word the host never sets.
    const int32_t stall_layer = wave_uniform(s_stall_layer);
    const uint64_t stall_ticks = (uint32_t)wave_uniform(s_stall_ticks);
    // Polls a flag word per lane until every lane reads `want`, one load
    // in flight at a time (keeping up to four in flight measured no faster:
    // the flag's propagation, not the poll spacing, sets the wait).
    auto poll = [&](int32_t want, auto load) {
      const uint64_t t0 = now_ticks();
      while (!abort) {
        if (__ballot(load() != want) == 0) return;
        if (now_ticks() - t0 > kWaitTicks) fail(1);
      }
    };
    // Layer `layer_i` is complete once all 8 XCD flags read `epoch`.
    const BufferRsrc flag_buf =
        buffer_of(p.global_flags, (int64_t)kNumModelLayers * kGlobalFlagStride * 4);
    auto wait_layer_device = [&](int32_t layer_i) {
      const int32_t off = (fslot(layer_i) * kGlobalFlagStride + (lane & (kXcds - 1))) * 4;
      poll(stamp(layer_i), [&] {
        return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(flag_buf, off, 0, kCoherentAux);
      });
    };
    // Ticket 0 of each XCD polls the 8 device flags and raises the XCD's
    // go flag in its L2; the other 31 workgroups poll that (an L2 round
    // trip, so they start together).
    const BufferRsrc go_buf = buffer_of(p.go_flags, (int64_t)kNumModelLayers * kXcds * 16 * 4);
    auto wait_layer = [&](int32_t layer_i) {
      const int32_t off = ((fslot(layer_i) * kXcds + xcd) * 16) * 4;
      if (ticket == 0) {
        wait_layer_device(layer_i);
        if (lane == 0)
          __builtin_amdgcn_raw_buffer_store_b32((uint32_t)stamp(layer_i), go_buf, off, 0, 0);
        return;
      }
      poll(stamp(layer_i), [&] {
        return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(go_buf, off, 0, kLocalLoadAux);
      });
    };
    // Ticket 0 of each XCD: collect the XCD's 32 local flags, then raise
    // the XCD's device-wide flag.
    const BufferRsrc local_buf =
        buffer_of(p.local_flags, (int64_t)kNumModelLayers * kXcds * kXcdSlots * 4);
    auto publish_xcd = [&](int32_t layer_i) {
      const int32_t off =
          ((fslot(layer_i) * kXcds + xcd) * kXcdSlots + (lane & (kXcdSlots - 1))) * 4;
      poll(stamp(layer_i), [&] {
        return (int32_t)__builtin_amdgcn_raw_buffer_load_b32(local_buf, off, 0, kLocalLoadAux);
      });
      if (lane == 0)
        coherent_store_i32(p.global_flags + fslot(layer_i) * kGlobalFlagStride + xcd,
                           stamp(layer_i));
    };
    // Lane (g, sp) = (lane / 32, lane % 32) reads split sp's row g, so the
    // reductions over splits stay within 32-lane halves (DPP row ops and
    // one swizzle per step).
    const int sp = lane & (kXcdSlots - 1);
    const int g = lane >> 5;
    const bool live = sp < p.splits;
    const BufferRsrc in_buf_q = buffer_of(p.q, (int64_t)p.layer_count * q_stride * 2);
    const BufferRsrc in_buf_k = buffer_of(p.new_k, (int64_t)p.layer_count * kv_stride * 2);
    const BufferRsrc in_buf_v = buffer_of(p.new_v, (int64_t)p.layer_count * kv_stride * 2);
    for (int32_t i = 0; i < p.layer_count; ++i) {
      STEP_MARK(0);
      // What the preparation needs besides the projections does not depend
      // on the previous layer: this layer's norm weights and the RoPE row of
      // the token's position are requested before the wait.
      const bool prep = p.q_norm_w != nullptr;
      uint4 w_q = make_uint4(0, 0, 0, 0), w_k = w_q;
      float rc[kPackElems], rs[kPackElems];
      if (prep) {
        const int cp = lane & 31;
        w_q = load128(p.q_norm_w + (int64_t)i * kSDim + cp * kPackElems);
        w_k = load128(p.k_norm_w + (int64_t)i * kSDim + cp * kPackElems);
        const int kind = is_global_i(i) ? 1 : 0;
        const int32_t pos = max(pos_at(i), 0);
        const int pair = (cp * kPackElems) % (kSDim / 2);
        const float4 *cr = reinterpret_cast<const float4 *>(p.rope_cos[kind] +
                                                             (int64_t)pos * (kSDim / 2) + pair);
        const float4 *sr = reinterpret_cast<const float4 *>(p.rope_sin[kind] +
                                                             (int64_t)pos * (kSDim / 2) + pair);
        const float4 c0 = cr[0], c1 = cr[1], s0 = sr[0], s1 = sr[1];
        rc[0] = c0.x; rc[1] = c0.y; rc[2] = c0.z; rc[3] = c0.w;
        rc[4] = c1.x; rc[5] = c1.y; rc[6] = c1.z; rc[7] = c1.w;
        rs[0] = s0.x; rs[1] = s0.y; rs[2] = s0.z; rs[3] = s0.w;
        rs[4] = s1.x; rs[5] = s1.y; rs[6] = s1.z; rs[7] = s1.w;
      }
      if (i > 0) wait_layer(i - 1);
      STEP_MARK(1);
      if (i == stall_layer && xcd == 0 && ticket == 0) {
        const uint64_t t0 = now_ticks();
        while (!abort && coherent_load_i32(p.header + kHeaderNeverSet) != epoch) {
          if (now_ticks() - t0 > stall_ticks) fail(1);
        }
      }
      // Layer i's inputs exist only now: q rows and appended K/V rows of the
      // unit, read device-coherently and staged in LDS for the compute waves.
      if (kFloor < 3) {
        const int32_t qoff = (int32_t)((i * q_stride + (u * kSGroup + (lane >> 5)) * kSDim +
                                        (lane & 31) * kPackElems) * 2);
        const int32_t kvoff = (int32_t)((i * kv_stride + u * kSDim + (lane & 31) * kPackElems) * 2);
        const u32x4 qv = __builtin_amdgcn_raw_buffer_load_b128(in_buf_q, qoff, 0, kCoherentAux);
        const u32x4 nv = lane < 32
                             ? __builtin_amdgcn_raw_buffer_load_b128(in_buf_k, kvoff, 0, kCoherentAux)
                             : __builtin_amdgcn_raw_buffer_load_b128(in_buf_v, kvoff, 0, kCoherentAux);
        uint4 qp = make_uint4(qv[0], qv[1], qv[2], qv[3]);
        uint4 np = make_uint4(nv[0], nv[1], nv[2], nv[3]);
        if (prep && pos_at(i) >= 0) {
          // Q rows and the new K row: learned RMSNorm + RoPE; the new V row:
          // scale-free RMSNorm (each row is one 32-lane half).
          qp = prep_row(qp, w_q, true, rc, rs, lane & 31);
          np = prep_row(np, w_k, lane < 32, rc, rs, lane & 31);
        }
        s_q[lane] = qp;
        s_new[lane] = np;
      }
      STEP_MARK(2);
      step_barrier<!kWalk>();  // A: layer i may start
      step_barrier<!kWalk>();  // B: this workgroup's compute waves finished layer i
      STEP_MARK(5);

      // Combine unit u's splits for the 8-dim chunks c = split, split +
      // splits, ... of both rows: one round of L2 loads per chunk; the
      // chunk is emptied again right after it is read.
      for (int32_t c = split; kFloor < 2 && active && c < kChunks; c += p.splits) {
        // Lanes past the live splits read split 0 and weigh it zero.
        const int32_t off = record(live ? sp : 0) + (c * kChunkFloats + g * kHalfChunk) * 4;
        struct Poll {
          u32x4 lo, hi;
          u32x2 ml;
        };
        auto issue = [&](Poll &q) {
          q.lo = __builtin_amdgcn_raw_buffer_load_b128(rec_buf, off, 0, kLocalLoadAux);
          q.hi = __builtin_amdgcn_raw_buffer_load_b128(rec_buf, off + 16, 0, kLocalLoadAux);
          q.ml = __builtin_amdgcn_raw_buffer_load_b64(rec_buf, off + 32, 0, kLocalLoadAux);
        };
        auto complete = [&](const Poll &q) {
          bool bad = q.ml[0] == kSentinel || q.ml[1] == kSentinel;
#pragma unroll
          for (int j = 0; j < 4; ++j) bad |= q.lo[j] == kSentinel || q.hi[j] == kSentinel;
          return __ballot(bad) == 0;
        };
        // One poll in flight at a time: measured faster than keeping
        // several staggered polls outstanding.
        Poll got;
        {
          const uint64_t t0 = now_ticks();
          issue(got);
          while (!complete(got) && !abort) {
            if (now_ticks() - t0 > kWaitTicks) fail(1);
            issue(got);
          }
        }
        {
          const float m_s = live ? __uint_as_float(got.ml[0]) : -INFINITY;
          const float l_s = live ? __uint_as_float(got.ml[1]) : 0.0f;
          // Reduce over the splits (lane bits 0..4) of each row g = lane bit 5.
          float big_m = m_s;
          big_m = xor_max<16>(big_m);
          big_m = fmaxf(big_m, lane_pair<8>(big_m));
          big_m = fmaxf(big_m, lane_pair<4>(big_m));
          big_m = fmaxf(big_m, lane_pair<2>(big_m));
          big_m = fmaxf(big_m, lane_pair<1>(big_m));
          const float m_ref = big_m == -INFINITY ? 0.0f : big_m;
          const float w = l_s > 0.0f ? __builtin_amdgcn_exp2f(m_s - m_ref) : 0.0f;
          float big_l = w * l_s;
          big_l = xor_sum<16>(big_l);
          big_l += lane_pair<8>(big_l);
          big_l += lane_pair<4>(big_l);
          big_l += lane_pair<2>(big_l);
          big_l += lane_pair<1>(big_l);
          // Value-splitting sum of the 8 weighted dims over the 32 split
          // lanes: lane holds the sum of dim (lane >> 2) & 7 afterwards.
          float v[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            v[j] = w * __uint_as_float(got.lo[j]);
            v[4 + j] = w * __uint_as_float(got.hi[j]);
          }
          split_butterfly<8, 16>(v, lane);
          if ((lane & 3) == 0) {
            const int dim = (lane >> 2) & 7;
            const float inv = big_l > 0.0f ? 1.0f / big_l : 0.0f;
            // Output rows go out device-coherent.
            const BufferRsrc out_buf = buffer_of(p.out + i * q_stride, q_stride * 2);
            // After a wait gave up, this wave's chunks are written as zeros.
            __builtin_amdgcn_raw_buffer_store_b16(
                abort ? (uint16_t)0 : (uint16_t)f32_to_bf16_bits(v[0] * inv), out_buf,
                ((u * kSGroup + g) * kSDim + c * kPackElems + dim) * 2, 0, kCoherentAux);
          }
        }
        if (live) {
          // Empty the chunk for the next layer (completed before this
          // workgroup's flag, so before any next-layer write).
          const u32x4 s4 = {kSentinel, kSentinel, kSentinel, kSentinel};
          const u32x2 s2 = {kSentinel, kSentinel};
          __builtin_amdgcn_raw_buffer_store_b128(s4, rec_buf, off, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b128(s4, rec_buf, off + 16, 0, 0);
          __builtin_amdgcn_raw_buffer_store_b64(s2, rec_buf, off + 32, 0, 0);
        }
      }
      STEP_MARK(6);
      step_barrier<!kWalk>();  // C: records read; compute waves may prefetch
      // My output slices and chunk resets are complete before my local flag.
      wait_stores_complete();
      if (lane == 0) {
        __builtin_amdgcn_raw_buffer_store_b32(
            (uint32_t)stamp(i), local_buf, ((fslot(i) * kXcds + xcd) * kXcdSlots + ticket) * 4,
            0, 0);
      }
      if (ticket == 0) publish_xcd(i);
      STEP_MARK(7);
    }
    if (xcd == 0 && ticket == 0) {
      // Every workgroup has read the header (and finished): advance it.
      wait_layer(p.layer_count - 1);
      if (lane == 0) coherent_store_i32(p.header + kHeaderEpoch, epoch);
      if (kWalk && !abort && lane < p.batch) {
        // Every workgroup read the lengths at entry: leave the metadata of
        // the walk's last step (as a decode step's preparation would).
        const int32_t last = p.seq_lengths[lane] + p.layer_count - 1;
        const_cast<int32_t *>(p.seq_lengths)[lane] = last + 1;
        const_cast<int32_t *>(p.token_position)[lane] = last;
      }
    }
    // This wave gave up a wait: its chunks of the layers before that are
    // zeroed too, so none of its output is left from a failed step.
    if (abort) zero_own_chunks(0);
    return;
  }

  // -------------------------------------------------------------- compute
  const int r = lane / kLPR;      // row half of a load: key rows 4r..4r+3
  const int cpack = lane % kLPR;  // 16-byte pack of the row
  const int idx = cpack >> kSBits;
  const int my_g = idx & (kSGroup - 1);
  const int my_kl = idx / kSGroup;

  // Layer view + row table for layer i of this split and wave: keys of the
  // wave's tiles go to s_rows[i & 1][wave] in tile order (tile j at 8j,
  // key 4r+kl).
  auto setup = [&](int32_t i, int slot) -> LayerView {
    LayerView v;
    const int32_t layer = p.first_layer + i;
    const int kind = !kWalk && model_layer_global(layer) ? 1 : 0;
    const Gemma4KvCacheConfig &c = p.c[kind];
    const int32_t cache_layer = kWalk ? p.walk_layer : wave_uniform(cache_layer_of(layer));
    const int32_t seq_len = seq_at(i), new_pos = pos_at(i);
    int32_t first = c.window_size > 0 ? seq_len - c.window_size : 0;
    first = first < 0 ? 0 : first;
    const int32_t n_keys = seq_len > first ? seq_len - first : 0;
    const int32_t split_size = (n_keys + p.splits - 1) / p.splits;
    const int32_t k0 = first + split * split_size;
    const int32_t k1 = active ? min(seq_len, k0 + split_size) : k0;
    const int32_t tiles = k1 > k0 ? (k1 - k0 + kTileKeys - 1) / kTileKeys : 0;
    v.n_tiles = tiles > wave && (kFloor == 0 || kFloor >= 4)
                    ? min((tiles - wave + kComputeWaves - 1) / kComputeWaves,
                          kWaveKeys / kTileKeys)
                    : 0;
    const bool live_new = new_pos >= first && new_pos < seq_len;
    const int32_t owner_split = live_new ? (new_pos - first) / max(split_size, 1) : 0;
    const int32_t owner_wave = live_new ? ((new_pos - k0) / kTileKeys) % kComputeWaves : 0;
    const int32_t new_row = split == owner_split && wave == owner_wave
                                ? append_row(c, p.page_table[kind], cache_layer, b, new_pos)
                                : -1;
    v.owner = live_new && split == owner_split && wave == owner_wave;
    {
      const int32_t kk = new_pos - k0;  // key index of the new token in the split
      v.new_j = v.owner ? (kk / kTileKeys) / kComputeWaves : -1;
      v.new_r = (kk % kTileKeys) / kTileLoads;
      v.new_kl = (kk % kTileKeys) % kTileLoads;
    }
    v.lds = kind == 1;
    v.par = slot;
    v.kind = kind;
    v.new_row = (kFloor >= 1 && kFloor <= 3) ? -1 : wave_uniform(new_row);
    // Two table entries per lane: wave-local key e = lane, lane + 64.
    const int32_t *pt = p.page_table[kind] + b * c.max_pages_per_seq;
    int32_t rows[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = lane + h * kWave;
      const int32_t t = wave + (e / kTileKeys) * kComputeWaves;
      const int32_t key = k0 + t * kTileKeys + e % kTileKeys;
      const int32_t logical = key / c.page_size;
      const int32_t physical = pt[logical % c.max_pages_per_seq];
      const bool ok = e / kTileKeys < v.n_tiles && key < k1 && !(live_new && key == new_pos) &&
                      physical >= 0 && physical < c.num_pages;
      rows[h] = ok ? ((cache_layer * c.num_pages + physical) * c.page_size +
                      (key - logical * c.page_size))
                   : kRowInvalid;
    }
    int32_t *tab = reinterpret_cast<int32_t *>(s_rows[v.par][wave]);
    tab[lane] = rows[0];
    tab[lane + kWave] = rows[1];
    wave_lds_sync();
    return v;
  };

  struct TileBuf {
    uint4 k[kTileLoads], v[kTileLoads];
    uint32_t valid;
  };
  const int32_t col = head * kSDim + cpack * kPackElems;  // element offset in a cache row
  // Walks: the cache as buffers (the host keeps it under 2 GiB).
  const int64_t walk_bytes = (int64_t)p.c[0].num_layers * p.c[0].num_pages * p.c[0].page_size *
                             kRowElems * 2;
  const BufferRsrc walk_k = buffer_of(p.cache_k[0], walk_bytes);
  const BufferRsrc walk_v = buffer_of(p.cache_v[0], walk_bytes);
  auto issue = [&](TileBuf &tb, const LayerView &v, int t) {
    const int4 rr = s_rows[v.par][wave][t * 2 + r];
    const int32_t rows[4] = {rr.x, rr.y, rr.z, rr.w};
    const uint16_t *kb = p.cache_k[v.kind] - (kFloor == 6 && v.kind == 1 ? head * kSDim : 0);
    const uint16_t *vb = p.cache_v[v.kind] - (kFloor == 6 && v.kind == 1 ? head * kSDim : 0);
    tb.valid = 0;
#pragma unroll
    for (int kl = 0; kl < kTileLoads; ++kl) {
      tb.valid |= (rows[kl] >= 0 ? 1u : 0u) << kl;
      const int64_t off = (int64_t)(rows[kl] < 0 ? 0 : rows[kl]) * kRowElems + col;
      if constexpr (kFloor == 4) {
        tb.k[kl] = make_uint4(rows[kl], lane, kl, t);
        tb.v[kl] = make_uint4(t, kl, lane, rows[kl]);
      } else if constexpr (kWalk) {
        // Rows appended earlier in this launch were written by other
        // workgroups of this XCD: sc0|nt loads skip this CU's L1 (which may
        // still hold the slot's previous row) and read the shared L2.
        const int32_t boff = (int32_t)(off * 2);
        const u32x4 kk = __builtin_amdgcn_raw_buffer_load_b128(walk_k, boff, 0, kLocalLoadAux);
        const u32x4 vv = __builtin_amdgcn_raw_buffer_load_b128(walk_v, boff, 0, kLocalLoadAux);
        tb.k[kl] = make_uint4(kk[0], kk[1], kk[2], kk[3]);
        tb.v[kl] = make_uint4(vv[0], vv[1], vv[2], vv[3]);
      } else {
        tb.k[kl] = load128_stream(kb + off);
        tb.v[kl] = load128_stream(vb + off);
      }
    }
  };

  uint32_t qw[kSGroup][4];
  float m[kSGroup], acc[kSGroup][8], l_lane;
  // One tile in two steps, so a tile read from LDS needs its V packs in
  // registers only after the K packs are done with: scores() updates the
  // online softmax and leaves the tile's probabilities in pv / alpha;
  // accumulate() adds P.V.
  float pv[kNP], alpha[kSGroup];
  auto scores = [&](const uint4 (&k)[kTileLoads], uint32_t valid_bits) {
    float part[kNP];
#pragma unroll
    for (int kl = 0; kl < kTileLoads; ++kl) {
      const uint32_t kw[4] = {k[kl].x, k[kl].y, k[kl].z, k[kl].w};
#pragma unroll
      for (int g = 0; g < kSGroup; ++g) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) a = dot2_bf16(qw[g][j], kw[j], a);
        part[kl * kSGroup + g] = a;
      }
    }
    split_butterfly<kNP, kLPR / 2>(part, lane);
    const bool valid = (valid_bits >> my_kl) & 1u;
    const float score = valid ? part[0] * p.q_scale : -INFINITY;
    float tmax[kSGroup];
    gather_heads<kSGroup, kSBits>(reduce_max_from<(1 << kSBits) * kSGroup>(score), my_g, tmax);
    float m_use[kSGroup];
#pragma unroll
    for (int g = 0; g < kSGroup; ++g) {
      const float m_new = fmaxf(m[g], tmax[g]);
      m_use[g] = m_new == -INFINITY ? 0.0f : m_new;
      alpha[g] = __builtin_amdgcn_exp2f(m[g] - m_use[g]);
      m[g] = m_new;
    }
    const float my_m = my_g ? m_use[1] : m_use[0];
    const float my_alpha = my_g ? alpha[1] : alpha[0];
    const float prob = __builtin_amdgcn_exp2f(score - my_m);
    l_lane = l_lane * my_alpha + prob;
    s_prob[wave][r * kNP + idx] = prob;
    wave_lds_sync();
#pragma unroll
    for (int i = 0; i < kNP; i += 4) {
      const float4 q4 = *reinterpret_cast<const float4 *>(&s_prob[wave][r * kNP + i]);
      pv[i] = q4.x; pv[i + 1] = q4.y; pv[i + 2] = q4.z; pv[i + 3] = q4.w;
    }
  };
  // P.V on v_dot2 over key pairs: the probabilities of keys (0, 1) and
  // (2, 3) of the lane's row half are packed as bf16 pairs (RNE), and each V
  // word pair of those keys is regrouped by dim with one byte permute, so a
  // dot2 adds both keys' terms of one dim (fp32 products and sums).
  auto accumulate = [&](const uint4 (&v)[kTileLoads], uint32_t valid_bits) {
#pragma unroll
    for (int g = 0; g < kSGroup; ++g) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] *= alpha[g];
    }
    uint32_t w[kTileLoads][4];
#pragma unroll
    for (int kl = 0; kl < kTileLoads; ++kl) {
      const bool ok = (valid_bits >> kl) & 1u;
      w[kl][0] = ok ? v[kl].x : 0u;
      w[kl][1] = ok ? v[kl].y : 0u;
      w[kl][2] = ok ? v[kl].z : 0u;
      w[kl][3] = ok ? v[kl].w : 0u;
    }
#pragma unroll
    for (int pr = 0; pr < kTileLoads / 2; ++pr) {
      uint32_t pp[kSGroup];
#pragma unroll
      for (int g = 0; g < kSGroup; ++g) {
        const bf16x2_t pair = {(__bf16)pv[(2 * pr) * kSGroup + g],
                               (__bf16)pv[(2 * pr + 1) * kSGroup + g]};
        pp[g] = __builtin_bit_cast(uint32_t, pair);
      }
#pragma unroll
      for (int wi = 0; wi < 4; ++wi) {
        const uint32_t a = w[2 * pr][wi], b = w[2 * pr + 1][wi];
        const uint32_t lo = __builtin_amdgcn_perm(b, a, 0x05040100u);  // dim 2wi of both keys
        const uint32_t hi = __builtin_amdgcn_perm(b, a, 0x07060302u);  // dim 2wi + 1
#pragma unroll
        for (int g = 0; g < kSGroup; ++g) {
          acc[g][2 * wi] = dot2_bf16(pp[g], lo, acc[g][2 * wi]);
          acc[g][2 * wi + 1] = dot2_bf16(pp[g], hi, acc[g][2 * wi + 1]);
        }
      }
    }
  };
  auto compute = [&](const TileBuf &t) {
    if constexpr (kFloor == 5) {
#pragma unroll
      for (int kl = 0; kl < kTileLoads; ++kl) {
        asm volatile("" ::"v"(t.k[kl].x), "v"(t.k[kl].y), "v"(t.k[kl].z), "v"(t.k[kl].w));
        asm volatile("" ::"v"(t.v[kl].x), "v"(t.v[kl].y), "v"(t.v[kl].z), "v"(t.v[kl].w));
      }
      return;
    }
    scores(t.k, t.valid);
    accumulate(t.v, t.valid);
  };
  // The appended token replaces its (masked) slot in its tile: the lanes of
  // its row take the new K/V packs from LDS.
  auto patch_packs = [&](uint4 (&x)[kTileLoads], uint32_t &valid, const LayerView &v,
                         int half) __attribute__((always_inline)) {
    const uint4 nw = s_new[half * kLPR + cpack];
#pragma unroll
    for (int kl = 0; kl < kTileLoads; ++kl) {
      const bool sel = kl == v.new_kl && r == v.new_r;
      x[kl].x = sel ? nw.x : x[kl].x;
      x[kl].y = sel ? nw.y : x[kl].y;
      x[kl].z = sel ? nw.z : x[kl].z;
      x[kl].w = sel ? nw.w : x[kl].w;
    }
    valid |= r == v.new_r ? 1u << v.new_kl : 0u;
  };
  auto patch_tile = [&](TileBuf &t, const LayerView &v, int32_t j)
                        __attribute__((always_inline)) {
    if (v.owner && j == v.new_j) {
      patch_packs(t.k, t.valid, v, 0);
      patch_packs(t.v, t.valid, v, 1);
    }
  };

  // Register prefetch: at the end of layer i (barrier C) the first tiles of
  // layer i+1 are requested. (Issuing them earlier -- several layers ahead
  // for a global layer, or two layers ahead for sliding ones -- was measured
  // slower: the waits of the layers in between then cover those loads too.)
  auto append_new = [&](const LayerView &v) {
    if (v.new_row >= 0 && r == 0) {
      const int64_t dst = (int64_t)v.new_row * kRowElems + col;
      store128(p.cache_k[v.kind] + dst, s_new[cpack]);
      store128(p.cache_v[v.kind] + dst, s_new[kLPR + cpack]);
    }
  };

  TileBuf buf[kPrefetchTiles];
  LayerView cur;
  auto prepare = [&](int32_t i) {  // at the end of layer i (i = -1: start)
    const int32_t n1 = i + 1;
    if (n1 >= p.layer_count) return;
    cur = setup(n1, n1 & 1);
#pragma unroll
    for (int j = 0; j < kPrefetchTiles; ++j)
      if (j < cur.n_tiles) issue(buf[j], cur, j);
  };
  prepare(-1);

  // This wave's record dwords: head g = lane / 32, dims d, d+1 of its
  // quarter, inside 8-dim chunk d / 8 (whose first lane also writes m, l).
  constexpr int kMergeDims = kSDim / kComputeWaves / kLPR;  // dims per lane
  const int rec_g = lane / kLPR;
  const int rec_d = wave * (kSDim / kComputeWaves) + (lane % kLPR) * kMergeDims;
  const int32_t rec_acc = (rec_d / kPackElems * kChunkFloats + rec_g * kHalfChunk + rec_d % kPackElems) * 4;
  const int32_t rec_ml = (rec_d / kPackElems * kChunkFloats + rec_g * kHalfChunk + kPackElems) * 4;

  for (int32_t i = 0; i < p.layer_count; ++i) {
    step_barrier<!kWalk>();  // A: layer i-1 published (or i == 0), inputs in LDS
    STEP_MARK(3);
    const LayerView view = cur;
    // A walk appends first, so the store has landed long before barrier B.
    if constexpr (kWalk) append_new(view);
#pragma unroll
    for (int g = 0; g < kSGroup; ++g) {
      const uint4 qp = s_q[g * kLPR + cpack];
      qw[g][0] = qp.x; qw[g][1] = qp.y; qw[g][2] = qp.z; qw[g][3] = qp.w;
      m[g] = -INFINITY;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] = 0.0f;
    }
    l_lane = 0.0f;
    {
      // Wave-local tiles: [0, 4) in registers, [4, lds_end) in LDS (global
      // layers), [lds_end, n) streamed through the register buffers, which
      // are refilled as the prefetched tiles are consumed.
      const int32_t n = view.n_tiles;
      int32_t lds_end = kPrefetchTiles;
      if (view.lds) {
        while (lds_end < n && wave + kComputeWaves * lds_end < kRegTiles + kLdsSlots) ++lds_end;
      }
      const int32_t n_stream = n > lds_end ? n - lds_end : 0;
#pragma unroll
      for (int j = 0; j < kPrefetchTiles; ++j) {
        if (j < n) {
          patch_tile(buf[j], view, j);
          compute(buf[j]);
        }
        if (j < n_stream) issue(buf[j], view, lds_end + j);
      }
      for (int32_t j = kPrefetchTiles; j < lds_end; ++j) {
        const int slot = wave + kComputeWaves * j - kRegTiles;
        const int4 rr = s_lds_rows[slot * 2 + r];
        const uint32_t valid = (rr.x >= 0 ? 1u : 0u) | (rr.y >= 0 ? 2u : 0u) |
                               (rr.z >= 0 ? 4u : 0u) | (rr.w >= 0 ? 8u : 0u);
        uint32_t valid_k = valid, valid_v = valid;
        const bool has_new = view.owner && j == view.new_j;
        uint4 kv[kTileLoads];
#pragma unroll
        for (int kl = 0; kl < kTileLoads; ++kl) kv[kl] = s_tiles[(slot * 8 + kl) * kWave + lane];
        if (has_new) patch_packs(kv, valid_k, view, 0);
        if constexpr (kFloor == 5) {
#pragma unroll
          for (int kl = 0; kl < kTileLoads; ++kl)
            asm volatile("" ::"v"(kv[kl].x), "v"(kv[kl].y), "v"(kv[kl].z), "v"(kv[kl].w));
          continue;
        }
        scores(kv, valid_k);
#pragma unroll
        for (int kl = 0; kl < kTileLoads; ++kl) kv[kl] = s_tiles[(slot * 8 + 4 + kl) * kWave + lane];
        if (has_new) patch_packs(kv, valid_v, view, 1);
        accumulate(kv, valid_v);
      }
      for (int32_t t0 = 0; t0 < n_stream; t0 += kPrefetchTiles) {
#pragma unroll
        for (int j = 0; j < kPrefetchTiles; ++j) {
          if (t0 + j < n_stream) {
            patch_tile(buf[j], view, lds_end + t0 + j);
            compute(buf[j]);
          }
          if (t0 + j + kPrefetchTiles < n_stream)
            issue(buf[j], view, lds_end + t0 + j + kPrefetchTiles);
        }
      }
    }
    if constexpr (!kWalk) {
      append_new(view);
    } else if (view.new_row >= 0) {
      // The appended row is in the L2 before this split's record, so every
      // split that reads it next iteration (after the records) sees it.
      wait_stores_complete();
    }

    // Wave totals to LDS, then the compute waves' partials are merged.
    float l_head[kSGroup];
    gather_heads<kSGroup, kSBits>(reduce_sum_from<(1 << kSBits) * kSGroup>(l_lane), my_g, l_head);
#pragma unroll
    for (int g = 0; g < kSGroup; ++g) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] = sum_rows<kLPR>(acc[g][j]);
    }
    if (lane == 0) {
#pragma unroll
      for (int g = 0; g < kSGroup; ++g) {
        s_ml[wave][g][0] = m[g];
        s_ml[wave][g][1] = l_head[g];
      }
    }
    if (r == 0) {
#pragma unroll
      for (int g = 0; g < kSGroup; ++g) {
        float4 *dst = reinterpret_cast<float4 *>(&s_acc[wave][g][cpack * 8]);
        dst[0] = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
        dst[1] = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
      }
    }
    STEP_MARK(4);
    step_barrier<!kWalk>();  // B
    if (kFloor < 2 && active) {
      float big_m = -INFINITY;
#pragma unroll
      for (int w = 0; w < kComputeWaves; ++w) big_m = fmaxf(big_m, s_ml[w][rec_g][0]);
      const float m_ref = big_m == -INFINITY ? 0.0f : big_m;
      float big_l = 0.0f, a0 = 0.0f, a1 = 0.0f;
#pragma unroll
      for (int w = 0; w < kComputeWaves; ++w) {
        const float f = __builtin_amdgcn_exp2f(s_ml[w][rec_g][0] - m_ref);
        big_l = fmaf(s_ml[w][rec_g][1], f, big_l);
        if constexpr (kMergeDims == 2) {
          const float2 a = *reinterpret_cast<const float2 *>(&s_acc[w][rec_g][rec_d]);
          a0 = fmaf(a.x, f, a0);
          a1 = fmaf(a.y, f, a1);
        } else {
          a0 = fmaf(s_acc[w][rec_g][rec_d], f, a0);
        }
      }
      // The chunk was emptied by its reader before the previous layer
      // completed, so these stores need no wait.
      const int32_t rec = record(split);
      if constexpr (kMergeDims == 2) {
        local_store2(rec_buf, rec + rec_acc, a0, a1);
      } else {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(a0), rec_buf, rec + rec_acc, 0, 0);
        (void)a1;
      }
      if (rec_d % kPackElems == 0) local_store2(rec_buf, rec + rec_ml, big_m, big_l);
    }
    STEP_MARK(9);
    step_barrier<!kWalk>();  // C: the control wave has read the split records
    prepare(i);
  }
}

__global__ void decode_step_workspace_init_kernel(int32_t *ints, int64_t n_ints,
                                                  uint32_t *records, int64_t n_records) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; x < n_ints; x += stride)
    ints[x] = 0;
  for (int64_t x = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; x < n_records; x += stride)
    records[x] = kSentinel;
}

// The reference model's global geometry (1 KV head x 512, src/gemma4.h:17-21)
// runs its layers as per-layer fused launches between the persistent runs,
// with the separate combine kernel (the in-kernel combine would put all 16
// query heads of a split set on one workgroup: 1.33 against 0.55 ms per
// config-2 step); their split partials live in the workspace. Their split
// plan targets one workgroup per CU (measured best against 128, 64 and 32),
// so batch x splits <= 256 + batch.
constexpr int kRefDim = 512;
constexpr int kRefTargetWorkgroups = kStepWorkgroups;
constexpr int64_t kRefPartialSlots = kRefTargetWorkgroups + kMaxBatch;  // (sequence, split) pairs

// Workspace: header | XCD ticket counters | local flags | global flags |
// probe slots | go flags | split records (sentinel-filled) | 1x512 split
// partials.
struct WorkspaceLayout {
  int32_t units, splits;
  int64_t tickets, local_flags, global_flags, probe, go_flags, int_count, record_floats,
      ref_partial_floats, bytes;
};
WorkspaceLayout workspace_layout(int32_t batch_count) {
  WorkspaceLayout w{};
  w.units = batch_count * kSHeads;
  w.splits = batch_count > 0 ? kXcdSlots / batch_count : 0;
  w.tickets = kHeaderInts;
  w.local_flags = w.tickets + kXcds * kTicketStride;
  w.global_flags = w.local_flags + (int64_t)kNumModelLayers * kXcds * kXcdSlots;
  w.probe = w.global_flags + (int64_t)kNumModelLayers * kGlobalFlagStride;
  w.go_flags = w.probe + kStepWorkgroups;
  w.int_count = w.go_flags + (int64_t)kNumModelLayers * kXcds * 16;
  w.record_floats = (int64_t)w.units * w.splits * kRecordFloats;
  w.ref_partial_floats = kRefPartialSlots * kQueryHeads * (2 + kRefDim);
  w.bytes = (w.int_count + w.record_floats + w.ref_partial_floats) * 4;
  w.bytes = (w.bytes + 7) / 8 * 8;
  if (STEP_TRACE) w.bytes += (int64_t)kStepWorkgroups * kNumModelLayers * 10 * 8;
  return w;
}

// Per-device result of the placement probe: 0 unknown, 1 ok, -1 unsupported
// (atomic: workspace_init and the steps may run on different host threads).
std::atomic<int> g_placement_ok[64];

StepParams base_params(void *workspace, const WorkspaceLayout &w, int32_t batch_count) {
  StepParams p{};
  int32_t *ints = static_cast<int32_t *>(workspace);
  p.header = ints;
  p.tickets = reinterpret_cast<uint32_t *>(ints + w.tickets);
  p.local_flags = ints + w.local_flags;
  p.global_flags = ints + w.global_flags;
  p.go_flags = ints + w.go_flags;
  p.records = reinterpret_cast<float *>(ints + w.int_count);
  if (STEP_TRACE) {
    const int64_t off = ((w.int_count + w.record_floats + w.ref_partial_floats) * 4 + 7) / 8 * 8;
    p.trace = reinterpret_cast<uint64_t *>(static_cast<char *>(workspace) + off);
  }
  p.batch = batch_count;
  p.units = w.units;
  p.splits = w.splits;
  return p;
}

// The placement probe at workspace initialisation is an ordinary launch;
// it checks that the 256 workgroups land 32 per XCD on 256 distinct CUs (the
// 157 KB of LDS a workgroup takes leaves room for no second one on a CU).
// The steps are ordinary launches by default: a cooperative launch costs
// ~18 us more per step to dispatch (405 vs 387 us per config-2 step), and
// every run under rocprofv3 that had made a cooperative launch crashed in
// exit() (cause not established; runs with ordinary launches only exit
// cleanly). Callers that share the GPU
// with other work can ask for cooperative step launches
// (gemma4_decode_step_set_cooperative), which the runtime admits only with
// all workgroups resident. Otherwise, should another kernel hold CUs during
// a step, the bounded waits give up and the error is recorded in the
// workspace header; nothing hangs.
std::atomic<int> g_cooperative{0};

hipError_t launch_step(StepParams &p, hipStream_t stream, bool walk = false) {
  void *args[] = {&p};
  const void *fn = walk ? reinterpret_cast<const void *>(decode_step_kernel<true>)
                        : reinterpret_cast<const void *>(decode_step_kernel<false>);
  if (p.probe == nullptr && g_cooperative.load(std::memory_order_relaxed) != 0) {
    return hipLaunchCooperativeKernel(fn, dim3(kStepWorkgroups), dim3(kStepThreads), args,
                                      kPadLds, stream);
  }
  return hipLaunchKernel(fn, dim3(kStepWorkgroups), dim3(kStepThreads), args, kPadLds, stream);
}

__global__ void decode_step_set_stall_kernel(int32_t *header, int32_t stall_layer_plus1,
                                             int32_t ticks) {
  if (threadIdx.x == 0) {
    header[kHeaderStallLayer] = stall_layer_plus1;
    header[kHeaderStallTicks] = ticks;
  }
}

bool step_geometry_ok(const Gemma4KvCacheConfig &c, int32_t batch_count) {
  return c.num_heads == kSHeads && c.head_dim == kSDim && c.page_size > 0 &&
         c.max_pages_per_seq > 0 && c.num_pages > 0 && c.batch_size >= batch_count;
}

}  // namespace
}  // namespace gemma4

using namespace gemma4;

extern "C" size_t gemma4_decode_step_workspace_bytes(int32_t batch_count) {
  if (batch_count < 1 || batch_count > kMaxBatch) return 0;
  return (size_t)workspace_layout(batch_count).bytes;
}

extern "C" hipError_t gemma4_decode_step_workspace_init(void *workspace, size_t workspace_bytes,
                                                        int32_t batch_count, hipStream_t stream) {
  const size_t need = gemma4_decode_step_workspace_bytes(batch_count);
  if (workspace == nullptr || need == 0 || workspace_bytes < need) return hipErrorInvalidValue;
  const WorkspaceLayout w = workspace_layout(batch_count);
  int32_t *ints = static_cast<int32_t *>(workspace);
  hipLaunchKernelGGL(decode_step_workspace_init_kernel, 256, 256, 0, stream, ints, w.int_count,
                     reinterpret_cast<uint32_t *>(ints + w.int_count), w.record_floats);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  int device = 0;
  e = hipGetDevice(&device);
  if (e != hipSuccess) return e;
  if (device < 0 || device >= 64) return hipErrorNotSupported;
  if (g_placement_ok[device].load() == 0) {
    for (const void *fn : {reinterpret_cast<const void *>(decode_step_kernel<false>),
                           reinterpret_cast<const void *>(decode_step_kernel<true>)}) {
      e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPadLds);
      if (e != hipSuccess) return e;
    }
    // One probe launch of the step kernel: every XCD must receive exactly
    // 32 of its workgroups, on 32 distinct CUs, for the XCD-local exchange.
    StepParams p = base_params(workspace, w, batch_count);
    p.probe = ints + w.probe;
    e = launch_step(p, stream);
    if (e != hipSuccess) return e;
    int32_t ids[kStepWorkgroups];
    e = hipMemcpyAsync(ids, p.probe, sizeof(ids), hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return e;
    int count[16] = {};
    bool seen[kXcds][256] = {};
    bool ok = true;
    for (int32_t id : ids) {
      const int32_t x = id & 0xff, cu = (id >> 8) & 0xff;
      if (x >= kXcds || seen[x][cu]) {
        ok = false;
        continue;
      }
      seen[x][cu] = true;
      ++count[x];
    }
    for (int x = 0; x < kXcds; ++x) ok &= count[x] == kXcdSlots;
    g_placement_ok[device].store(ok ? 1 : -1);
  }
  return g_placement_ok[device].load() == 1 ? hipSuccess : hipErrorNotSupported;
}

extern "C" hipError_t gemma4_decode_step_status(const void *workspace, int32_t *status) {
  if (workspace == nullptr || status == nullptr) return hipErrorInvalidValue;
  int32_t header[2] = {0, 0};
  const hipError_t e = hipMemcpy(header, workspace, sizeof(header), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return e;
  *status = header[kHeaderError];
  return hipSuccess;
}

extern "C" hipError_t gemma4_decode_step_status_async(const void *workspace, int32_t *status,
                                                      hipStream_t stream) {
  if (workspace == nullptr || status == nullptr) return hipErrorInvalidValue;
  return hipMemcpyAsync(status, static_cast<const int32_t *>(workspace) + kHeaderError,
                        sizeof(int32_t), hipMemcpyDefault, stream);
}

extern "C" hipError_t gemma4_decode_step_set_cooperative(int32_t enable) {
  if (enable != 0 && enable != 1) return hipErrorInvalidValue;
  g_cooperative.store(enable, std::memory_order_relaxed);
  return hipSuccess;
}

extern "C" hipError_t gemma4_decode_step_inject_stall(void *workspace, int32_t layer,
                                                      uint32_t limit_ticks, hipStream_t stream) {
  if (workspace == nullptr || layer < -1 || layer >= kNumModelLayers ||
      limit_ticks > 0x7fffffffu)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(decode_step_set_stall_kernel, 1, 64, 0, stream,
                     static_cast<int32_t *>(workspace), layer + 1, (int32_t)limit_ticks);
  return hipGetLastError();
}

namespace gemma4 {
namespace {

// Preparation inputs of a step (all null: q/k/v already prepared). Norm
// weights: [layer_count][head_dim] of each layer's geometry, back to back;
// RoPE tables per kind: [position][rotary_dim / 2].
struct StepPrep {
  const uint16_t *q_norm_w = nullptr;
  const uint16_t *k_norm_w = nullptr;
  const float *cos[2] = {nullptr, nullptr};
  const float *sin[2] = {nullptr, nullptr};
};

// Whether the persistent kernel accepts model layers [first_layer,
// first_layer + layer_count), all of them in 8 x 256 caches (no launch).
hipError_t step_check(gemma4_bf16 *const ck[2], gemma4_bf16 *const cv[2],
                      const int32_t *const pt[2], const Gemma4KvCacheConfig cfg[2],
                      int32_t first_layer, int32_t layer_count, int32_t batch_count) {
  const WorkspaceLayout w = workspace_layout(batch_count);
  bool need_kind[2] = {false, false};
  int32_t last_index[2] = {-1, -1};  // highest cache layer of each kind in use
  for (int32_t l = first_layer; l < first_layer + layer_count; ++l) {
    const int kind = (l == kNumModelLayers - 1 || (l + 1) % kGlobalPeriod == 0) ? 1 : 0;
    need_kind[kind] = true;
    last_index[kind] = gemma4_kv_cache_layer_index(l, kind == 1);
  }
  for (int kind = 0; kind < 2; ++kind) {
    if (!need_kind[kind]) continue;
    const Gemma4KvCacheConfig &c = cfg[kind];
    if (ck[kind] == nullptr || cv[kind] == nullptr || pt[kind] == nullptr ||
        !step_geometry_ok(c, batch_count) || (kind == 0) != (c.window_size > 0))
      return hipErrorInvalidValue;
    // Longest live key range a sequence can have in this cache, per split.
    const int64_t live = kind == 0 ? c.window_size : (int64_t)c.max_pages_per_seq * c.page_size;
    if ((live + w.splits - 1) / w.splits > kMaxSplitKeys) return hipErrorInvalidValue;
    const int64_t rows = (int64_t)c.num_layers * c.num_pages * c.page_size;
    if (rows * kRowElems >= (int64_t)1 << 31 || last_index[kind] >= c.num_layers)
      return hipErrorInvalidValue;
  }
  return hipSuccess;
}

// One persistent launch over model layers [first_layer, first_layer + count),
// all of them in 8 x 256 caches.
hipError_t step_run(uint16_t *out, const uint16_t *q, const uint16_t *k, const uint16_t *v,
                    gemma4_bf16 *const ck[2], gemma4_bf16 *const cv[2],
                    const int32_t *const pt[2], const Gemma4KvCacheConfig cfg[2],
                    const int32_t *seq_lengths, const int32_t *token_position,
                    int32_t first_layer, int32_t layer_count, float scale,
                    int32_t batch_count, void *workspace, hipStream_t stream,
                    const StepPrep &prep) {
  const hipError_t ok = step_check(ck, cv, pt, cfg, first_layer, layer_count, batch_count);
  if (ok != hipSuccess) return ok;
  const WorkspaceLayout w = workspace_layout(batch_count);
  StepParams p = base_params(workspace, w, batch_count);
  p.out = out;
  p.q = q;
  p.new_k = k;
  p.new_v = v;
  for (int kind = 0; kind < 2; ++kind) {
    p.cache_k[kind] = reinterpret_cast<uint16_t *>(ck[kind]);
    p.cache_v[kind] = reinterpret_cast<uint16_t *>(cv[kind]);
    p.page_table[kind] = pt[kind];
    p.c[kind] = cfg[kind];
  }
  p.seq_lengths = seq_lengths;
  p.token_position = token_position;
  p.first_layer = first_layer;
  p.layer_count = layer_count;
  p.q_scale = scale * kLog2e;
  if (prep.q_norm_w != nullptr) {
    p.q_norm_w = prep.q_norm_w;
    p.k_norm_w = prep.k_norm_w;
    for (int kind = 0; kind < 2; ++kind) {
      p.rope_cos[kind] = prep.cos[kind];
      p.rope_sin[kind] = prep.sin[kind];
    }
  }
  return launch_step(p, stream);
}

}  // namespace
}  // namespace gemma4

namespace gemma4 {
namespace {
hipError_t step_layers(
    gemma4_bf16 *out, const gemma4_bf16 *q, const gemma4_bf16 *k, const gemma4_bf16 *v,
    gemma4_bf16 *sliding_cache_k, gemma4_bf16 *sliding_cache_v,
    const int32_t *sliding_page_table, Gemma4KvCacheConfig sliding_config,
    gemma4_bf16 *global_cache_k, gemma4_bf16 *global_cache_v,
    const int32_t *global_page_table, Gemma4KvCacheConfig global_config,
    const int32_t *seq_lengths, const int32_t *token_position, int32_t first_layer,
    int32_t layer_count, float scale, int32_t batch_count, void *workspace,
    size_t workspace_bytes, hipStream_t stream, const StepPrep &prep) {
  const size_t need = gemma4_decode_step_workspace_bytes(batch_count);
  if (out == nullptr || q == nullptr || k == nullptr || v == nullptr || seq_lengths == nullptr ||
      token_position == nullptr || workspace == nullptr || need == 0 || workspace_bytes < need ||
      first_layer < 0 || layer_count < 1 || first_layer + layer_count > kNumModelLayers ||
      !(scale > 0.0f))
    return hipErrorInvalidValue;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64 ||
      g_placement_ok[device].load() != 1)
    return hipErrorNotSupported;  // gemma4_decode_step_workspace_init first
  gemma4_bf16 *const ck[2] = {sliding_cache_k, global_cache_k};
  gemma4_bf16 *const cv[2] = {sliding_cache_v, global_cache_v};
  const int32_t *const pt[2] = {sliding_page_table, global_page_table};
  const Gemma4KvCacheConfig cfg[2] = {sliding_config, global_config};
  const bool ref_global = global_config.num_heads == 1 && global_config.head_dim == kRefDim;
  auto is_global = [](int32_t l) { return l == kNumModelLayers - 1 || (l + 1) % kGlobalPeriod == 0; };
  const int32_t last = first_layer + layer_count;
  if (!ref_global) {
    return step_run(reinterpret_cast<uint16_t *>(out), reinterpret_cast<const uint16_t *>(q),
                    reinterpret_cast<const uint16_t *>(k), reinterpret_cast<const uint16_t *>(v),
                    ck, cv, pt, cfg, seq_lengths, token_position, first_layer, layer_count,
                    scale, batch_count, workspace, stream, prep);
  }
  // Reference global geometry: runs of sliding layers go to the persistent
  // kernel, each global layer to one fused append + split-K launch and the
  // combine kernel (its partials in the workspace), gated by the workspace
  // status like the persistent launches. Stream order keeps layer i after
  // layer i-1. Rows are laid out back to back,
  // layer by layer, each layer's [batch][16][head_dim] (q, out) and
  // [batch][Hk][head_dim] (k, v) at its own width.
  int32_t ref_split = 0, ref_splits = 0;
  bool have_global = false;
  for (int32_t l = first_layer; l < last; ++l) have_global |= is_global(l);
  if (have_global) {
    const Gemma4KvCacheConfig &g = global_config;
    if (g.window_size != 0 || g.batch_size < batch_count || g.max_pages_per_seq <= 0 ||
        g.page_size <= 0)
      return hipErrorInvalidValue;
    const int64_t capacity = (int64_t)g.max_pages_per_seq * g.page_size;
    if (capacity > 0x7fffffff) return hipErrorInvalidValue;
    const hipError_t e = gemma4_decode_split_plan(g, batch_count, (int32_t)capacity,
                                                  kRefTargetWorkgroups, &ref_split, &ref_splits);
    if (e != hipSuccess) return e;
    if ((int64_t)batch_count * ref_splits > kRefPartialSlots) return hipErrorInvalidValue;
  }
  // Everything is checked before the first launch, so a rejected call
  // leaves every cache and output untouched: each run of sliding layers as
  // the persistent kernel will see it, each global layer as its launch will.
  for (int32_t l = first_layer; l < last;) {
    if (is_global(l)) {
      if (global_cache_k == nullptr || global_cache_v == nullptr ||
          global_page_table == nullptr ||
          !decode_geometry_ok(global_config, gemma4_kv_cache_layer_index(l, true), batch_count,
                              ref_split, ref_splits))
        return hipErrorInvalidValue;
      ++l;
      continue;
    }
    int32_t run = 0;
    while (l + run < last && !is_global(l + run)) ++run;
    const hipError_t e = step_check(ck, cv, pt, cfg, l, run, batch_count);
    if (e != hipSuccess) return e;
    l += run;
  }
  const WorkspaceLayout w = workspace_layout(batch_count);
  int32_t *ints = static_cast<int32_t *>(workspace);
  float *ref_partials = reinterpret_cast<float *>(ints + w.int_count) + w.record_floats;
  const int64_t rows = (int64_t)batch_count * kQueryHeads;
  const uint16_t *qp = reinterpret_cast<const uint16_t *>(q);
  const uint16_t *kp = reinterpret_cast<const uint16_t *>(k);
  const uint16_t *vp = reinterpret_cast<const uint16_t *>(v);
  uint16_t *op = reinterpret_cast<uint16_t *>(out);
  StepPrep lp = prep;  // norm weights advance with the layers
  for (int32_t l = first_layer; l < last;) {
    if (is_global(l)) {
      const int64_t slots = rows * ref_splits;
      // With preparation the split kernel prepares q and the new K (V from
      // the raw K, as the 1 x 512 geometry defines it).
      const hipError_t e = decode_append_gated(
          op, ref_partials, ref_partials + slots, ref_partials + 2 * slots, qp,
          reinterpret_cast<uint16_t *>(global_cache_k),
          reinterpret_cast<uint16_t *>(global_cache_v), global_page_table, seq_lengths,
          token_position, kp, lp.q_norm_w != nullptr ? nullptr : vp, global_config,
          gemma4_kv_cache_layer_index(l, true), scale, ref_split, ref_splits, batch_count,
          ints + kHeaderError, stream, lp.q_norm_w, lp.k_norm_w, lp.cos[1], lp.sin[1]);
      if (e != hipSuccess) return e;
      qp += rows * kRefDim;
      op += rows * kRefDim;
      kp += (int64_t)batch_count * kRefDim;
      vp += (int64_t)batch_count * kRefDim;
      if (lp.q_norm_w != nullptr) {
        lp.q_norm_w += kRefDim;
        lp.k_norm_w += kRefDim;
      }
      ++l;
      continue;
    }
    int32_t run = 0;
    while (l + run < last && !is_global(l + run)) ++run;
    const hipError_t e = step_run(op, qp, kp, vp, ck, cv, pt, cfg, seq_lengths, token_position,
                                  l, run, scale, batch_count, workspace, stream, lp);
    if (e != hipSuccess) return e;
    qp += run * rows * kSDim;
    op += run * rows * kSDim;
    kp += (int64_t)run * batch_count * kRowElems;
    vp += (int64_t)run * batch_count * kRowElems;
    if (lp.q_norm_w != nullptr) {
      lp.q_norm_w += (int64_t)run * kSDim;
      lp.k_norm_w += (int64_t)run * kSDim;
    }
    l += run;
  }
  return hipSuccess;
}
}  // namespace
}  // namespace gemma4

extern "C" hipError_t gemma4_decode_step_layers_bf16(
    gemma4_bf16 *out, const gemma4_bf16 *q, const gemma4_bf16 *k, const gemma4_bf16 *v,
    gemma4_bf16 *sliding_cache_k, gemma4_bf16 *sliding_cache_v,
    const int32_t *sliding_page_table, Gemma4KvCacheConfig sliding_config,
    gemma4_bf16 *global_cache_k, gemma4_bf16 *global_cache_v,
    const int32_t *global_page_table, Gemma4KvCacheConfig global_config,
    const int32_t *seq_lengths, const int32_t *token_position, int32_t first_layer,
    int32_t layer_count, float scale, int32_t batch_count, void *workspace,
    size_t workspace_bytes, hipStream_t stream) {
  return step_layers(out, q, k, v, sliding_cache_k, sliding_cache_v, sliding_page_table,
                     sliding_config, global_cache_k, global_cache_v, global_page_table,
                     global_config, seq_lengths, token_position, first_layer, layer_count, scale,
                     batch_count, workspace, workspace_bytes, stream, StepPrep{});
}

extern "C" hipError_t gemma4_decode_step_layers_prep_bf16(
    gemma4_bf16 *out, const gemma4_bf16 *q, const gemma4_bf16 *k, const gemma4_bf16 *v,
    gemma4_bf16 *sliding_cache_k, gemma4_bf16 *sliding_cache_v,
    const int32_t *sliding_page_table, Gemma4KvCacheConfig sliding_config,
    gemma4_bf16 *global_cache_k, gemma4_bf16 *global_cache_v,
    const int32_t *global_page_table, Gemma4KvCacheConfig global_config,
    const int32_t *seq_lengths, const int32_t *token_position, const gemma4_bf16 *q_norm_weight,
    const gemma4_bf16 *k_norm_weight, const float *sliding_cos, const float *sliding_sin,
    const float *global_cos, const float *global_sin, int32_t first_layer, int32_t layer_count,
    float scale, int32_t batch_count, void *workspace, size_t workspace_bytes,
    hipStream_t stream) {
  bool has_sliding = false, has_global = false;
  for (int32_t l = first_layer; l >= 0 && l < first_layer + layer_count && l < kNumModelLayers;
       ++l) {
    const bool g = l == kNumModelLayers - 1 || (l + 1) % kGlobalPeriod == 0;
    has_global |= g;
    has_sliding |= !g;
  }
  if (q_norm_weight == nullptr || k_norm_weight == nullptr ||
      (has_sliding && (sliding_cos == nullptr || sliding_sin == nullptr)) ||
      (has_global && (global_cos == nullptr || global_sin == nullptr)))
    return hipErrorInvalidValue;
  StepPrep prep;
  prep.q_norm_w = reinterpret_cast<const uint16_t *>(q_norm_weight);
  prep.k_norm_w = reinterpret_cast<const uint16_t *>(k_norm_weight);
  prep.cos[0] = sliding_cos;
  prep.sin[0] = sliding_sin;
  prep.cos[1] = global_cos;
  prep.sin[1] = global_sin;
  return step_layers(out, q, k, v, sliding_cache_k, sliding_cache_v, sliding_page_table,
                     sliding_config, global_cache_k, global_cache_v, global_page_table,
                     global_config, seq_lengths, token_position, first_layer, layer_count, scale,
                     batch_count, workspace, workspace_bytes, stream, prep);
}

extern "C" hipError_t gemma4_decode_walk_bf16(
    gemma4_bf16 *out, const gemma4_bf16 *q, const gemma4_bf16 *k, const gemma4_bf16 *v,
    gemma4_bf16 *cache_k, gemma4_bf16 *cache_v, const int32_t *page_table,
    Gemma4KvCacheConfig config, int32_t layer, int32_t *seq_lengths, int32_t *token_position,
    int32_t steps, float scale, int32_t batch_count, void *workspace, size_t workspace_bytes,
    hipStream_t stream) {
  const size_t need = gemma4_decode_step_workspace_bytes(batch_count);
  if (out == nullptr || q == nullptr || k == nullptr || v == nullptr || cache_k == nullptr ||
      cache_v == nullptr || page_table == nullptr || seq_lengths == nullptr ||
      token_position == nullptr || workspace == nullptr || need == 0 ||
      workspace_bytes < need || steps < 1 || steps > kMaxWalkSteps || !(scale > 0.0f) ||
      !step_geometry_ok(config, batch_count) || layer < 0 || layer >= config.num_layers)
    return hipErrorInvalidValue;
  const WorkspaceLayout w = workspace_layout(batch_count);
  // Every iteration's split must fit the row tables: the window, or the
  // longest global range the cache can hold.
  const int64_t live =
      config.window_size > 0 ? config.window_size : (int64_t)config.max_pages_per_seq * config.page_size;
  if ((live + w.splits - 1) / w.splits > kMaxSplitKeys) return hipErrorInvalidValue;
  // The cache is read through buffer descriptors and the rows through
  // 32-bit byte offsets.
  const int64_t cache_bytes =
      (int64_t)config.num_layers * config.num_pages * config.page_size * kRowElems * 2;
  const int64_t io_bytes = (int64_t)steps * w.units * kSGroup * kSDim * 2;
  if (cache_bytes >= ((int64_t)1 << 31) || io_bytes >= ((int64_t)1 << 31))
    return hipErrorInvalidValue;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64 ||
      g_placement_ok[device].load() != 1)
    return hipErrorNotSupported;  // gemma4_decode_step_workspace_init first
  StepParams p = base_params(workspace, w, batch_count);
  p.out = reinterpret_cast<uint16_t *>(out);
  p.q = reinterpret_cast<const uint16_t *>(q);
  p.new_k = reinterpret_cast<const uint16_t *>(k);
  p.new_v = reinterpret_cast<const uint16_t *>(v);
  for (int kind = 0; kind < 2; ++kind) {
    p.cache_k[kind] = reinterpret_cast<uint16_t *>(cache_k);
    p.cache_v[kind] = reinterpret_cast<uint16_t *>(cache_v);
    p.page_table[kind] = page_table;
    p.c[kind] = config;
  }
  p.seq_lengths = seq_lengths;
  p.token_position = token_position;
  p.first_layer = 0;
  p.layer_count = steps;
  p.walk_layer = layer;
  p.q_scale = scale * kLog2e;
  return launch_step(p, stream, true);
}
