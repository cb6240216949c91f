// Decode and prefill attention over gemma.c's paged bf16 K/V cache,
// MI355X (gfx950) build. All entry points are extern "C", stream-ordered,
// allocate nothing, and return hipErrorInvalidValue on bad geometry or null
// pointers before any launch (the reference convention,
// src/gemma4_flash_attention_decode.cu:1121-1157).
#pragma once

#include "gemma4_kv_cache.h"

#ifdef __cplusplus
extern "C" {
#endif

// Paged split-K decode attention (flash decoding) for one cache layer.
//
// The reference removed its standalone decode entry point and keeps the
// attention as phases of a cooperative layer kernel; this signature is the
// standalone form of those phases: phase_decode_paged_grouped_split
// (src/gemma4_flash_attention_decode.cu:691-878) + phase_decode_paged_reduce
// (src/gemma4_flash_attention_decode.cu:880-977), extended from batch 1 to
// `batch_count` rows as their batch-indexed signatures allow.
//
//   d_out          [batch_count][16][head_dim] bf16
//   d_q            [batch_count][16][head_dim] bf16 (prepared Q)
//   d_seq_lengths  [batch_count] live length per sequence; the live keys are
//                  [max(0, len - window_size), len) for a sliding cache and
//                  [0, len) for a global one
//   d_page_table   [batch_size][max_pages_per_seq] physical page per ring slot
//   partials       partial_m/l [(row * num_splits + split)],
//                  partial_acc [(row * num_splits + split) * head_dim + d],
//                  row = b * 16 + q_head. Unused when num_splits == 1 (the
//                  single split writes d_out directly; may then be null).
// Split `s` covers live keys [first + s*split_size, first + (s+1)*split_size);
// splits past the live count do nothing. Supported geometries:
// (num_heads, head_dim) = (8, 256) and (1, 512); 16 query heads.
hipError_t gemma4_flash_attention_decode_paged_bf16(
    gemma4_bf16 *d_out, float *d_partial_m, float *d_partial_l,
    float *d_partial_acc, const gemma4_bf16 *d_q, const gemma4_bf16 *d_cache_k,
    const gemma4_bf16 *d_cache_v, const int32_t *d_page_table,
    const int32_t *d_seq_lengths, Gemma4KvCacheConfig config, int32_t layer,
    float softmax_scale, int32_t split_size, int32_t num_splits,
    int32_t batch_count, hipStream_t stream);

// Fused decode step: appends the current token's prepared K/V
// (d_k/d_v [batch_count][num_heads][head_dim]) at d_token_position[b] with the
// skip rules of gemma4_kv_cache_write_bf16 (token_batch[b] == b), then attends
// exactly as gemma4_flash_attention_decode_paged_bf16. One launch (two with
// the split combine); the split holding the new key reads it from d_k/d_v
// while writing it, so the result equals append-then-attend bit for bit in
// the cache and in the attention inputs. Replaces the append + attention
// phases of decode_megakernel_fused_layer_kernel
// (src/gemma4_flash_attention_decode.cu:306-375, 979-1034) without the
// RMSNorm/RoPE preparation (K/V arrive prepared).
// d_token_position[b] must be a live key of sequence b (seq_lengths[b] - 1 in
// a decode step) or a position whose slot holds no live key.
// d_split_counters: null -> a second kernel combines the splits; otherwise
// [batch_count * num_heads] int32, zero before the first call, and the last
// split workgroup of each (b, kv_head) combines in the same launch and
// re-arms its counter to zero. Calls sharing a counter array must not overlap.
hipError_t gemma4_flash_attention_append_decode_paged_bf16(
    gemma4_bf16 *d_out, float *d_partial_m, float *d_partial_l,
    float *d_partial_acc, const gemma4_bf16 *d_q, gemma4_bf16 *d_cache_k,
    gemma4_bf16 *d_cache_v, const int32_t *d_page_table,
    const int32_t *d_seq_lengths, const int32_t *d_token_position,
    const gemma4_bf16 *d_k, const gemma4_bf16 *d_v, int32_t *d_split_counters,
    Gemma4KvCacheConfig config, int32_t layer, float softmax_scale,
    int32_t split_size, int32_t num_splits, int32_t batch_count,
    hipStream_t stream);

// Allocation-free form of gemma4_flash_attention_append_decode_paged_bf16
// (no counterpart in the reference): for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc). Same arguments without the partial buffers and split
// counters; the split partials live in a fixed 40 MiB device array inside
// the library (one per GPU, held until the process ends), the combine is the
// separate kernel. Calls whose partials exceed it --
// batch_count * 16 * num_splits * (head_dim + 2) * 4 bytes > 40 MiB -- return
// hipErrorOutOfMemory before any launch. The call allocates nothing. All
// calls on one GPU share that array: calls that overlap in time on one GPU
// (different streams, or host threads) race and must not be issued.
hipError_t gemma4_flash_attention_append_decode_paged_bf16_noalloc(
    gemma4_bf16 *d_out, const gemma4_bf16 *d_q, gemma4_bf16 *d_cache_k,
    gemma4_bf16 *d_cache_v, const int32_t *d_page_table, const int32_t *d_seq_lengths,
    const int32_t *d_token_position, const gemma4_bf16 *d_k, const gemma4_bf16 *d_v,
    Gemma4KvCacheConfig config, int32_t layer, float softmax_scale, int32_t split_size,
    int32_t num_splits, int32_t batch_count, hipStream_t stream);

// Fused decode layer attention for raw projections: prepares q (learned
// RMSNorm + RoPE at d_token_position[b]) inside every split workgroup, has the
// split that owns the new key prepare its K (RMSNorm + RoPE) and V
// (scale-free RMSNorm; derived from the raw K when config.num_heads == 1,
// d_v may then be null) and write them into the cache, then attends exactly
// as gemma4_flash_attention_append_decode_paged_bf16. One launch replaces
// gemma4_decode_prep_append_bf16 followed by the append+decode call: the
// reference's fused layer phases phase_decode_q_paged_kv_norm_rope +
// split + reduce (src/gemma4_flash_attention_decode.cu:216-375, 691-977).
// d_q / d_k / d_v are the raw [batch_count][heads][head_dim] rows; cos/sin
// are [position][rotary/2] (rotary = head_dim for 8x256, head_dim/4 for
// 1x512). A sequence with d_token_position[b] < 0 appends nothing and uses
// its q as given. The prepared q is not written out.
hipError_t gemma4_flash_attention_prep_append_decode_paged_bf16(
    gemma4_bf16 *d_out, float *d_partial_m, float *d_partial_l,
    float *d_partial_acc, const gemma4_bf16 *d_q, gemma4_bf16 *d_cache_k,
    gemma4_bf16 *d_cache_v, const int32_t *d_page_table,
    const int32_t *d_seq_lengths, const int32_t *d_token_position,
    const gemma4_bf16 *d_k, const gemma4_bf16 *d_v, const gemma4_bf16 *d_q_norm_weight,
    const gemma4_bf16 *d_k_norm_weight, const float *d_cos, const float *d_sin,
    int32_t *d_split_counters, Gemma4KvCacheConfig config, int32_t layer,
    float softmax_scale, int32_t split_size, int32_t num_splits, int32_t batch_count,
    hipStream_t stream);

// The two phases of gemma4_flash_attention_decode_paged_bf16 as separate
// launches, for callers that schedule them apart (or time them): the split
// phase (phase_decode_paged_grouped_split,
// src/gemma4_flash_attention_decode.cu:691-878), with the fused append of
// gemma4_flash_attention_append_decode_paged_bf16 when d_token_position is not
// null; with num_splits == 1 it writes d_out directly. The combine phase
// (phase_decode_paged_reduce, src/gemma4_flash_attention_decode.cu:880-977)
// reduces the live splits of every (batch, query head) row into d_out.
hipError_t gemma4_flash_attention_decode_split_paged_bf16(
    gemma4_bf16 *d_out, float *d_partial_m, float *d_partial_l,
    float *d_partial_acc, const gemma4_bf16 *d_q, gemma4_bf16 *d_cache_k,
    gemma4_bf16 *d_cache_v, const int32_t *d_page_table,
    const int32_t *d_seq_lengths, const int32_t *d_token_position,
    const gemma4_bf16 *d_k, const gemma4_bf16 *d_v, Gemma4KvCacheConfig config,
    int32_t layer, float softmax_scale, int32_t split_size, int32_t num_splits,
    int32_t batch_count, hipStream_t stream);
hipError_t gemma4_flash_attention_decode_combine_bf16(
    gemma4_bf16 *d_out, const float *d_partial_m, const float *d_partial_l,
    const float *d_partial_acc, const int32_t *d_seq_lengths,
    Gemma4KvCacheConfig config, int32_t split_size, int32_t num_splits,
    int32_t batch_count, hipStream_t stream);

// Causal GQA prefill attention of a chunk of `chunk_len` new rows per
// sequence with bf16 MFMA. Chunk row r of sequence b sits at absolute position
// P_b + r, P_b = d_prior_lengths[b]; it attends to keys
// [max(0, pos - window + 1), pos] (window = config.window_size, 0 = no
// window): keys at positions >= P_b come from the chunk's own prepared
// d_k/d_v [batch][chunk_len][num_heads][head_dim], earlier keys from the paged
// cache through the page table (unmapped pages are skipped). The cache is
// only read: the caller writes the chunk afterwards
// (gemma4_kv_cache_write_prefill_bf16), as the reference writes after
// attention (src/gemma4_prefill_megakernel.cu:171-207). d_prior_lengths ==
// null means plain self-attention of the chunk (the reference launchers'
// seqlen_q == seqlen_k case) and the cache arguments are ignored.
// q/out: [batch][chunk_len][16][head_dim]. Geometry: 8 kv heads x 256.
// Replaces gemma4_flash_fwd_bf16_kernel
// (src/gemma4_flash_attention_prefill.cu:767-954) and lifts its
// seqlen_q == seqlen_k restriction (:1131, :1205).
hipError_t gemma4_flash_attention_prefill_chunk_paged_bf16(
    gemma4_bf16 *d_out, const gemma4_bf16 *d_q, const gemma4_bf16 *d_k,
    const gemma4_bf16 *d_v, const gemma4_bf16 *d_cache_k, const gemma4_bf16 *d_cache_v,
    const int32_t *d_page_table, const int32_t *d_prior_lengths, Gemma4KvCacheConfig config,
    int32_t layer, int32_t batch_size, int32_t chunk_len, float softmax_scale,
    hipStream_t stream);

// The same attention with the causal work of a global chunk (window 0, two
// or more 64-row blocks) balanced over workgroups: row blocks j and nb-1-j
// are served by two workgroups with equal key tiles, and the one block a pair
// splits is merged through d_workspace. Results equal the entry point above
// up to float summation order. d_workspace: at least
// gemma4_flash_attention_prefill_chunk_workspace_bytes(batch_size,
// chunk_len, config) bytes, 256-byte aligned, zero-filled once before its
// first use (every call leaves its arrival counters at zero again); one
// sized for the largest chunk and batch also serves every smaller call;
// calls that share a workspace must not overlap. Sliding chunks (window > 0) run
// the plain kernel and ignore the workspace. No counterpart in the
// reference, whose prefill launcher (src/gemma4_flash_attention_prefill.cu:
// 1131-1183) assigns one causal row block per block.
size_t gemma4_flash_attention_prefill_chunk_workspace_bytes(
    int32_t batch_size, int32_t chunk_len, Gemma4KvCacheConfig config);
hipError_t gemma4_flash_attention_prefill_chunk_paged_bf16_ws(
    gemma4_bf16 *d_out, const gemma4_bf16 *d_q, const gemma4_bf16 *d_k,
    const gemma4_bf16 *d_v, const gemma4_bf16 *d_cache_k, const gemma4_bf16 *d_cache_v,
    const int32_t *d_page_table, const int32_t *d_prior_lengths, Gemma4KvCacheConfig config,
    int32_t layer, int32_t batch_size, int32_t chunk_len, float softmax_scale,
    void *d_workspace, size_t workspace_bytes, hipStream_t stream);

// Prefill self-attention with Q/K/V preparation (seqlen_q == seqlen_k, no
// prior context), same names, argument order and validation as the
// reference launchers (src/gemma4_flash_attention.cuh:9-45,
// src/gemma4_flash_attention_prefill.cu:1110-1257). Row r of the
// [batch_size][seqlen_q] token rows is prepared at absolute position
// d_token_position[r] (rows with a negative position are not prepared):
// Q and K get learned RMSNorm then split-half RoPE from d_cos/d_sin
// ([position][rotary_dim/2]); V gets scale-free RMSNorm. Sliding: 8 kv heads
// x 256, RoPE over the whole head, V from d_v, causal attention within
// `window_size` keys (> 0). Global: 1 kv head x 512, RoPE over the first 128
// dims, V derived from the raw K (d_v does not exist), causal attention.
// Prepared tensors keep the attention layout: q [rows][16][D], k/v
// [rows][Hk][D]; out [rows][16][D]. The caller owns all buffers; these
// entry points have C linkage here (the reference's are C++).
hipError_t gemma4_flash_attention_sliding_fwd_bf16_norm_rope(
    gemma4_bf16 *d_out, gemma4_bf16 *d_q_prepared, gemma4_bf16 *d_k_prepared,
    gemma4_bf16 *d_v_prepared, const gemma4_bf16 *d_q, const gemma4_bf16 *d_k,
    const gemma4_bf16 *d_v, const gemma4_bf16 *d_q_norm_weight,
    const gemma4_bf16 *d_k_norm_weight, const float *d_cos, const float *d_sin,
    const int32_t *d_token_position, int batch_size, int seqlen_q, int seqlen_k, int window_size,
    float softmax_scale, hipStream_t stream);
hipError_t gemma4_flash_attention_global_fwd_bf16_norm_rope(
    gemma4_bf16 *d_out, gemma4_bf16 *d_q_prepared, gemma4_bf16 *d_k_prepared,
    gemma4_bf16 *d_v_prepared, const gemma4_bf16 *d_q, const gemma4_bf16 *d_k,
    const gemma4_bf16 *d_q_norm_weight, const gemma4_bf16 *d_k_norm_weight, const float *d_cos,
    const float *d_sin, const int32_t *d_token_position, int batch_size, int seqlen_q,
    int seqlen_k, float softmax_scale, hipStream_t stream);

// Split plan for the MI355X: the split size (a multiple of the kernel's key
// wave chunk) that gives about `target_workgroups` split workgroups (0 = default:
// one per CU for one sequence, 32 per CU for a batch) for `batch_count` sequences of up to `max_live_keys` live keys,
// and the split count that covers `max_live_keys`. With the default target,
// one sequence whose splits would hold two key tiles or fewer (a 1024-key
// sliding window) gets one-tile splits instead, up to two workgroups per CU. Replaces the fixed
// GEMMA4_SLIDING_DECODE_SPLIT_SIZE (src/gemma4.h:24) and the active split
// count of src/gemma4_decode_megakernel.cu:158-167.
hipError_t gemma4_decode_split_plan(Gemma4KvCacheConfig config,
                                    int32_t batch_count, int32_t max_live_keys,
                                    int32_t target_workgroups,
                                    int32_t *split_size, int32_t *num_splits);

// Decode-token preparation + cache append (replaces
// phase_decode_q_paged_kv_norm_rope, src/gemma4_flash_attention_decode.cu:285-375):
// for each sequence b < batch_count with token_position[b] >= 0, every query
// head of q [b][16][D] gets learned RMSNorm (q_norm_weight [D]) and split-half
// RoPE over the rotary prefix (D for the (8,256) geometry, D/4 for (1,512)),
// written to q_prepared [b][16][D]; each KV head's key [b][Hk][D] gets the
// same with k_norm_weight and is stored in the cache row of token_position[b]
// (its page's ring slot; skipped when the page is unmapped); V [b][Hk][D]
// gets scale-free RMSNorm (for (1,512), V is the scale-free norm of the raw
// key and `v` may be null). cos/sin: [position][rotary_dim/2] fp32 tables
// (the runtime state's). eps 1e-6.
hipError_t gemma4_decode_prep_append_bf16(
    gemma4_bf16 *q_prepared, gemma4_bf16 *cache_k, gemma4_bf16 *cache_v,
    Gemma4KvCacheConfig config, const int32_t *page_table, const int32_t *token_position,
    int32_t layer, const gemma4_bf16 *q, const gemma4_bf16 *k, const gemma4_bf16 *v,
    const gemma4_bf16 *q_norm_weight, const gemma4_bf16 *k_norm_weight, const float *cos,
    const float *sin, int32_t batch_count, hipStream_t stream);

// ---- persistent decode step over consecutive layers --------------------
// One persistent launch (an ordinary launch of 256 workgroups, one per CU;
// it relies on all of them being resident together, which holds while no
// other kernel occupies CUs during the step) that runs, for model layers
// first_layer .. first_layer + layer_count - 1 in order, the fused K/V
// append of the current token and the split-K decode attention with its
// combine, for `batch_count` sequences. Replaces the per-layer attention
// launches of the reference decode loop (src/gemma4_decode_megakernel.cu:172-183
// -> gemma4_decode_megakernel_flash_attention_layer_bf16, append + attention
// phases src/gemma4_flash_attention_decode.cu:979-1067).
//   Sliding layers use the sliding cache/config/page table, global layers
//   (every 6th and the last) the global ones. Sliding geometry: 8 KV heads
//   x 256. Global geometry: 8 x 256 (all layers then run in the persistent
//   launch), or the reference model's 1 KV head x 512 (src/gemma4.h:17-21):
//   then each run of sliding layers is one persistent launch and each global
//   layer one fused append + split-K launch with its combine, all in stream
//   order (16 launches for 48 layers).
//   q, out / k, v (the appended rows): the layers' rows back to back, layer
//   by layer, each layer's [batch_count][16][head_dim] (q, out) and
//   [batch_count][num_heads][head_dim] (k, v) at its own geometry; with 8 x
//   256 everywhere that is [layer_count][batch_count][16 or 8][256]. Layer i
//   reads its q/k/v only after layer i-1's output is complete (the order a
//   real decode step imposes). seq_lengths / token_position: as for the
//   per-layer entry points (one step: the same for every layer).
// `workspace` (gemma4_decode_step_workspace_bytes bytes) holds the split
// records and layer flags; initialise it once with
// gemma4_decode_step_workspace_init (which also checks, once per device,
// that the workgroups land one per CU, 32 per XCD; hipErrorNotSupported
// otherwise), then reuse it for every step (stream order). Calls sharing a
// workspace must not overlap.
// Failure is stream-ordered and sticky: every wait of the step is bounded
// (0.2 s); if one gives up (another kernel held CUs), the launch writes
// zeros for the output chunks whose wait gave up and records a nonzero
// status in the workspace; every later launch on that workspace (with the
// 1 x 512 global geometry also the global layers' launches) then writes
// zeros to all of its outputs, appends nothing and returns at once, until
// gemma4_decode_step_workspace_init is called again. Status codes: 0 ok, 1 a
// wait gave up, 2 a split exceeded the 512-key row table.
// gemma4_decode_step_status reads it synchronously;
// gemma4_decode_step_status_async copies it (4 bytes) to `status` (host
// pinned or device memory) in stream order.
size_t gemma4_decode_step_workspace_bytes(int32_t batch_count);
hipError_t gemma4_decode_step_workspace_init(void *workspace, size_t workspace_bytes,
                                             int32_t batch_count, hipStream_t stream);
hipError_t gemma4_decode_step_status(const void *workspace, int32_t *status);
hipError_t gemma4_decode_step_status_async(const void *workspace, int32_t *status,
                                           hipStream_t stream);
// Process-wide launch mode of the persistent step (no counterpart in the
// reference): 0 (default) ordinary launches; 1 cooperative launches, which
// the runtime admits only with all 256 workgroups resident -- for callers
// that share the GPU with other kernels -- at ~18 us more dispatch cost per
// step. Do not run a process that makes cooperative step launches under
// rocprofv3: every profiled run that made a cooperative launch crashed with
// SIGSEGV in exit() after the profiler had written its files; the cause of
// that crash has not been established, and ordinary launches avoid it.
hipError_t gemma4_decode_step_set_cooperative(int32_t enable);
// Fault injection for tests (no counterpart in the reference): from the next
// launch on, at launch-relative layer `layer` one workgroup waits for a
// workspace word that is never set, giving up after `limit_ticks` of the
// 100 MHz real-time clock, so a failed step can be produced without holding
// CUs. layer -1 switches it off; workspace_init clears it.
hipError_t gemma4_decode_step_inject_stall(void *workspace, int32_t layer,
                                           uint32_t limit_ticks, hipStream_t stream);
hipError_t gemma4_decode_step_layers_bf16(
    gemma4_bf16 *out, const gemma4_bf16 *q, const gemma4_bf16 *k, const gemma4_bf16 *v,
    gemma4_bf16 *sliding_cache_k, gemma4_bf16 *sliding_cache_v,
    const int32_t *sliding_page_table, Gemma4KvCacheConfig sliding_config,
    gemma4_bf16 *global_cache_k, gemma4_bf16 *global_cache_v,
    const int32_t *global_page_table, Gemma4KvCacheConfig global_config,
    const int32_t *seq_lengths, const int32_t *token_position, int32_t first_layer,
    int32_t layer_count, float scale, int32_t batch_count, void *workspace,
    size_t workspace_bytes, hipStream_t stream);

// The same step from the layers' raw projections, as the reference's fused
// decode layer takes them (src/gemma4_flash_attention_decode.cu:216-375,
// 1036-1067: per-head Q/K RMSNorm with learned weights, split-half RoPE at
// the token's position, scale-free RMSNorm of V, then append + attention).
// q, k, v: raw rows in the layout above. q_norm_weight, k_norm_weight: each
// launch layer's weights back to back ([layer_count][head_dim] at each
// layer's geometry). RoPE tables [position][rotary_dim / 2] fp32: sliding
// layers use sliding_cos/sin (rotary over all 256 dims), global layers
// global_cos/sin (8 x 256: all 256 dims; 1 x 512: the first 128 dims, the
// runtime state's global tables; there V is derived from the raw K and `v`'s
// global rows are not read). A prepared value can differ from the reference
// per-head preparation by one bf16 ulp (the sum of squares is reduced in
// another order). Otherwise as gemma4_decode_step_layers_bf16;
// the tables of a kind that the layer range does not use may be null.
hipError_t gemma4_decode_step_layers_prep_bf16(
    gemma4_bf16 *out, const gemma4_bf16 *q, const gemma4_bf16 *k, const gemma4_bf16 *v,
    gemma4_bf16 *sliding_cache_k, gemma4_bf16 *sliding_cache_v,
    const int32_t *sliding_page_table, Gemma4KvCacheConfig sliding_config,
    gemma4_bf16 *global_cache_k, gemma4_bf16 *global_cache_v,
    const int32_t *global_page_table, Gemma4KvCacheConfig global_config,
    const int32_t *seq_lengths, const int32_t *token_position, const gemma4_bf16 *q_norm_weight,
    const gemma4_bf16 *k_norm_weight, const float *sliding_cos, const float *sliding_sin,
    const float *global_cos, const float *global_sin, int32_t first_layer, int32_t layer_count,
    float scale, int32_t batch_count, void *workspace, size_t workspace_bytes,
    hipStream_t stream);

// ---- persistent walk over decode steps of one layer ----------------------
// `steps` consecutive decode steps of one 8 x 256 cache layer in one
// persistent launch (the same kernel, placement and workspace as the step
// above): step s appends token s of every sequence at position
// seq_lengths[b] + s and attends over its seq_lengths[b] + s + 1 keys, the
// window's last ones for a sliding cache. This is the reference's per-step
// loop for one layer (src/gemma4_decode_megakernel.cu:172-183 preparing
// each step with gemma4_runtime_prepare_decode_step,
// src/gemma4_runtime.cu:276-341) without a launch per step; step s reads its
// q/k/v only after step s-1's output is complete.
//   q, out: [steps][batch_count][16][256]; k, v: [steps][batch_count][8][256].
//   seq_lengths: device lengths before the walk (the runtime's current
//   ones); the page table must map every position the walk appends
//   (gemma4_runtime_prepare_decode_walk does both). On completion, in stream
//   order, seq_lengths and token_position hold the last step's values, as
//   after that many gemma4_runtime_prepare_decode_step calls.
// steps <= 65535; cache (one of K/V) and q under 2 GiB. Workspace, status and
// failure semantics as for gemma4_decode_step_layers_bf16.
hipError_t gemma4_decode_walk_bf16(
    gemma4_bf16 *out, const gemma4_bf16 *q, const gemma4_bf16 *k, const gemma4_bf16 *v,
    gemma4_bf16 *cache_k, gemma4_bf16 *cache_v, const int32_t *page_table,
    Gemma4KvCacheConfig config, int32_t layer, int32_t *seq_lengths, int32_t *token_position,
    int32_t steps, float scale, int32_t batch_count, void *workspace, size_t workspace_bytes,
    hipStream_t stream);

#ifdef __cplusplus
}  // extern "C"
#endif
