/*
 * ftmoe -- C ABI of the MI355X (gfx950) fused MoE-layer hot path.
 *
 * Every entry point:
 *   - is extern "C", takes plain pointers and sizes (device pointers unless
 *     stated), and runs asynchronously on the given HIP stream (NULL = the
 *     default stream); none synchronises the host and none allocates device
 *     memory -- scratch comes from a caller-provided workspace whose size is
 *     reported by the matching *_workspace() query;
 *   - returns FTMOE_OK (0) or a negative ftmoe_status; the message of the last
 *     failure on the calling thread is available from ftmoe_last_error();
 *   - uses fixed shapes and no host reads of device data, so it can be captured
 *     in a HIP graph;
 *   - takes M = 0 tokens (an empty batch, whose tensors may have NULL data
 *     pointers) as a no-op that returns FTMOE_OK without reading any pointer
 *     (routers and expert calls); M < 0 is FTMOE_ERR_INVALID.
 *
 * Number formats: bf16 is passed as uint16 bit patterns; fp8 is OCP e4m3fn;
 * fp4 is OCP e2m1 packed two per byte, low nibble = even k; e8m0 scale codes
 * decode to 2^(code-127).
 *
 * Reference interfaces (paths relative to python/freetoken/ of FreeToken) are
 * cited on each declaration.
 */
#ifndef FTMOE_H
#define FTMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* ftmoe_stream_t; /* == hipStream_t */

enum ftmoe_status {
  FTMOE_OK = 0,
  FTMOE_ERR_INVALID = -1,     /* bad argument (null pointer, shape mismatch) */
  FTMOE_ERR_UNSUPPORTED = -2, /* valid but unsupported shape or format */
  FTMOE_ERR_HIP = -3,         /* a HIP runtime call failed */
  FTMOE_ERR_WORKSPACE = -4,   /* workspace smaller than *_workspace() */
  FTMOE_ERR_BUSY = -5,        /* the object is still referenced (captured graphs) */
  FTMOE_ERR_TIMEOUT = -6      /* a watchdog found no progress; the object is unhealthy */
};

enum ftmoe_dtype { FTMOE_DTYPE_F32 = 0, FTMOE_DTYPE_BF16 = 1 };

enum ftmoe_format {
  FTMOE_FMT_NONE = -1,
  FTMOE_FMT_BF16 = 0,     /* bf16 weights */
  FTMOE_FMT_FP8_B128 = 1, /* e4m3 weights + float32 128x128 block scales */
  FTMOE_FMT_MXFP4 = 2     /* e2m1 weights + e8m0 scale per 32 K (row-major "ds_fp4" layout) */
};

enum ftmoe_activation { FTMOE_ACT_SILU = 0, FTMOE_ACT_GELU = 1, FTMOE_ACT_GELU_TANH = 2 };

/* Indices of the int64 counters accumulated by ftmoe_slot_map (moe/offload_cache.py:205-229). */
enum ftmoe_stat { FTMOE_STAT_ACTIVE = 0, FTMOE_STAT_MISS = 1, FTMOE_STAT_CALLS = 2, FTMOE_STAT_MISSED_ROUTES = 3 };

/* One expert bank: S rows (experts, or expert-cache slots), each a SwiGLU MLP.
 * Layouts follow layers/moe.py:60-92 and kernel/triton/dsv4/fused_moe.py:10-14:
 *   gate_up [S, 2I, H] (gate rows [0,I), up rows [I,2I)), down [S, H, I];
 *   FP8_B128: gate_up_scale float [S, 2I/128, H/128], down_scale float [S, H/128, I/128];
 *   MXFP4:    gate_up [S, 2I, H/2] bytes, gate_up_scale uint8 [S, 2I, H/32],
 *             down [S, H, I/2] bytes, down_scale uint8 [S, H, I/32];
 *   BF16:     scales NULL.
 * H and I must be multiples of 128. */
typedef struct ftmoe_bank {
  int format;
  int num_rows;
  int hidden;
  int inter;
  const void* gate_up;
  const void* gate_up_scale;
  const void* down;
  const void* down_scale;
  /* > 0: clamped SwiGLU, act = silu(min(gate, L)) * clamp(up, -L, L) on the
   * bf16 gate and up values (DeepSeek-V4's ds_fp4 experts and shared expert,
   * moe/fused_ds_fp4.py:105-124,192-226, kernel/triton/dsv4/fused_moe.py:121-141);
   * 0: no clamp.  Finite and >= 0; > 0 needs the silu activation. */
  float swiglu_limit;
} ftmoe_bank;

const char* ftmoe_last_error(void);
int ftmoe_version(void);

/* Softmax top-k router; replaces fused_topk (moe/fused.py:38-85, torch fallback
 * :16-35).  logits [M,E] float32 or bf16 (logits_dtype); selection on the fp32
 * logits, ties to the lower expert index; with renormalize the k weights are
 * the softmax over the selected logits, else the softmax over all E.
 * Writes topk_w float32 [M,k] and topk_ids int32 [M,k] in rank order.
 * E <= 1024, k <= min(E, 64). */
int ftmoe_route_softmax_topk(const void* logits, int logits_dtype, int M, int E, int k, int renormalize,
                             float* topk_w, int32_t* topk_ids, ftmoe_stream_t stream);

/* DeepSeek-V3 grouped sigmoid router; replaces Glm4MoeSparseBlock._route /
 * _group_limited (models/glm4_moe/moe.py:53-75).  logits float32 [M,E]; bias
 * float32 [E] or NULL; E % n_group == 0, n_group <= 64, E <= 1024. */
int ftmoe_route_grouped_sigmoid(const float* logits, const float* bias, int M, int E, int n_group, int topk_group,
                                int k, int renormalize, float routed_scaling_factor, float* topk_w,
                                int32_t* topk_ids, ftmoe_stream_t stream);

/* Buffer sizes of ftmoe_align (moe/fused.py:139-147). */
void ftmoe_align_sizes(int numel, int num_experts, int block_size, int* max_num_tokens_padded,
                       int* max_num_m_blocks);

/* moe_align_block_size (moe/fused.py:88-158; kernel/triton/moe_align.py:216-325)
 * with the canonical stable order (ascending flat route index inside each
 * expert).  sorted_ids [max_num_tokens_padded] (sentinel numel in unused
 * slots), expert_ids [max_num_m_blocks] (-1 for unused blocks),
 * num_tokens_post_pad [1].  num_experts <= 1023. */
int ftmoe_align(const int32_t* topk_ids, int numel, int num_experts, int block_size, int32_t* sorted_ids,
                int32_t* expert_ids, int32_t* num_tokens_post_pad, ftmoe_stream_t stream);

/* Expert-cache indirection: slot_ids[i] = slot_for_id[topk_ids[i]] (-1 when the
 * expert is not resident or the id is out of range); replaces the id -> slot
 * rewrite of OffloadMoeCache.ensure_experts (moe/offload_cache.py:800-810,
 * moe/offload_kernels.py:185-188) without admission.  slot_ids may alias
 * topk_ids (in-place rewrite).  miss_mask (nullable) [numel] = 1 where the
 * route missed.  stats (nullable) int64 [4] is ACCUMULATED:
 * active distinct experts, missing distinct experts, calls, missed routes. */
int ftmoe_slot_map(const int32_t* topk_ids, int numel, const int32_t* slot_for_id, int num_experts,
                   int32_t* slot_ids, uint8_t* miss_mask, int64_t* stats, ftmoe_stream_t stream);

/* Routing histogram of one layer's decode step: freq[e] += the number of
 * entries of topk_ids equal to e, ids outside [0, num_experts) skipped
 * (int64 freq [num_experts], accumulated, never cleared here); replaces the
 * opt-in decode_freq scatter of OffloadMoeCache.ensure_experts
 * (moe/offload_cache.py:234-236,803-807), run on the raw expert ids before
 * they are rewritten to slots.  Device-side and graph-capturable, so the
 * histogram also accumulates in replayed decode steps.  num_experts <= 16384. */
int ftmoe_route_histogram(const int32_t* topk_ids, int numel, int num_experts, int64_t* freq, ftmoe_stream_t stream);

/* Expert-cache admission (the miss path of OffloadMoeCache.ensure_experts):
 * replaces lru_ensure / ensure_experts (moe/offload_kernels.py:19-40) and the
 * capped admission of ensure_experts_hybrid with the "lowest_id" or
 * "recency" order (offload_kernels.py:43-60), following their CPU mirror
 * (offload_kernels.py:128-188).  One call:
 *   step += 1; the distinct ids of expert_ids are seen; resident seen experts
 *   get usage[slot] = step; missing seen experts are ordered by ascending id,
 *   or, with recency (nullable, int64 [num_experts] of this layer), by most
 *   recent first then ascending id; the first min(misses, cap, capacity) of
 *   them take, one after the other, the slot with the
 *   smallest (usage, slot) -- its previous owner, of any layer, is unmapped
 *   -- and are listed in evict_slots / src_indices (layer-local rows), at
 *   most as many as there are slots with usage < step after the touch (no
 *   slot is taken twice, and no slot of an expert of this call is taken: the
 *   exclusion of the reference's GPU kernel, offload_kernels.py:369-387);
 *   recency of every seen expert = step; expert_ids are rewritten in place to
 *   slots (-1 for unfetched misses and ids outside [0, num_experts)).
 *   cap = max_fetch (< 0: no cap); with fetch_frac_q16 in (0, 65536] (the
 *   hybrid_fetch_fraction f of offload_cache.py:131-136 in Q16) it is instead
 *   the n in {floor(m f), floor(m f) + 1} with the smaller max(n (1 - f),
 *   (m - n) f), lower n on a tie (offload_kernels.py:160-164), m the misses.
 *   cpu_ids (nullable) int32 [numel] receives, per route, the expert id of
 *   an unfetched miss and -1 elsewhere: the routes the hybrid decode gives
 *   the CPU (layers/moe.py:350-352).
 *   slot_for_id int32 [num_layers * num_experts] (row layer_id is this layer),
 *   id_of_slot int32 [cache_size] (flat ids, -1 empty), usage int64
 *   [cache_size], step int64 [1]; num_indices / num_missing int32 [1] receive
 *   the admitted and the missing counts; stats (nullable) int64 [4] is
 *   accumulated as in ftmoe_slot_map, counted before admission; unserved
 *   (nullable) int64 [1] accumulates the misses the cap admitted but no free
 *   slot (or staging entry) could take -- nonzero means the cache is smaller
 *   than a call's distinct experts.
 * num_experts, cache_size <= 8192. */
int ftmoe_lru_ensure(int32_t* expert_ids, int numel, int layer_id, int num_layers, int num_experts,
                     int32_t* slot_for_id, int32_t* id_of_slot, int64_t* usage, int64_t* step, int cache_size,
                     int64_t* recency, int max_fetch, int fetch_frac_q16, int32_t* evict_slots,
                     int32_t* src_indices, int capacity, int32_t* num_indices, int32_t* num_missing,
                     int32_t* cpu_ids, int64_t* stats, int64_t* unserved, ftmoe_stream_t stream);

/* Exact-size pinned host memory (hipHostMalloc), for the host expert banks:
 * replaces alloc_pinned_tensor (kernel/pinned.py:42-45).  torch's pinned
 * allocator rounds every request up to a power of two, which for multi-GB
 * expert layers nearly doubles the pinned footprint. */
int ftmoe_host_alloc(size_t bytes, void** ptr);
int ftmoe_host_free(void* ptr);

/* Whole-layer placement of the prefill movement: replaces materialize_layer
 * (moe/offload_cache.py:833-838, _materialize_layer_kernel,
 * moe/offload_kernels.py:250-281).  Expert e of layer_id goes to slot e:
 * slots holding this layer's experts are emptied (usage 0); other layers'
 * experts in slots [0, num_experts) lose their mapping; step += 1; slots
 * [0, num_experts) map to the layer with usage = step; evict_slots /
 * src_indices (int32 [num_experts]) = 0..E-1 and num_indices = E, the
 * entries of a following ftmoe_fetch_experts.  cache_size >= num_experts. */
int ftmoe_materialize_layer(int layer_id, int num_layers, int num_experts, int32_t* slot_for_id, int32_t* id_of_slot,
                            int64_t* usage, int64_t* step, int cache_size, int32_t* evict_slots,
                            int32_t* src_indices, int32_t* num_indices, ftmoe_stream_t stream);

/* Release of slots [slot_begin, slot_end): replaces the prefill double
 * buffer's _invalidate_prefill_buffer (moe/offload_cache.py:592-600): the
 * experts held there lose their mapping; the slots become empty, usage 0. */
int ftmoe_release_slots(int slot_begin, int slot_end, int num_layers, int num_experts, int32_t* slot_for_id,
                        int32_t* id_of_slot, int64_t* usage, int cache_size, ftmoe_stream_t stream);

/* Hit compaction of the prefill double buffer's hit/miss split: replaces
 * prefill_hit_compact (moe/offload_kernels.py:63-86, used by _prefetch_split,
 * moe/offload_cache.py:703-773).  Lists the experts e of one layer whose
 * slot (slot_for_id_row[e], int32 [num_experts]) is >= threshold -- resident
 * outside the buffers, which own the slots below -- in ascending e as
 * dst_rows[i] = dst_base + e (the buffer row) and src_rows[i] = the slot
 * (int32 [num_experts] each), and *num_hits (int32) = their count: the
 * entries of an ftmoe_fetch_experts gather from the slot banks into the
 * buffer, device to device.  num_experts <= 8192. */
int ftmoe_prefill_hit_compact(const int32_t* slot_for_id_row, int num_experts, int threshold, int dst_base,
                              int32_t* dst_rows, int32_t* src_rows, int32_t* num_hits, ftmoe_stream_t stream);

/* One bank of the gather below: this layer's expert rows in pinned host
 * memory ([num_experts, row_bytes]) and the slot bank ([cache_size,
 * row_bytes]) on the device.  host_rows may be device memory instead (the
 * slot bank itself, for the prefill hit gather). */
typedef struct ftmoe_fetch_bank {
  const void* host_rows;
  void* slot_bank;
  size_t row_bytes; /* multiple of 16; pointers 16-byte aligned */
} ftmoe_fetch_bank;

/* Copies, for i < *num_indices (a device value, at most max_entries), row
 * src_indices[i] of every bank's host rows into row evict_slots[i] of its slot
 * bank; replaces copy_missing / fast_index_copy_multi (moe/offload_cache.py:
 * 968-1010, kernel/csrc/jit/fast_index_copy.cuh:486-562).  The host memory is
 * read in place by the GPU (pinned memory from hipHostMalloc); no host
 * synchronisation, graph-capturable.  nbanks <= 8. */
int ftmoe_fetch_experts(const ftmoe_fetch_bank* banks, int nbanks, const int32_t* evict_slots,
                        const int32_t* src_indices, const int32_t* num_indices, int max_entries,
                        ftmoe_stream_t stream);

/* Per-token per-128-group FP8 activation quantisation; replaces
 * per_token_group_quant_fp8 (kernel/triton/fp8_block_linear.py:38-82, mode 0:
 * float32 scale amax/448) and the DSV4 act_quant with power-of-two scales
 * (kernel/triton/dsv4/fp8_linear.py:54-80, mode 1: uint8 e8m0 codes).
 * x bf16 [rows, K]; q e4m3 [rows, K]; scales [rows, K/128]; K % 128 == 0. */
int ftmoe_act_quant_fp8(const void* x, int rows, int K, int mode, void* q, void* scales, ftmoe_stream_t stream);

/* Decode (W8A16 / W4A16 / bf16) expert computation for a precomputed routing;
 * replaces fused_experts_decode_impl (moe/fused.py:340-423),
 * fused_experts_decode_fp8_block (moe/fused_fp8_block.py:32-44) and
 * routed_experts_fp4 (moe/fused_ds_fp4.py:97-132, without the DSV4 FP8
 * activation round trip), plus the shared-expert add of the model block
 * (models/glm4_moe/moe.py:81-82).
 *   x bf16 [M,H]; topk_w float32 [M,k]; topk_ids int32 [M,k] index bank rows
 *   (ids outside [0, num_rows) are skipped); shared: nullable bank with
 *   num_rows == 1 whose output is added; y bf16 [M,H] (may not alias x).
 * apply_router_weight_on_input scales the gate_up outputs instead of the
 * down outputs (moe/fused.py:240).
 * num_rows <= 16383 (an expert cache's slots); above 1023 rows a call holds
 * at most 16384 routes (M * k). */
size_t ftmoe_experts_decode_workspace(int M, int top_k, const ftmoe_bank* bank, const ftmoe_bank* shared);
int ftmoe_experts_decode(const void* x, int M, int top_k, const float* topk_w, const int32_t* topk_ids,
                         const ftmoe_bank* bank, const ftmoe_bank* shared, int activation,
                         int apply_router_weight_on_input, void* y, void* workspace, size_t workspace_bytes,
                         ftmoe_stream_t stream);

/* Decode that allocates nothing: ftmoe_experts_decode with its workspace in a
 * static device array of ftmoe_experts_decode_noalloc_capacity() bytes
 * (64 MiB: C4-shaped decode -- H 7168, I 2048, top-8, shared expert -- up to
 * batch 256), which each GPU the library runs on holds until the process
 * ends.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as
 * ftmoe_experts_decode without the workspace; a call whose workspace would
 * exceed the array fails with FTMOE_ERR_WORKSPACE before any launch.  stream
 * must belong to the current device.  Every call on a GPU shares that GPU's
 * array (nothing in it needs clearing between calls): calls that overlap on
 * one GPU -- on different streams, or from different host threads -- race and
 * must be serialised by the caller.  The first call on a device looks up the
 * array's address there and must run outside graph capture (refused with
 * FTMOE_ERR_UNSUPPORTED under capture); later calls can be captured and
 * replayed. */
size_t ftmoe_experts_decode_noalloc_capacity(void);
int ftmoe_experts_decode_noalloc(const void* x, int M, int top_k, const float* topk_w, const int32_t* topk_ids,
                                 const ftmoe_bank* bank, const ftmoe_bank* shared, int activation,
                                 int apply_router_weight_on_input, void* y, ftmoe_stream_t stream);

/* Decode over an expert-slot cache in one call: the id -> slot rewrite of
 * OffloadMoeCache.ensure_experts (moe/offload_cache.py:800-810, as
 * ftmoe_slot_map: slot_ids[i] = slot_for_id[topk_ids[i]], -1 when absent or
 * out of range, optional miss_mask and accumulated stats) followed by
 * OffloadMoELayer.routed_forward (layers/moe.py:234-252) on the slot bank.
 * The lookup rides in the permutation step, saving a launch per layer.
 *   topk_ids: expert ids in [0, num_experts); slot_ids: int32 [M,k] out (may
 *   alias topk_ids); bank rows are slots.  Workspace as ftmoe_experts_decode. */
int ftmoe_experts_decode_cached(const void* x, int M, int top_k, const float* topk_w, const int32_t* topk_ids,
                                const int32_t* slot_for_id, int num_experts, int32_t* slot_ids, uint8_t* miss_mask,
                                int64_t* stats, const ftmoe_bank* bank, const ftmoe_bank* shared, int activation,
                                int apply_router_weight_on_input, void* y, void* workspace, size_t workspace_bytes,
                                ftmoe_stream_t stream);

/* A router for ftmoe_experts_decode_routed. */
enum { FTMOE_ROUTER_SOFTMAX_TOPK = 0, FTMOE_ROUTER_GROUPED_SIGMOID = 1 };
typedef struct ftmoe_router {
  int kind;                    /* FTMOE_ROUTER_* */
  const void* logits;          /* [M, num_experts]; float32, or bf16 for the softmax router */
  int logits_dtype;            /* FTMOE_DTYPE_F32 / FTMOE_DTYPE_BF16 */
  int num_experts;             /* E of the router (logit columns) */
  int renormalize;
  const float* bias;           /* grouped sigmoid: nullable [E] selection bias */
  int n_group, topk_group;     /* grouped sigmoid */
  float routed_scaling_factor; /* grouped sigmoid */
} ftmoe_router;

/* Decode from router logits in one call: the router (as
 * ftmoe_route_softmax_topk or ftmoe_route_grouped_sigmoid, writing topk_w /
 * topk_ids) followed by ftmoe_experts_decode, or, with slot_for_id (nullable),
 * by ftmoe_experts_decode_cached; replaces MoELayer.forward's decode path
 * (fused_topk + experts, layers/moe.py:166-194, moe/fused.py:16-85) and the
 * DeepSeek-V3 block's _route + routed_forward (models/glm4_moe/moe.py:53-83).
 * For decode-sized calls (at most 16 tokens and 64 routes) the router and the
 * permutation share one launch.  Workspace as ftmoe_experts_decode. */
int ftmoe_experts_decode_routed(const void* x, int M, int top_k, const ftmoe_router* router, float* topk_w,
                                int32_t* topk_ids, const int32_t* slot_for_id, int num_experts, int32_t* slot_ids,
                                uint8_t* miss_mask, int64_t* stats, const ftmoe_bank* bank, const ftmoe_bank* shared,
                                int activation, int apply_router_weight_on_input, void* y, void* workspace,
                                size_t workspace_bytes, ftmoe_stream_t stream);

/* Prefill (grouped GEMM) expert computation for a precomputed routing;
 * replaces fused_experts_fp8_block (moe/fused_fp8_block.py:16-29 ->
 * kernel/triton/fp8_blockscale_moe.py:218-256, W8A8 with per-token per-128
 * activation scales), routed_experts_fp4_prefill (moe/fused_ds_fp4.py:181-235,
 * FP8-round-tripped activations with power-of-two scales) and the bf16
 * fused_experts_impl (moe/fused.py:233-337), plus the shared-expert add.
 * Same tensor conventions as ftmoe_experts_decode; the shared expert (nullable)
 * must have the routed format and intermediate size.  Router weights always
 * scale the down outputs. */
size_t ftmoe_experts_prefill_workspace(int M, int top_k, const ftmoe_bank* bank, const ftmoe_bank* shared);
int ftmoe_experts_prefill(const void* x, int M, int top_k, const float* topk_w, const int32_t* topk_ids,
                          const ftmoe_bank* bank, const ftmoe_bank* shared, int activation, void* y,
                          void* workspace, size_t workspace_bytes, ftmoe_stream_t stream);

/* Host-side expert executor of the hybrid decode (CPU pool computing the
 * routes whose experts are on the host; replaces the CPU MoE executor of the
 * hybrid backend, moe/cpu_executor.py:538-600 and
 * kernel/csrc/cpu_moe/cpu_moe_ext.cpp:1574-1668, run beside the GPU as in
 * layers/moe.py:325-372).  Banks are ftmoe_bank with HOST pointers (bf16,
 * FP8 128x128, MXFP4 as on the device).  x bf16 [M,H], w float32 [M,k], ids
 * int32 [M,k] bank rows (< 0 or >= num_rows skipped), y bf16 [M,H] =
 * bf16(sum over the token's routes, in route order, of bf16(w * expert(x))),
 * expert rounding as ftmoe_experts_decode; tokens without routes get 0.
 * threads <= 0: one per hardware thread. */
typedef struct ftmoe_cpu_executor ftmoe_cpu_executor;
ftmoe_cpu_executor* ftmoe_cpu_executor_create(int threads);
/* Waits for queued jobs and frees the executor.  Refused (FTMOE_ERR_BUSY,
 * nothing freed) while jobs captured into graphs exist, unless
 * graphs_released says that every such graph is destroyed: a replay would
 * run their host functions against the freed executor.  Also refused, at
 * once, when the watchdog abandoned a job that the pool is still computing
 * (a wedged pool: its threads cannot be joined); the caller keeps the handle
 * for the life of the process.  The stream work of the executor's calls
 * (host functions, or the flag handshake's stream writes and waits on its
 * pinned flag words, which are freed here) must have completed: synchronise
 * the streams first. */
int ftmoe_cpu_executor_destroy(ftmoe_cpu_executor* ex, int graphs_released);
const char* ftmoe_cpu_executor_isa(ftmoe_cpu_executor* ex);
/* Watchdog (replaces the flag watchdog of moe/cpu_executor.py:602-656): a
 * wait for a job (the stream's wait host function, or a synchronous run) that
 * sees neither the job done nor any progress of the pool (a work unit or a
 * job completed) for the watchdog period fails the job and every queued one,
 * returns (so the stream is not blocked for ever), and marks the executor
 * unhealthy for good: later jobs fail at once.  Their outputs are not
 * written; callers check ftmoe_cpu_executor_healthy once per step (0 =
 * healthy, FTMOE_ERR_TIMEOUT after the watchdog fired).  The period is
 * FTMOE_CPU_WATCHDOG_S seconds (default 10; 0 turns the watchdog off) or
 * set_watchdog's milliseconds.  A job abandoned while the pool computes it
 * takes no further work units and writes no more rows of its y.  hold 1 keeps
 * the driver from starting jobs; hold 2 lets the driver take its next job and
 * stall inside it until hold 0 (maintenance; tests force a stalled or wedged
 * pool with them). */
int ftmoe_cpu_executor_healthy(ftmoe_cpu_executor* ex);
/* Handshake of the stream-ordered entry points (_submit / _wait): mode 0 (the
 * default) host functions; mode 1 stream memory operations -- _submit
 * enqueues hipStreamWriteValue64 of the job's "ready" flag (mapped pinned
 * memory), a coordinator thread of the executor polls the flags and hands a
 * ready job to the pool, the pool raises the job's "done" flag, and _wait
 * enqueues hipStreamWaitValue64 on it plus its reset: no host-function round
 * trip per call (replaces the flag handshake of moe/cpu_executor.py:32-50,
 * cpu_moe_ext.cpp:560-657).  Mode 1 is taken after a functional probe on a
 * private stream of the current device; FTMOE_ERR_UNSUPPORTED (host functions
 * kept) when it fails.  Under graph capture the flags are used only when the
 * probe also captured and replayed them.  The watchdog covers flag jobs too:
 * a job without pool progress for the period is failed and its done flag
 * raised, so no stream waits for ever.  ftmoe_cpu_executor_handshake returns
 * 0 (host functions), 1 (flags, eager calls) or 2 (flags, also captured). */
int ftmoe_cpu_executor_set_handshake(ftmoe_cpu_executor* ex, int mode);
int ftmoe_cpu_executor_handshake(ftmoe_cpu_executor* ex);
void ftmoe_cpu_executor_set_watchdog(ftmoe_cpu_executor* ex, int ms);
void ftmoe_cpu_executor_hold(ftmoe_cpu_executor* ex, int hold);
/* Synchronous run on the calling thread's behalf (FTMOE_ERR_TIMEOUT when the
 * watchdog fired). */
int ftmoe_cpu_experts(ftmoe_cpu_executor* ex, const ftmoe_bank* host_bank, const void* x, const float* w,
                      const int32_t* ids, int M, int k, int activation, void* y);
/* Stream-ordered run: _submit enqueues a host function that starts the job when
 * the stream reaches it (x, w, ids then must hold the inputs: pinned buffers
 * filled by earlier copies on the stream) and returns at once; _wait enqueues a
 * host function that blocks the stream until the job is done.  Work on the
 * stream between the two overlaps the CPU job.  Graph-capturable (a captured
 * job keeps its record for the graph's lifetime).  One executor runs its jobs
 * in submission order. */
int ftmoe_cpu_experts_submit(ftmoe_cpu_executor* ex, const ftmoe_bank* host_bank, const void* x, const float* w,
                             const int32_t* ids, int M, int k, int activation, void* y, ftmoe_stream_t stream,
                             void** job);
int ftmoe_cpu_experts_wait(ftmoe_cpu_executor* ex, void* job, ftmoe_stream_t stream);

/* Instrumentation (no counterpart in the reference, whose NVTX ranges play this
 * role): between begin and end, every ftmoe_experts_* call made outside graph
 * capture records a HIP event on its stream before its first kernel and after
 * each kernel.  end synchronises on those events, writes the summed
 * milliseconds of each stage (decode: align, gate_up, down, combine; prefill:
 * align, x quant, gate_up, act quant, down, combine) and releases them. */
int ftmoe_stage_timing_begin(void);
int ftmoe_stage_timing_end(double* stage_ms, int max_stages, int* n_stages, int* n_calls);

#ifdef __cplusplus
}
#endif

#endif /* FTMOE_H */
