// Argument structs and launch entry points shared by the kernels and the C ABI.
#pragma once

#include "ftmoe_common.h"

namespace ftmoe {

enum WFmt : int { FMT_BF16 = 0, FMT_FP8 = 1, FMT_MXFP4 = 2, FMT_NONE = -1 };

struct AlignArgs {
  const int32_t* ids;          // [numel] expert ids (or expert ids to map)
  const int32_t* slot_for_id;  // nullable: [table_size] expert -> slot (-1 absent)
  int table_size;
  int32_t* slot_ids;           // nullable: mapped ids out [numel] (may alias ids)
  uint8_t* miss_mask;          // nullable: [numel]
  long long* stats;            // nullable: [4] accumulated counters
  int numel;
  int num_experts;             // experts of the aligned id space (slots if mapped)
  int block_size;
  int32_t* sorted_ids;         // [max_padded]
  int max_padded;
  int32_t* expert_ids;         // [max_blocks]
  int max_blocks;
  int32_t* ntpp;               // [1]
  int32_t* seg_expert;         // nullable: compact segments (an expert's routes in
  int32_t* seg_start;          //   pieces of at most seg_cap; at most
  int32_t* seg_count;          //   min(numel, num_experts + numel / seg_cap) of them)
  int32_t* n_seg;              // [1]
  int seg_cap;                 // > 0 when segments are requested
  int32_t* cum_out;            // nullable: [num_experts + 2] padded region starts
};

struct BankView {
  const uint8_t* w;  // weights, [S, N, K] elements of the format
  const void* s;     // fp8: float [S, N/128, K/128]; mxfp4: uint8 [S, N, K/32]; bf16: null
};

// Decode segments hold at most this many routes: one workgroup covers a whole
// segment in one pass over its weight rows.
constexpr int kDecodeSegCap = 32;

// FP8 decode calls of at least kWideMinTokens tokens cut segments at 64
// routes (the wide kernels read an expert once for up to 64 routes).
constexpr int kDecodeSegCapWide = 64;
constexpr int kWideMinTokens = 144;
inline int decode_seg_cap(int M, bool fp8) { return fp8 && M >= kWideMinTokens ? kDecodeSegCapWide : kDecodeSegCap; }
inline int decode_max_segments(int numel, int num_experts, int seg_cap = kDecodeSegCap) {
  const int bound = num_experts + numel / seg_cap;
  return numel < bound ? numel : bound;
}

struct DecodeArgs {
  const uint16_t* x;        // [M, H] bf16
  const float* topk_w;      // [M*k]
  const int32_t* sorted;    // route indices grouped by segment
  const int32_t* seg_expert;
  const int32_t* seg_start;
  const int32_t* seg_count;
  const int32_t* n_seg;
  int M, k, H, I, Is;       // Is: shared expert intermediate size (0: none)
  int max_seg;              // routed segments of the grid (the shared expert's pieces follow)
  int seg_cap;              // routes per segment at most (also the shared expert's token pieces)
  BankView gate_up, down;   // routed bank
  BankView sh_gate_up, sh_down;
  uint16_t* act;            // [M*k + M, act_stride] bf16
  int act_stride;
  uint16_t* ic3;            // [M*k, H] bf16
  uint16_t* sh_out;         // [M, H] bf16
  int act_kind;
  float act_limit;          // clamped SwiGLU of the routed experts (> 0), else 0
  float sh_act_limit;       // ... of the shared expert
  int weight_on_input;
};

hipError_t launch_softmax_topk(const void* logits, int logits_bf16, int M, int E, int k, int renorm, float* w,
                               int32_t* ids, hipStream_t stream);
hipError_t launch_grouped_sigmoid(const float* logits, const float* bias, int M, int E, int n_group,
                                  int topk_group, int k, int renorm, float scale, float* w, int32_t* ids,
                                  hipStream_t stream);
hipError_t launch_align(const AlignArgs& a, hipStream_t stream);
// Rows up to which the counting align keeps per-row counts in LDS; decode-form
// calls over larger banks take the sort-based align, which bounds the routes
// of one call instead.
constexpr int kCountMaxRows = 1023;
constexpr int kSortMaxRows = 16383;
constexpr int kSortMaxRoutes = 16384;

// A router call (softmax top-k or grouped sigmoid top-k) feeding the decode
// permutation.
struct RouteArgs {
  int grouped;            // 0: softmax top-k, 1: grouped sigmoid
  const void* logits;     // [M, E] float32 (or bf16 for softmax)
  int logits_bf16;
  int M, E, k, renorm;
  const float* bias;      // grouped: nullable [E]
  int n_group, topk_group;
  float scale;            // grouped: routed scaling factor
  float* out_w;           // [M, k]
  int32_t* out_ids;       // [M, k]
};
// Router then permutation: one kernel when the permutation fits one wave
// (a.ids must be r.out_ids), else the router and launch_align.
hipError_t launch_route_align(const RouteArgs& r, const AlignArgs& a, hipStream_t stream);
// Multi-workgroup align for large route counts without slot lookup, stats or
// segments; gcount: align_gcount_ints(numel, num_experts) ints of workspace.
size_t align_gcount_ints(int numel, int num_experts);
hipError_t launch_align_large(const AlignArgs& a, int32_t* gcount, hipStream_t stream);
hipError_t launch_slot_map(const int32_t* ids, int numel, const int32_t* slot_for_id, int table_size,
                           int32_t* slot_ids, uint8_t* miss_mask, long long* stats, hipStream_t stream);
hipError_t launch_route_histogram(const int32_t* ids, int numel, int num_experts, long long* freq,
                                  hipStream_t stream);
// shared_pieces false: the shared expert's pieces are left out of the grid
// (its gate_up already ran beside the router, launch_route_shared)
hipError_t launch_decode_stage(int stage, int fmt_r, int fmt_s, const DecodeArgs& a, hipStream_t stream,
                               bool shared_pieces = true);
// Router + permutation (as launch_route_align) and, in the same launch, the
// shared expert's gate_up; hipErrorNotSupported when the call does not
// qualify (grouped router, shared expert, at most 4 tokens, the one-wave
// align, at most 256 experts).
hipError_t launch_route_shared(const RouteArgs& r, const AlignArgs& al, int fmt_s, const DecodeArgs& a,
                               hipStream_t stream);
struct PrefillGemmArgs {
  // rows of the activation operand
  const uint8_t* xq;        // fp8 [rows, K] (FP8 / MXFP4) or bf16 [rows, K] (BF16)
  const void* xs;           // float [rows, K/128] (FP8) or uint32 e8m0 codes [rows, K/128] (MXFP4)
  int x_token_rows;         // 1: gate_up (row = token = route / k, shared row = token)
                            // 0: down    (row = route, shared row = M*k + token)
  const int32_t* sorted;    // [max_padded] route indices per BM block, sentinel numel
  const int32_t* cum;       // [E + 2] region starts of every expert (incl. the sentinel bucket)
  const int32_t* ntpp;      // [1]
  int num_experts;          // bank rows taking part
  int numel;                // M * k
  int M, k;
  int max_blocks;           // routed M blocks of the grid
  int shared_blocks;        // ceil(M / BM) if a shared expert is present, else 0
  int ntiles;               // N tiles
  int K;                    // reduction length
  int N;                    // weight rows of one expert (2I or H)
  int inter;                // I (gate/up split) for MODE gate_up
  BankView w;               // routed weights
  BankView ws;              // shared weights
  // outputs
  uint16_t* out;            // gate_up (bf16): act [numel + M, inter]; down: ic3 [numel, N]
  uint8_t* act_q;           // gate_up (FP8, MXFP4): e4m3 act [numel + M, inter] ...
  void* act_s;              // ... and its scales per 128 (float, or uint32 e8m0 codes)
  uint16_t* sh_out;         // down: shared out [M, N]
  const float* topk_w;      // [numel] (down)
  int act_kind;
  float act_limit;          // clamped SwiGLU of the routed experts (> 0), else 0
  float sh_act_limit;       // ... of the shared expert
};

// Routes per M block of the prefill GEMMs (the align block size): the
// quantised kernels tile 256 routes, the bf16 kernel 128.
inline int prefill_block_size(int fmt) { return fmt == FMT_BF16 ? 128 : 256; }

hipError_t launch_act_quant(int mode, const uint16_t* x, int rows, int K, uint8_t* q, void* scales,
                            hipStream_t stream);
hipError_t launch_prefill_gemm(int fmt, int gate_up, const PrefillGemmArgs& a, hipStream_t stream);

// Expert-cache admission (cache.hip): one call's ids -> slots with LRU
// admission of the missing experts.
struct LruArgs {
  int32_t* ids;           // [numel] expert ids in, slot ids out (-1: unfetched miss or id outside [0, E))
  int numel;
  int layer, num_layers, num_experts, cache_size;
  int32_t* slot_for_id;   // [num_layers * num_experts]
  int32_t* id_of_slot;    // [cache_size] flat id layer * E + expert, -1 empty
  int64_t* usage;         // [cache_size] step of last use
  int64_t* step;          // [1]
  int64_t* recency;       // nullable [num_experts] of this layer: order misses by recency
  int sort_len;           // power of two >= the largest miss count (recency order), else 0
  int max_fetch;          // < 0: every miss
  int fetch_frac_q16;     // > 0: fetch the bandwidth-matched share of the misses instead of max_fetch
  int capacity;           // entries of evict_slots / src_indices
  int32_t* evict_slots;   // [capacity]
  int32_t* src_indices;   // [capacity] layer-local expert rows
  int32_t* num_indices;   // [1] entries admitted
  int32_t* num_missing;   // [1] distinct missing experts before the cap
  int32_t* cpu_ids;       // nullable [numel]: the expert id of an unfetched miss, else -1
  long long* stats;       // nullable [4] accumulated: active, missing, calls, missed routes
  long long* unserved;    // nullable [1] accumulated: misses left unfetched for want of a free slot
};
hipError_t launch_lru_ensure(const LruArgs& a, hipStream_t stream);

// Whole-layer placement and slot release of the prefill movement.
struct PlaceArgs {
  int layer, num_layers, num_experts, cache_size;
  int32_t* slot_for_id;  // [num_layers * num_experts]
  int32_t* id_of_slot;   // [cache_size]
  int64_t* usage;        // [cache_size]
  int64_t* step;         // [1] (materialize)
  int32_t* evict_slots;  // [num_experts] (materialize)
  int32_t* src_indices;  // [num_experts] (materialize)
  int32_t* num_indices;  // [1] (materialize)
  int slot_begin, slot_end;  // release range
};
hipError_t launch_materialize_layer(const PlaceArgs& a, hipStream_t stream);
hipError_t launch_release_slots(const PlaceArgs& a, hipStream_t stream);
size_t lru_lds_bytes(int num_experts, int cache_size, int sort_len);

constexpr int kMaxFetchBanks = 8;
struct FetchArgs {
  const uint8_t* src[kMaxFetchBanks];   // this layer's host rows (pinned, device-mapped), per bank
  uint8_t* dst[kMaxFetchBanks];         // slot banks
  uint64_t row_bytes[kMaxFetchBanks];   // bytes of one expert in each bank (multiple of 16)
  int chunk_start[kMaxFetchBanks];      // first 64 KiB chunk of each bank within an entry
  int chunks_per_entry;
  int nbanks;
  int max_entries;                      // bound on *num_indices (the size of the two lists)
  const int32_t* evict_slots;
  const int32_t* src_indices;
  const int32_t* num_indices;
};
hipError_t launch_fetch_experts(const FetchArgs& a, int max_entries, hipStream_t stream);
hipError_t launch_hit_compact(const int32_t* slot_row, int num_experts, int threshold, int dst_base, int32_t* dst_rows,
                              int32_t* src_rows, int32_t* num, hipStream_t stream);
int fetch_chunks(uint64_t row_bytes);

// Records the message of a failed C-ABI call (ftmoe_last_error) and returns code.
int report_error(int code, const char* msg);
hipError_t launch_combine(const uint16_t* ic3, const int32_t* ids, int num_rows, const uint16_t* sh_out, int M,
                          int k, int H, uint16_t* y, hipStream_t stream);

}  // namespace ftmoe
