// C ABI of the MoE-layer hot path (declarations and contracts: include/ftmoe.h).
// Validates arguments on the host, carves the caller's workspace and launches
// the kernels of route.hip, align.hip and decode.hip on the caller's stream.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "ftmoe.h"

#include "kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_hip(hipError_t err, const char* what) {
  if (err != hipSuccess) return fail(FTMOE_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
  return FTMOE_OK;
}

constexpr size_t kAlignBytes = 256;

size_t round_up(size_t v) { return (v + kAlignBytes - 1) / kAlignBytes * kAlignBytes; }

// Sequential carve-out of a workspace buffer.
struct Carver {
  uint8_t* base;
  size_t off = 0;
  template <typename T>
  T* take(size_t n) {
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += round_up(n * sizeof(T));
    return p;
  }
};

int check_bank(const ftmoe_bank* b, const char* name, bool shared) {
  if (!b) return fail(FTMOE_ERR_INVALID, "%s bank is NULL", name);
  if (b->format < FTMOE_FMT_BF16 || b->format > FTMOE_FMT_MXFP4)
    return fail(FTMOE_ERR_UNSUPPORTED, "%s bank: unknown format %d", name, b->format);
  if (b->hidden <= 0 || b->inter <= 0 || b->hidden % 128 || b->inter % 128)
    return fail(FTMOE_ERR_UNSUPPORTED, "%s bank: hidden %d / inter %d must be positive multiples of 128", name,
                b->hidden, b->inter);
  if (b->num_rows <= 0 || (shared && b->num_rows != 1))
    return fail(FTMOE_ERR_INVALID, "%s bank: num_rows %d", name, b->num_rows);
  if (!b->gate_up || !b->down) return fail(FTMOE_ERR_INVALID, "%s bank: NULL weights", name);
  if (b->format != FTMOE_FMT_BF16 && (!b->gate_up_scale || !b->down_scale))
    return fail(FTMOE_ERR_INVALID, "%s bank: NULL scales for a quantized format", name);
  if (!std::isfinite(b->swiglu_limit) || b->swiglu_limit < 0.f)
    return fail(FTMOE_ERR_INVALID, "%s bank: swiglu_limit %g (finite, >= 0)", name, b->swiglu_limit);
  return FTMOE_OK;
}

// The clamped SwiGLU of a bank (swiglu_limit > 0) is a SiLU form.
int check_limit(const ftmoe_bank* b, const ftmoe_bank* shared, int activation, const char* what) {
  if (activation != FTMOE_ACT_SILU && ((b && b->swiglu_limit > 0.f) || (shared && shared->swiglu_limit > 0.f)))
    return fail(FTMOE_ERR_UNSUPPORTED, "%s: swiglu_limit > 0 needs the silu activation (got %d)", what, activation);
  return FTMOE_OK;
}

struct DecodeLayout {
  int32_t* sorted;
  int32_t* ntpp;
  int32_t* seg_expert;
  int32_t* seg_start;
  int32_t* seg_count;
  int32_t* n_seg;
  uint16_t* act;
  uint16_t* ic3;
  uint16_t* sh_out;
  int act_stride;
  size_t bytes;
};

DecodeLayout decode_layout(void* ws, int M, int k, const ftmoe_bank* bank, const ftmoe_bank* shared) {
  DecodeLayout L{};
  Carver c{static_cast<uint8_t*>(ws)};
  const int numel = M * k;
  L.sorted = c.take<int32_t>(numel);
  L.ntpp = c.take<int32_t>(1);
  const int max_seg = ftmoe::decode_max_segments(numel, bank->num_rows);
  L.seg_expert = c.take<int32_t>(max_seg);
  L.seg_start = c.take<int32_t>(max_seg);
  L.seg_count = c.take<int32_t>(max_seg);
  L.n_seg = c.take<int32_t>(1);
  L.act_stride = shared ? std::max(bank->inter, shared->inter) : bank->inter;
  L.act = c.take<uint16_t>(static_cast<size_t>(numel + M) * L.act_stride);
  L.ic3 = c.take<uint16_t>(static_cast<size_t>(numel) * bank->hidden);
  L.sh_out = shared ? c.take<uint16_t>(static_cast<size_t>(M) * bank->hidden) : nullptr;
  L.bytes = c.off;
  return L;
}


// ---- stage timing (instrumentation) ----------------------------------------
struct StageTimer {
  bool on = false;
  bool active = false;  // a call is being recorded
  std::vector<std::vector<hipEvent_t>> calls;  // events of each recorded call
  std::vector<hipEvent_t> cur;
  hipStream_t stream = nullptr;

  void start_call(hipStream_t s) {
    active = false;
    if (!on) return;
    // the legacy null stream cannot be captured; other streams are asked
    if (s != nullptr) {
      hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone) return;
    }
    stream = s;
    active = true;
    cur.clear();
    mark();
  }
  void mark() {
    if (!active) return;
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return;
    if (hipEventRecord(e, stream) != hipSuccess) {
      (void)hipEventDestroy(e);
      return;
    }
    cur.push_back(e);
  }
  void end_call() {
    if (!active) return;
    calls.push_back(cur);
    cur.clear();
    active = false;
  }
};
StageTimer g_timer;

struct PrefillLayout {
  int32_t* sorted;
  int32_t* expert_ids;
  int32_t* ntpp;
  int32_t* cum;
  int32_t* gcount;  // per-wave counts of the multi-workgroup align
  uint8_t* xq;
  void* xs;
  uint16_t* act;
  uint8_t* actq;
  void* as;
  uint16_t* ic3;
  uint16_t* sh_out;
  int max_padded, max_blocks;
  size_t bytes;
};

PrefillLayout prefill_layout(void* ws, int M, int k, const ftmoe_bank* bank, const ftmoe_bank* shared) {
  PrefillLayout L{};
  Carver c{static_cast<uint8_t*>(ws)};
  const int numel = M * k;
  const int H = bank->hidden, I = bank->inter;
  ftmoe_align_sizes(numel, bank->num_rows, ftmoe::prefill_block_size(bank->format), &L.max_padded, &L.max_blocks);
  L.sorted = c.take<int32_t>(L.max_padded);
  L.expert_ids = c.take<int32_t>(L.max_blocks);
  L.ntpp = c.take<int32_t>(1);
  L.cum = c.take<int32_t>(bank->num_rows + 2);
  L.gcount = c.take<int32_t>(ftmoe::align_gcount_ints(numel, bank->num_rows));
  const bool quant = bank->format != FTMOE_FMT_BF16;
  const size_t sc = 4;  // float scale (FP8) or e8m0 code in 32 bits (MXFP4)
  const size_t rows = static_cast<size_t>(numel) + (shared ? M : 0);
  if (quant) {
    L.xq = c.take<uint8_t>(static_cast<size_t>(M) * H);
    L.xs = c.take<uint8_t>(static_cast<size_t>(M) * (H / 128) * sc);
  }
  if (quant) {  // the gate/up GEMM writes the quantised activations directly
    L.act = nullptr;
    L.actq = c.take<uint8_t>(rows * I);
    L.as = c.take<uint8_t>(rows * (I / 128) * sc);
  } else {
    L.act = c.take<uint16_t>(rows * I);
  }
  L.ic3 = c.take<uint16_t>(static_cast<size_t>(numel) * H);
  L.sh_out = shared ? c.take<uint16_t>(static_cast<size_t>(M) * H) : nullptr;
  L.bytes = c.off;
  return L;
}

}  // namespace

namespace ftmoe {
int report_error(int code, const char* msg) { return fail(code, "%s", msg); }
}  // namespace ftmoe

extern "C" {

const char* ftmoe_last_error(void) { return g_last_error.c_str(); }

int ftmoe_version(void) { return 1; }

int ftmoe_route_softmax_topk(const void* logits, int logits_dtype, int M, int E, int k, int renormalize,
                             float* topk_w, int32_t* topk_ids, ftmoe_stream_t stream) {
  if (M < 0) return fail(FTMOE_ERR_INVALID, "route_softmax_topk: M=%d", M);
  if ((!logits || !topk_w || !topk_ids) && M) return fail(FTMOE_ERR_INVALID, "route_softmax_topk: NULL pointer");
  if (logits_dtype != FTMOE_DTYPE_F32 && logits_dtype != FTMOE_DTYPE_BF16)
    return fail(FTMOE_ERR_UNSUPPORTED, "route_softmax_topk: logits dtype %d", logits_dtype);
  if (E <= 0 || E > 1024 || k <= 0 || k > E || k > 64)
    return fail(FTMOE_ERR_UNSUPPORTED, "route_softmax_topk: M=%d E=%d k=%d (need E<=1024, 0<k<=min(E,64))", M, E, k);
  if (M == 0) return FTMOE_OK;
  return check_hip(ftmoe::launch_softmax_topk(logits, logits_dtype == FTMOE_DTYPE_BF16, M, E, k, renormalize,
                                              topk_w, topk_ids, stream),
                   "route_softmax_topk launch");
}

int ftmoe_route_grouped_sigmoid(const float* logits, const float* bias, int M, int E, int n_group, int topk_group,
                                int k, int renormalize, float routed_scaling_factor, float* topk_w,
                                int32_t* topk_ids, ftmoe_stream_t stream) {
  if (M < 0) return fail(FTMOE_ERR_INVALID, "route_grouped_sigmoid: M=%d", M);
  if ((!logits || !topk_w || !topk_ids) && M)
    return fail(FTMOE_ERR_INVALID, "route_grouped_sigmoid: NULL pointer");
  if (E <= 0 || E > 1024 || n_group <= 0 || n_group > 64 || E % n_group || topk_group <= 0 ||
      topk_group > n_group || k <= 0 || k > 64 || k > E / n_group * topk_group)
    return fail(FTMOE_ERR_UNSUPPORTED, "route_grouped_sigmoid: M=%d E=%d n_group=%d topk_group=%d k=%d", M, E,
                n_group, topk_group, k);
  if (n_group > 1 && E / n_group < 2)
    return fail(FTMOE_ERR_UNSUPPORTED, "route_grouped_sigmoid: groups need >= 2 experts");
  if (M == 0) return FTMOE_OK;
  return check_hip(ftmoe::launch_grouped_sigmoid(logits, bias, M, E, n_group, topk_group, k, renormalize,
                                                 routed_scaling_factor, topk_w, topk_ids, stream),
                   "route_grouped_sigmoid launch");
}

void ftmoe_align_sizes(int numel, int num_experts, int block_size, int* max_padded, int* max_blocks) {
  const long long mp = numel < num_experts + 1 ? static_cast<long long>(numel) * block_size
                                               : numel + static_cast<long long>(num_experts + 1) * (block_size - 1);
  if (max_padded) *max_padded = static_cast<int>(mp);
  if (max_blocks) *max_blocks = static_cast<int>((mp + block_size - 1) / block_size);
}

int ftmoe_align(const int32_t* topk_ids, int numel, int num_experts, int block_size, int32_t* sorted_ids,
                int32_t* expert_ids, int32_t* num_tokens_post_pad, ftmoe_stream_t stream) {
  if (numel < 0 || num_experts <= 0 || num_experts > 1023 || block_size <= 0)
    return fail(FTMOE_ERR_UNSUPPORTED, "align: numel=%d num_experts=%d block_size=%d", numel, num_experts,
                block_size);
  int max_padded = 0, max_blocks = 0;
  ftmoe_align_sizes(numel, num_experts, block_size, &max_padded, &max_blocks);
  if ((!topk_ids && numel) || (!sorted_ids && max_padded) || (!expert_ids && max_blocks) || !num_tokens_post_pad)
    return fail(FTMOE_ERR_INVALID, "align: NULL pointer");
  ftmoe::AlignArgs a{};
  a.ids = topk_ids;
  a.numel = numel;
  a.num_experts = num_experts;
  a.block_size = block_size;
  a.sorted_ids = sorted_ids;
  ftmoe_align_sizes(numel, num_experts, block_size, &a.max_padded, &a.max_blocks);
  a.expert_ids = expert_ids;
  a.ntpp = num_tokens_post_pad;
  return check_hip(ftmoe::launch_align(a, stream), "align launch");
}

int ftmoe_slot_map(const int32_t* topk_ids, int numel, const int32_t* slot_for_id, int num_experts,
                   int32_t* slot_ids, uint8_t* miss_mask, int64_t* stats, ftmoe_stream_t stream) {
  if ((!topk_ids && numel) || !slot_for_id || !slot_ids) return fail(FTMOE_ERR_INVALID, "slot_map: NULL pointer");
  if (numel < 0 || num_experts <= 0 || num_experts > 4096)
    return fail(FTMOE_ERR_UNSUPPORTED, "slot_map: numel=%d num_experts=%d", numel, num_experts);
  return check_hip(ftmoe::launch_slot_map(topk_ids, numel, slot_for_id, num_experts, slot_ids, miss_mask,
                                          reinterpret_cast<long long*>(stats), stream),
                   "slot_map launch");
}

int ftmoe_route_histogram(const int32_t* topk_ids, int numel, int num_experts, int64_t* freq, ftmoe_stream_t stream) {
  if ((!topk_ids && numel) || !freq) return fail(FTMOE_ERR_INVALID, "route_histogram: NULL pointer");
  if (numel < 0 || num_experts <= 0 || num_experts > 16384)
    return fail(FTMOE_ERR_UNSUPPORTED, "route_histogram: numel=%d num_experts=%d", numel, num_experts);
  if (numel == 0) return FTMOE_OK;
  return check_hip(ftmoe::launch_route_histogram(topk_ids, numel, num_experts, reinterpret_cast<long long*>(freq),
                                                 stream),
                   "route_histogram launch");
}

int ftmoe_lru_ensure(int32_t* expert_ids, int numel, int layer_id, int num_layers, int num_experts,
                     int32_t* slot_for_id, int32_t* id_of_slot, int64_t* usage, int64_t* step, int cache_size,
                     int64_t* recency, int max_fetch, int fetch_frac_q16, int32_t* evict_slots,
                     int32_t* src_indices, int capacity, int32_t* num_indices, int32_t* num_missing,
                     int32_t* cpu_ids, int64_t* stats, int64_t* unserved, ftmoe_stream_t stream) {
  if ((!expert_ids && numel) || !slot_for_id || !id_of_slot || !usage || !step || !num_indices || !num_missing ||
      ((!evict_slots || !src_indices) && capacity))
    return fail(FTMOE_ERR_INVALID, "lru_ensure: NULL pointer");
  if (numel < 0 || num_experts <= 0 || num_experts > 8192 || cache_size <= 0 || cache_size > 8192 ||
      num_layers <= 0 || layer_id < 0 || layer_id >= num_layers || capacity < 0 || fetch_frac_q16 < 0 ||
      fetch_frac_q16 > (1 << 16))
    return fail(FTMOE_ERR_UNSUPPORTED, "lru_ensure: numel=%d E=%d S=%d layer=%d/%d capacity=%d frac_q16=%d", numel,
                num_experts, cache_size, layer_id, num_layers, capacity, fetch_frac_q16);
  ftmoe::LruArgs a{};
  a.ids = expert_ids;
  a.numel = numel;
  a.layer = layer_id;
  a.num_layers = num_layers;
  a.num_experts = num_experts;
  a.cache_size = cache_size;
  a.slot_for_id = slot_for_id;
  a.id_of_slot = id_of_slot;
  a.usage = usage;
  a.step = step;
  a.recency = recency;
  a.sort_len = 0;
  if (recency) {
    const int most = std::max(1, std::min(numel, num_experts));
    a.sort_len = 1;
    while (a.sort_len < most) a.sort_len <<= 1;
  }
  a.max_fetch = max_fetch;
  a.fetch_frac_q16 = fetch_frac_q16;
  a.cpu_ids = cpu_ids;
  a.capacity = capacity;
  a.evict_slots = evict_slots;
  a.src_indices = src_indices;
  a.num_indices = num_indices;
  a.num_missing = num_missing;
  a.stats = reinterpret_cast<long long*>(stats);
  a.unserved = reinterpret_cast<long long*>(unserved);
  if (ftmoe::lru_lds_bytes(num_experts, cache_size, a.sort_len) > 160 * 1024 - 4096)
    return fail(FTMOE_ERR_UNSUPPORTED, "lru_ensure: E=%d S=%d exceed the LDS of one workgroup", num_experts,
                cache_size);
  return check_hip(ftmoe::launch_lru_ensure(a, stream), "lru_ensure launch");
}

int ftmoe_host_alloc(size_t bytes, void** ptr) {
  if (!ptr) return fail(FTMOE_ERR_INVALID, "host_alloc: NULL ptr");
  *ptr = nullptr;
  return check_hip(hipHostMalloc(ptr, bytes ? bytes : 1, hipHostMallocDefault), "host_alloc hipHostMalloc");
}

int ftmoe_host_free(void* ptr) { return ptr ? check_hip(hipHostFree(ptr), "host_free hipHostFree") : FTMOE_OK; }

int ftmoe_materialize_layer(int layer_id, int num_layers, int num_experts, int32_t* slot_for_id, int32_t* id_of_slot,
                            int64_t* usage, int64_t* step, int cache_size, int32_t* evict_slots,
                            int32_t* src_indices, int32_t* num_indices, ftmoe_stream_t stream) {
  if (!slot_for_id || !id_of_slot || !usage || !step || !evict_slots || !src_indices || !num_indices)
    return fail(FTMOE_ERR_INVALID, "materialize_layer: NULL pointer");
  if (num_experts <= 0 || cache_size < num_experts || num_layers <= 0 || layer_id < 0 || layer_id >= num_layers ||
      static_cast<long long>(num_layers) * num_experts > (1ll << 30))
    return fail(FTMOE_ERR_UNSUPPORTED, "materialize_layer: E=%d S=%d layer=%d/%d (needs S >= E)", num_experts,
                cache_size, layer_id, num_layers);
  ftmoe::PlaceArgs a{};
  a.layer = layer_id;
  a.num_layers = num_layers;
  a.num_experts = num_experts;
  a.cache_size = cache_size;
  a.slot_for_id = slot_for_id;
  a.id_of_slot = id_of_slot;
  a.usage = usage;
  a.step = step;
  a.evict_slots = evict_slots;
  a.src_indices = src_indices;
  a.num_indices = num_indices;
  return check_hip(ftmoe::launch_materialize_layer(a, stream), "materialize_layer launch");
}

int ftmoe_release_slots(int slot_begin, int slot_end, int num_layers, int num_experts, int32_t* slot_for_id,
                        int32_t* id_of_slot, int64_t* usage, int cache_size, ftmoe_stream_t stream) {
  if (!slot_for_id || !id_of_slot || !usage) return fail(FTMOE_ERR_INVALID, "release_slots: NULL pointer");
  if (slot_begin < 0 || slot_end < slot_begin || slot_end > cache_size || num_layers <= 0 || num_experts <= 0)
    return fail(FTMOE_ERR_UNSUPPORTED, "release_slots: [%d, %d) of %d slots", slot_begin, slot_end, cache_size);
  ftmoe::PlaceArgs a{};
  a.num_layers = num_layers;
  a.num_experts = num_experts;
  a.cache_size = cache_size;
  a.slot_for_id = slot_for_id;
  a.id_of_slot = id_of_slot;
  a.usage = usage;
  a.slot_begin = slot_begin;
  a.slot_end = slot_end;
  return check_hip(ftmoe::launch_release_slots(a, stream), "release_slots launch");
}

int ftmoe_prefill_hit_compact(const int32_t* slot_for_id_row, int num_experts, int threshold, int dst_base,
                              int32_t* dst_rows, int32_t* src_rows, int32_t* num_hits, ftmoe_stream_t stream) {
  if (!slot_for_id_row || !dst_rows || !src_rows || !num_hits)
    return fail(FTMOE_ERR_INVALID, "prefill_hit_compact: NULL pointer");
  if (num_experts <= 0 || num_experts > 8192 || threshold < 0 || dst_base < 0)
    return fail(FTMOE_ERR_UNSUPPORTED, "prefill_hit_compact: num_experts=%d threshold=%d dst_base=%d", num_experts,
                threshold, dst_base);
  return check_hip(ftmoe::launch_hit_compact(slot_for_id_row, num_experts, threshold, dst_base, dst_rows, src_rows,
                                             num_hits, stream),
                   "prefill_hit_compact launch");
}

int ftmoe_fetch_experts(const ftmoe_fetch_bank* banks, int nbanks, const int32_t* evict_slots,
                        const int32_t* src_indices, const int32_t* num_indices, int max_entries,
                        ftmoe_stream_t stream) {
  if (!banks || !num_indices || ((!evict_slots || !src_indices) && max_entries))
    return fail(FTMOE_ERR_INVALID, "fetch_experts: NULL pointer");
  if (nbanks <= 0 || nbanks > ftmoe::kMaxFetchBanks || max_entries < 0)
    return fail(FTMOE_ERR_UNSUPPORTED, "fetch_experts: nbanks=%d max_entries=%d", nbanks, max_entries);
  ftmoe::FetchArgs a{};
  int chunks = 0;
  for (int b = 0; b < nbanks; ++b) {
    const ftmoe_fetch_bank& k = banks[b];
    if (!k.host_rows || !k.slot_bank) return fail(FTMOE_ERR_INVALID, "fetch_experts: bank %d NULL", b);
    if (k.row_bytes == 0 || k.row_bytes % 16 || reinterpret_cast<uintptr_t>(k.host_rows) % 16 ||
        reinterpret_cast<uintptr_t>(k.slot_bank) % 16)
      return fail(FTMOE_ERR_UNSUPPORTED, "fetch_experts: bank %d rows must be 16-byte multiples at 16-byte addresses",
                  b);
    a.src[b] = static_cast<const uint8_t*>(k.host_rows);
    a.dst[b] = static_cast<uint8_t*>(k.slot_bank);
    a.row_bytes[b] = k.row_bytes;
    a.chunk_start[b] = chunks;
    chunks += ftmoe::fetch_chunks(k.row_bytes);
  }
  a.chunks_per_entry = chunks;
  a.nbanks = nbanks;
  a.evict_slots = evict_slots;
  a.src_indices = src_indices;
  a.num_indices = num_indices;
  a.max_entries = max_entries;
  if (max_entries == 0) return FTMOE_OK;
  return check_hip(ftmoe::launch_fetch_experts(a, max_entries, stream), "fetch_experts launch");
}

int ftmoe_act_quant_fp8(const void* x, int rows, int K, int mode, void* q, void* scales, ftmoe_stream_t stream) {
  if ((!x || !q || !scales) && rows) return fail(FTMOE_ERR_INVALID, "act_quant_fp8: NULL pointer");
  if (rows < 0 || K <= 0 || K % 128 || (mode != 0 && mode != 1))
    return fail(FTMOE_ERR_UNSUPPORTED, "act_quant_fp8: rows=%d K=%d mode=%d", rows, K, mode);
  if (rows == 0) return FTMOE_OK;
  return check_hip(ftmoe::launch_act_quant(mode, static_cast<const uint16_t*>(x), rows, K, static_cast<uint8_t*>(q),
                                           scales, stream),
                   "act_quant_fp8 launch");
}

size_t ftmoe_experts_decode_workspace(int M, int top_k, const ftmoe_bank* bank, const ftmoe_bank* shared) {
  if (!bank || M <= 0 || top_k <= 0) return 0;
  return decode_layout(nullptr, M, top_k, bank, shared).bytes;
}

namespace {

// Optional expert-slot lookup in front of the decode permutation.
struct SlotLookup {
  const int32_t* slot_for_id;
  int num_experts;
  int32_t* slot_ids;
  uint8_t* miss_mask;
  int64_t* stats;
};

// route (nullable): the router call that produces topk_w / topk_ids first
// (fused with the permutation when both fit one launch).
int experts_decode_impl(const void* x, int M, int top_k, const float* topk_w, const int32_t* topk_ids,
                        const SlotLookup* slots, const ftmoe_bank* bank, const ftmoe_bank* shared, int activation,
                        int apply_router_weight_on_input, void* y, void* workspace, size_t workspace_bytes,
                        ftmoe_stream_t stream, const ftmoe::RouteArgs* route = nullptr) {
  int rc = check_bank(bank, "routed", false);
  if (rc) return rc;
  if (shared) {
    rc = check_bank(shared, "shared", true);
    if (rc) return rc;
    if (shared->hidden != bank->hidden) return fail(FTMOE_ERR_INVALID, "shared hidden %d != %d", shared->hidden, bank->hidden);
  }
  if (M < 0 || top_k <= 0) return fail(FTMOE_ERR_INVALID, "experts_decode: M=%d top_k=%d", M, top_k);
  if (M == 0) return FTMOE_OK;  // an empty batch: nothing to compute, no pointer is read
  if (!x || !topk_w || !topk_ids || !y) return fail(FTMOE_ERR_INVALID, "experts_decode: NULL pointer");
  if (bank->num_rows > ftmoe::kSortMaxRows ||
      (bank->num_rows > ftmoe::kCountMaxRows && M * top_k > ftmoe::kSortMaxRoutes))
    return fail(FTMOE_ERR_UNSUPPORTED, "experts_decode: num_rows %d with %d routes (rows <= %d, and routes <= %d "
                "above %d rows)", bank->num_rows, M * top_k, ftmoe::kSortMaxRows, ftmoe::kSortMaxRoutes,
                ftmoe::kCountMaxRows);
  if (activation < FTMOE_ACT_SILU || activation > FTMOE_ACT_GELU_TANH)
    return fail(FTMOE_ERR_UNSUPPORTED, "experts_decode: activation %d", activation);
  rc = check_limit(bank, shared, activation, "experts_decode");
  if (rc) return rc;
  const DecodeLayout need = decode_layout(nullptr, M, top_k, bank, shared);
  {
    // the decode kernels address activations and one expert's matrices with
    // 32-bit buffer offsets
    const size_t lim = size_t{1} << 31;
    const size_t act_bytes = static_cast<size_t>(M) * (top_k + 1) * need.act_stride * 2;
    const size_t x_bytes = static_cast<size_t>(M) * bank->hidden * 2;
    const auto mat_bytes = [](const ftmoe_bank* b) {
      const size_t n = static_cast<size_t>(2) * b->inter * b->hidden;  // gate_up elements
      return b->format == FTMOE_FMT_BF16 ? 2 * n : b->format == FTMOE_FMT_FP8_B128 ? n : n / 2;
    };
    if (act_bytes >= lim || x_bytes >= lim || mat_bytes(bank) >= lim || (shared && mat_bytes(shared) >= lim))
      return fail(FTMOE_ERR_UNSUPPORTED, "experts_decode: batch %d or expert size beyond the decode path's 2 GiB "
                  "buffer ranges (use experts_prefill)", M);
  }
  if (!workspace || workspace_bytes < need.bytes)
    return fail(FTMOE_ERR_WORKSPACE, "experts_decode: workspace %zu < %zu bytes", workspace_bytes, need.bytes);
  const DecodeLayout L = decode_layout(workspace, M, top_k, bank, shared);
  const int numel = M * top_k;

  ftmoe::AlignArgs al{};
  al.ids = topk_ids;
  al.numel = numel;
  al.num_experts = bank->num_rows;
  al.block_size = 1;
  al.sorted_ids = L.sorted;
  // the decode kernels read the segments only: no block expert ids, no
  // sentinel fill of the unused tail
  al.max_padded = 0;
  al.max_blocks = 0;
  al.expert_ids = nullptr;
  al.ntpp = L.ntpp;
  al.seg_expert = L.seg_expert;
  al.seg_start = L.seg_start;
  al.seg_count = L.seg_count;
  al.n_seg = L.n_seg;
  // segment cap (the workspace is sized for the smaller one, which gives more segments)
  const int seg_cap = ftmoe::decode_seg_cap(M, bank->format == FTMOE_FMT_FP8_B128);
  al.seg_cap = seg_cap;
  if (slots) {
    al.slot_for_id = slots->slot_for_id;
    al.table_size = slots->num_experts;
    al.slot_ids = slots->slot_ids;
    al.miss_mask = slots->miss_mask;
    al.stats = reinterpret_cast<long long*>(slots->stats);
  }
  // ids the later kernels see: slot ids when the lookup ran here
  const int32_t* route_ids = slots ? slots->slot_ids : topk_ids;

  ftmoe::DecodeArgs d{};
  d.x = static_cast<const uint16_t*>(x);
  d.topk_w = topk_w;
  d.sorted = L.sorted;
  d.seg_expert = L.seg_expert;
  d.seg_start = L.seg_start;
  d.seg_count = L.seg_count;
  d.n_seg = L.n_seg;
  d.M = M;
  d.k = top_k;
  d.H = bank->hidden;
  d.I = bank->inter;
  d.Is = shared ? shared->inter : 0;
  d.max_seg = ftmoe::decode_max_segments(numel, bank->num_rows, seg_cap);
  d.seg_cap = seg_cap;
  d.gate_up = {static_cast<const uint8_t*>(bank->gate_up), bank->gate_up_scale};
  d.down = {static_cast<const uint8_t*>(bank->down), bank->down_scale};
  if (shared) {
    d.sh_gate_up = {static_cast<const uint8_t*>(shared->gate_up), shared->gate_up_scale};
    d.sh_down = {static_cast<const uint8_t*>(shared->down), shared->down_scale};
  }
  d.act = L.act;
  d.act_stride = L.act_stride;
  d.ic3 = L.ic3;
  d.sh_out = L.sh_out;
  d.act_kind = activation;
  d.act_limit = bank->swiglu_limit;
  d.sh_act_limit = shared ? shared->swiglu_limit : 0.f;
  d.weight_on_input = apply_router_weight_on_input;
  const int fmt_s = shared ? shared->format : FTMOE_FMT_NONE;

  g_timer.start_call(stream);
  // small grouped-router calls with a shared expert: the shared expert's
  // gate_up runs in the router's launch
  bool shared_ran = false;
  if (route && shared) {
    const hipError_t e = ftmoe::launch_route_shared(*route, al, fmt_s, d, stream);
    if (e == hipSuccess) shared_ran = true;
    else if (e != hipErrorNotSupported) return check_hip(e, "experts_decode route + align + shared gate_up");
  }
  if (!shared_ran) {
    rc = route ? check_hip(ftmoe::launch_route_align(*route, al, stream), "experts_decode route + align")
               : check_hip(ftmoe::launch_align(al, stream), "experts_decode align");
    if (rc) return rc;
  }
  g_timer.mark();

  rc = check_hip(ftmoe::launch_decode_stage(0, bank->format, fmt_s, d, stream, !shared_ran), "experts_decode gate_up");
  if (rc) return rc;
  g_timer.mark();
  rc = check_hip(ftmoe::launch_decode_stage(1, bank->format, shared ? shared->format : FTMOE_FMT_NONE, d, stream),
                 "experts_decode down");
  if (rc) return rc;
  g_timer.mark();
  rc = check_hip(ftmoe::launch_combine(L.ic3, route_ids, bank->num_rows, L.sh_out, M, top_k, bank->hidden,
                                       static_cast<uint16_t*>(y), stream),
                 "experts_decode combine");
  g_timer.mark();
  g_timer.end_call();
  return rc;
}

}  // namespace

int ftmoe_experts_decode(const void* x, int M, int top_k, const float* topk_w, const int32_t* topk_ids,
                         const ftmoe_bank* bank, const ftmoe_bank* shared, int activation,
                         int apply_router_weight_on_input, void* y, void* workspace, size_t workspace_bytes,
                         ftmoe_stream_t stream) {
  return experts_decode_impl(x, M, top_k, topk_w, topk_ids, nullptr, bank, shared, activation,
                             apply_router_weight_on_input, y, workspace, workspace_bytes, stream);
}

int ftmoe_experts_decode_cached(const void* x, int M, int top_k, const float* topk_w, const int32_t* topk_ids,
                                const int32_t* slot_for_id, int num_experts, int32_t* slot_ids, uint8_t* miss_mask,
                                int64_t* stats, const ftmoe_bank* bank, const ftmoe_bank* shared, int activation,
                                int apply_router_weight_on_input, void* y, void* workspace, size_t workspace_bytes,
                                ftmoe_stream_t stream) {
  if (M != 0 && (!slot_for_id || !slot_ids))
    return fail(FTMOE_ERR_INVALID, "experts_decode_cached: NULL slot table or slot ids");
  if (num_experts <= 0 || num_experts > 16384)
    return fail(FTMOE_ERR_UNSUPPORTED, "experts_decode_cached: num_experts=%d", num_experts);
  const SlotLookup sl{slot_for_id, num_experts, slot_ids, miss_mask, stats};
  return experts_decode_impl(x, M, top_k, topk_w, topk_ids, &sl, bank, shared, activation,
                             apply_router_weight_on_input, y, workspace, workspace_bytes, stream);
}

int ftmoe_experts_decode_routed(const void* x, int M, int top_k, const ftmoe_router* router, float* topk_w,
                                int32_t* topk_ids, const int32_t* slot_for_id, int num_experts, int32_t* slot_ids,
                                uint8_t* miss_mask, int64_t* stats, const ftmoe_bank* bank, const ftmoe_bank* shared,
                                int activation, int apply_router_weight_on_input, void* y, void* workspace,
                                size_t workspace_bytes, ftmoe_stream_t stream) {
  if (!router) return fail(FTMOE_ERR_INVALID, "experts_decode_routed: NULL router");
  const int E = router->num_experts, k = top_k;
  ftmoe::RouteArgs r{};
  r.logits = router->logits;
  r.M = M;
  r.E = E;
  r.k = k;
  r.renorm = router->renormalize;
  r.out_w = topk_w;
  r.out_ids = topk_ids;
  if (router->kind == FTMOE_ROUTER_SOFTMAX_TOPK) {
    if (router->logits_dtype != FTMOE_DTYPE_F32 && router->logits_dtype != FTMOE_DTYPE_BF16)
      return fail(FTMOE_ERR_UNSUPPORTED, "experts_decode_routed: logits dtype %d", router->logits_dtype);
    if (E <= 0 || E > 1024 || k <= 0 || k > E || k > 64)
      return fail(FTMOE_ERR_UNSUPPORTED, "experts_decode_routed: E=%d k=%d (need E<=1024, 0<k<=min(E,64))", E, k);
    r.grouped = 0;
    r.logits_bf16 = router->logits_dtype == FTMOE_DTYPE_BF16;
  } else if (router->kind == FTMOE_ROUTER_GROUPED_SIGMOID) {
    const int ng = router->n_group, tg = router->topk_group;
    if (router->logits_dtype != FTMOE_DTYPE_F32)
      return fail(FTMOE_ERR_UNSUPPORTED, "experts_decode_routed: grouped routing takes float32 logits");
    if (E <= 0 || E > 1024 || ng <= 0 || ng > 64 || E % ng || tg <= 0 || tg > ng || k <= 0 || k > 64 ||
        k > E / ng * tg || (ng > 1 && E / ng < 2))
      return fail(FTMOE_ERR_UNSUPPORTED, "experts_decode_routed: E=%d n_group=%d topk_group=%d k=%d", E, ng, tg, k);
    r.grouped = 1;
    r.bias = router->bias;
    r.n_group = ng;
    r.topk_group = tg;
    r.scale = router->routed_scaling_factor;
  } else {
    return fail(FTMOE_ERR_UNSUPPORTED, "experts_decode_routed: router kind %d", router->kind);
  }
  if (M < 0) return fail(FTMOE_ERR_INVALID, "experts_decode_routed: M=%d", M);
  if (M == 0) return FTMOE_OK;  // an empty batch: nothing to route or compute
  if (!router->logits || !topk_w || !topk_ids)
    return fail(FTMOE_ERR_INVALID, "experts_decode_routed: NULL logits or router outputs");
  if (!slot_for_id)
    return experts_decode_impl(x, M, top_k, topk_w, topk_ids, nullptr, bank, shared, activation,
                               apply_router_weight_on_input, y, workspace, workspace_bytes, stream, &r);
  if (!slot_ids) return fail(FTMOE_ERR_INVALID, "experts_decode_routed: NULL slot ids");
  if (num_experts <= 0 || num_experts > 16384)
    return fail(FTMOE_ERR_UNSUPPORTED, "experts_decode_routed: num_experts=%d", num_experts);
  const SlotLookup sl{slot_for_id, num_experts, slot_ids, miss_mask, stats};
  return experts_decode_impl(x, M, top_k, topk_w, topk_ids, &sl, bank, shared, activation,
                             apply_router_weight_on_input, y, workspace, workspace_bytes, stream, &r);
}

size_t ftmoe_experts_prefill_workspace(int M, int top_k, const ftmoe_bank* bank, const ftmoe_bank* shared) {
  if (!bank || M <= 0 || top_k <= 0) return 0;
  return prefill_layout(nullptr, M, top_k, bank, shared).bytes;
}

int ftmoe_experts_prefill(const void* x, int M, int top_k, const float* topk_w, const int32_t* topk_ids,
                          const ftmoe_bank* bank, const ftmoe_bank* shared, int activation, void* y,
                          void* workspace, size_t workspace_bytes, ftmoe_stream_t stream) {
  int rc = check_bank(bank, "routed", false);
  if (rc) return rc;
  if (shared) {
    rc = check_bank(shared, "shared", true);
    if (rc) return rc;
    if (shared->hidden != bank->hidden || shared->inter != bank->inter || shared->format != bank->format)
      return fail(FTMOE_ERR_UNSUPPORTED, "experts_prefill: the shared expert must match the routed format and shape");
  }
  if (M < 0 || top_k <= 0) return fail(FTMOE_ERR_INVALID, "experts_prefill: M=%d top_k=%d", M, top_k);
  if (M == 0) return FTMOE_OK;  // an empty batch: nothing to compute, no pointer is read
  if (!x || !topk_w || !topk_ids || !y) return fail(FTMOE_ERR_INVALID, "experts_prefill: NULL pointer");
  if (bank->num_rows > 1023) return fail(FTMOE_ERR_UNSUPPORTED, "experts_prefill: num_rows %d > 1023", bank->num_rows);
  if (activation < FTMOE_ACT_SILU || activation > FTMOE_ACT_GELU_TANH)
    return fail(FTMOE_ERR_UNSUPPORTED, "experts_prefill: activation %d", activation);
  rc = check_limit(bank, shared, activation, "experts_prefill");
  if (rc) return rc;
  const PrefillLayout need = prefill_layout(nullptr, M, top_k, bank, shared);
  if (!workspace || workspace_bytes < need.bytes)
    return fail(FTMOE_ERR_WORKSPACE, "experts_prefill: workspace %zu < %zu bytes", workspace_bytes, need.bytes);
  const PrefillLayout L = prefill_layout(workspace, M, top_k, bank, shared);
  const int numel = M * top_k;
  const int H = bank->hidden, I = bank->inter;
  const int fmt = bank->format;
  // the quantised GEMMs address each operand (activations, one expert's
  // weights) through a buffer descriptor with 31-bit offsets
  if (fmt != FTMOE_FMT_BF16 && (static_cast<int64_t>(numel + M) * I > INT32_MAX ||
                                static_cast<int64_t>(M) * H > INT32_MAX || 2 * static_cast<int64_t>(I) * H > INT32_MAX))
    return fail(FTMOE_ERR_UNSUPPORTED, "experts_prefill: an operand beyond 2 GiB (M=%d top_k=%d H=%d I=%d)", M,
                top_k, H, I);

  ftmoe::AlignArgs al{};
  al.ids = topk_ids;
  al.numel = numel;
  al.num_experts = bank->num_rows;
  const int bm = ftmoe::prefill_block_size(bank->format);
  al.block_size = bm;
  al.sorted_ids = L.sorted;
  al.max_padded = L.max_padded;
  al.expert_ids = L.expert_ids;
  al.max_blocks = L.max_blocks;
  al.ntpp = L.ntpp;
  al.cum_out = L.cum;
  g_timer.start_call(stream);
  rc = check_hip(ftmoe::launch_align_large(al, L.gcount, stream), "experts_prefill align");
  if (rc) return rc;
  g_timer.mark();

  const uint16_t* xb = static_cast<const uint16_t*>(x);
  const int qmode = fmt == FTMOE_FMT_MXFP4 ? 2 : 0;
  if (fmt != FTMOE_FMT_BF16) {
    rc = check_hip(ftmoe::launch_act_quant(qmode, xb, M, H, L.xq, L.xs, stream), "experts_prefill x quant");
    if (rc) return rc;
  }
  g_timer.mark();
  ftmoe::PrefillGemmArgs g{};
  g.sorted = L.sorted;
  g.cum = L.cum;
  g.ntpp = L.ntpp;
  g.num_experts = bank->num_rows;
  g.numel = numel;
  g.M = M;
  g.k = top_k;
  g.max_blocks = L.max_blocks;
  g.shared_blocks = shared ? (M + bm - 1) / bm : 0;
  g.w = {nullptr, nullptr};
  g.act_kind = activation;
  g.act_limit = bank->swiglu_limit;
  g.sh_act_limit = shared ? shared->swiglu_limit : 0.f;
  g.topk_w = topk_w;

  // gate_up + SwiGLU -> act
  g.xq = fmt == FTMOE_FMT_BF16 ? reinterpret_cast<const uint8_t*>(xb) : L.xq;
  g.xs = L.xs;
  g.x_token_rows = 1;
  g.ntiles = I / 64;
  g.K = H;
  g.N = 2 * I;
  g.inter = I;
  g.w = {static_cast<const uint8_t*>(bank->gate_up), bank->gate_up_scale};
  if (shared) g.ws = {static_cast<const uint8_t*>(shared->gate_up), shared->gate_up_scale};
  g.out = L.act;  // bf16 act (bf16 format); FP8 / MXFP4 write act_q and act_s
  g.act_q = L.actq;
  g.act_s = L.as;
  rc = check_hip(ftmoe::launch_prefill_gemm(fmt, 1, g, stream), "experts_prefill gate_up");
  if (rc) return rc;
  g_timer.mark();
  g_timer.mark();  // (the activation quantisation is fused into the gate/up epilogue)

  // down (x router weight) -> ic3 / shared out
  g.xq = fmt == FTMOE_FMT_BF16 ? reinterpret_cast<const uint8_t*>(L.act) : L.actq;
  g.xs = L.as;
  g.x_token_rows = 0;
  g.ntiles = H / 128;
  g.K = I;
  g.N = H;
  g.w = {static_cast<const uint8_t*>(bank->down), bank->down_scale};
  if (shared) g.ws = {static_cast<const uint8_t*>(shared->down), shared->down_scale};
  g.out = L.ic3;
  g.sh_out = L.sh_out;
  rc = check_hip(ftmoe::launch_prefill_gemm(fmt, 0, g, stream), "experts_prefill down");
  if (rc) return rc;
  g_timer.mark();
  rc = check_hip(ftmoe::launch_combine(L.ic3, topk_ids, bank->num_rows, L.sh_out, M, top_k, H,
                                       static_cast<uint16_t*>(y), stream),
                 "experts_prefill combine");
  g_timer.mark();
  g_timer.end_call();
  return rc;
}

}  // extern "C"

// ---- decode without allocation ---------------------------------------------
// The workspace of ftmoe_experts_decode_noalloc is this file-scope device
// array: each GPU the library runs on holds its own copy for the life of the
// process.  Host code never uses its name as an address (on the host it is a
// stand-in); the address on each device comes from hipGetSymbolAddress, taken
// once per device with that device current.
constexpr size_t kNoallocScratchBytes = size_t{64} << 20;
static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The scratch array's address on the current device (which must own stream).
int noalloc_scratch(ftmoe_stream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(FTMOE_ERR_HIP, "experts_decode_noalloc: no current device (or device %d beyond %d)", dev, kMaxDevices);
  if (stream) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess)
      return fail(FTMOE_ERR_HIP, "experts_decode_noalloc: stream device query failed");
    if (sdev != dev)
      return fail(FTMOE_ERR_INVALID, "experts_decode_noalloc: stream of device %d, current device %d", sdev, dev);
  }
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    // the lookup may load the library's code object on this device: not a
    // call to make while the stream is being captured
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (stream && hipStreamIsCapturing(stream, &cs) != hipSuccess)
      return fail(FTMOE_ERR_HIP, "experts_decode_noalloc: stream capture query failed");
    if (cs != hipStreamCaptureStatusNone)
      return fail(FTMOE_ERR_UNSUPPORTED, "experts_decode_noalloc: the first call on device %d must run outside graph "
                  "capture (it looks up the scratch array's address)", dev);
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p)
      return fail(FTMOE_ERR_HIP, "experts_decode_noalloc: scratch address on device %d: %s", dev,
                  hipGetErrorString(err));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FTMOE_OK;
}

}  // namespace

extern "C" {

size_t ftmoe_experts_decode_noalloc_capacity(void) { return kNoallocScratchBytes; }

int ftmoe_experts_decode_noalloc(const void* x, int M, int top_k, const float* topk_w, const int32_t* topk_ids,
                                 const ftmoe_bank* bank, const ftmoe_bank* shared, int activation,
                                 int apply_router_weight_on_input, void* y, ftmoe_stream_t stream) {
  if (!bank || M < 0 || top_k <= 0)
    return fail(FTMOE_ERR_INVALID, "experts_decode_noalloc: bank %p, M=%d top_k=%d", static_cast<const void*>(bank),
                M, top_k);
  if (M == 0) return FTMOE_OK;  // an empty batch: nothing to compute
  const size_t need = decode_layout(nullptr, M, top_k, bank, shared).bytes;
  if (need > kNoallocScratchBytes)
    return fail(FTMOE_ERR_WORKSPACE, "experts_decode_noalloc: batch %d x top-%d needs %zu bytes of scratch, beyond the "
                "static %zu (use ftmoe_experts_decode with a caller workspace)", M, top_k, need, kNoallocScratchBytes);
  void* ws = nullptr;
  const int rc = noalloc_scratch(stream, &ws);
  if (rc) return rc;
  // every workspace field the kernels read is written earlier in the same call:
  // nothing needs clearing between calls
  return experts_decode_impl(x, M, top_k, topk_w, topk_ids, nullptr, bank, shared, activation,
                             apply_router_weight_on_input, y, ws, kNoallocScratchBytes, stream);
}

int ftmoe_stage_timing_begin(void) {
  g_timer.on = true;
  g_timer.calls.clear();
  return FTMOE_OK;
}

int ftmoe_stage_timing_end(double* stage_ms, int max_stages, int* n_stages, int* n_calls) {
  g_timer.on = false;
  int ns = 0;
  for (auto& c : g_timer.calls) ns = std::max(ns, static_cast<int>(c.size()) - 1);
  for (int i = 0; i < max_stages && stage_ms; ++i) stage_ms[i] = 0.0;
  int rc = FTMOE_OK;
  for (auto& c : g_timer.calls) {
    if (c.empty()) continue;
    if (hipEventSynchronize(c.back()) != hipSuccess) rc = fail(FTMOE_ERR_HIP, "stage timing: event sync failed");
    for (size_t i = 1; i < c.size(); ++i) {
      float ms = 0.f;
      if (hipEventElapsedTime(&ms, c[i - 1], c[i]) == hipSuccess && stage_ms && static_cast<int>(i - 1) < max_stages)
        stage_ms[i - 1] += ms;
    }
    for (hipEvent_t e : c) (void)hipEventDestroy(e);
  }
  if (n_stages) *n_stages = ns;
  if (n_calls) *n_calls = static_cast<int>(g_timer.calls.size());
  g_timer.calls.clear();
  return rc;
}

}  // extern "C"
