// Expert-cache miss path: LRU admission of a step's routed experts into the
// slot cache, and the gather of the admitted experts' rows from the pinned
// host banks into their slots (over PCIe, by the shader: the number of rows is
// on the device, so the copy needs no host synchronisation and replays in a
// graph).
//
// Admission contract (reference: the CPU mirror of the admission kernel,
// moe/offload_kernels.py:128-188, whose decisions the reference's tests hold
// bit-identical to its GPU path; ensure_experts, offload_kernels.py:19-40):
//   step += 1; the distinct ids of the call are "seen"; every resident seen
//   expert's slot gets usage = step; the missing seen experts are ordered by
//   ascending id, or with a recency table by (most recently seen first, then
//   ascending id); the first min(misses, cap, free) of them take, one after
//   the other, the slot with the smallest (usage, slot) -- the previous owner
//   (any layer) loses its mapping, the slot gets usage = step -- and are listed
//   in (evict_slots, src_indices); the recency of every seen expert becomes
//   step; finally every id is rewritten to its slot (-1 for unfetched misses
//   and for ids outside [0, num_experts)).
// "free" is the number of slots with usage < step after the touch: slots that
// neither hold an expert of this call nor were admitted by it.  An admitted
// slot gets usage = step, so while fewer than "free" misses have been placed
// the smallest (usage, slot) is always such a slot: no victim repeats and no
// expert of the call loses its slot (the reference's GPU kernel excludes the
// same slots, offload_kernels.py:369-387).  Misses beyond it stay unfetched
// and are counted in unserved (nullable, int64, accumulated).
// The cap is max_fetch (< 0: none), or with a fetch fraction f (Q16, > 0) the
// integer n in {floor(m f), floor(m f) + 1} with the smaller max(n (1 - f),
// (m - n) f) -- PCIe fetch and CPU overflow balanced, lower n on a tie
// (offload_kernels.py:160-164).  cpu_ids, when given, receives per route the
// expert id of an unfetched miss and -1 elsewhere: the routes the CPU computes
// in the hybrid decode (layers/moe.py:350-352).
#include "kernels.h"

namespace ftmoe {

constexpr int kLruThreads = 1024;
constexpr int kLruWaves = kLruThreads / kWave;

__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) { return ~wave_max_u64(~v); }

// Block-wide exclusive scan of v (returns the prefix, the total in *tot).
__device__ int lru_block_scan(int v, int* s_tmp, int* tot) {
  const int lane = lane_id();
  const int w = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  if (lane == kWave - 1) s_tmp[w] = x;
  __syncthreads();
  if (w == 0) {
    int t = lane < kLruWaves ? s_tmp[lane] : 0;
#pragma unroll
    for (int o = 1; o < kLruWaves; o <<= 1) {
      const int y = __shfl_up(t, o, kWave);
      if (lane >= o) t += y;
    }
    if (lane < kLruWaves) s_tmp[kLruWaves + lane] = t;
  }
  __syncthreads();
  const int before = w == 0 ? 0 : s_tmp[kLruWaves + w - 1];
  *tot = s_tmp[2 * kLruWaves - 1];
  __syncthreads();
  return before + x - v;
}

// One workgroup.  LDS: seen state per expert (0 unseen, 1 resident, 2
// missing), the ordered miss list, the slots' usage and the sort keys.
__global__ void __launch_bounds__(kLruThreads) lru_ensure_kernel(LruArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int E = a.num_experts, S = a.cache_size;
  int64_t* u = reinterpret_cast<int64_t*>(lds);                 // [S]
  uint64_t* keys = reinterpret_cast<uint64_t*>(u + S);          // [P] (recency order)
  int* list = reinterpret_cast<int*>(keys + a.sort_len);        // [E]
  uint8_t* seen = reinterpret_cast<uint8_t*>(list + E);         // [E]
  __shared__ int s_tmp[2 * kLruWaves];
  __shared__ uint64_t s_min[kLruWaves];
  const int tid = threadIdx.x, lane = lane_id(), w = tid / kWave;
  const int base = a.layer * E;
  const int64_t step = a.step[0] + 1;

  for (int e = tid; e < E; e += kLruThreads) seen[e] = 0;
  for (int s = tid; s < S; s += kLruThreads) u[s] = a.usage[s];
  __syncthreads();
  for (int i = tid; i < a.numel; i += kLruThreads) {
    const int e = a.ids[i];
    if (e >= 0 && e < E) seen[e] = 1;  // every writer stores the same value
  }
  __syncthreads();
  // touch the resident seen experts; mark the missing ones
  const int per = (E + kLruThreads - 1) / kLruThreads;  // contiguous experts per thread
  int nmiss = 0, nact = 0;
  for (int q = 0; q < per; ++q) {
    const int e = tid * per + q;
    if (e < E && seen[e]) {
      ++nact;
      const int s = a.slot_for_id[base + e];
      if (s >= 0 && s < S) {
        u[s] = step;
      } else {
        seen[e] = 2;
        ++nmiss;
      }
    }
  }
  int m = 0;
  int pos = lru_block_scan(nmiss, s_tmp, &m);  // its barriers publish the touched usage
  for (int q = 0; q < per; ++q) {
    const int e = tid * per + q;
    if (e < E && seen[e] == 2) list[pos++] = e;
  }
  int nfree_local = 0;
  for (int s = tid; s < S; s += kLruThreads) nfree_local += u[s] < step ? 1 : 0;
  int nfree = 0;
  (void)lru_block_scan(nfree_local, s_tmp, &nfree);
  if (a.recency) {
    // (most recent first, then ascending id): ascending sort of
    // (max - recency) << 13 | id over the miss list padded to sort_len
    constexpr uint64_t kRecMax = (1ull << 51) - 1;
    for (int i = tid; i < a.sort_len; i += kLruThreads) {
      if (i < m) {
        const int e = list[i];
        const int64_t r = a.recency[e];
        const uint64_t rr = r < 0 ? 0 : (static_cast<uint64_t>(r) > kRecMax ? kRecMax : static_cast<uint64_t>(r));
        keys[i] = ((kRecMax - rr) << 13) | static_cast<uint64_t>(e);
      } else {
        keys[i] = ~0ull;
      }
    }
    __syncthreads();
    for (int k = 2; k <= a.sort_len; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < a.sort_len; i += kLruThreads) {
          const int p = i ^ j;
          if (p > i) {
            const uint64_t x = keys[i], y = keys[p];
            const bool up = (i & k) == 0;
            if ((x > y) == up) {
              keys[i] = y;
              keys[p] = x;
            }
          }
        }
        __syncthreads();
      }
    }
    for (int i = tid; i < m; i += kLruThreads) list[i] = static_cast<int>(keys[i] & 0x1FFFu);
    __syncthreads();
  }
  int nfetch = a.max_fetch < 0 ? m : min(m, a.max_fetch);
  if (a.fetch_frac_q16 > 0) {
    const long long f = a.fetch_frac_q16, q = 1ll << 16;
    const long long lo = (static_cast<long long>(m) * f) >> 16;
    const long long c0 = max(lo * (q - f), (m - lo) * f), c1 = max((lo + 1) * (q - f), (m - lo - 1) * f);
    nfetch = min(m, static_cast<int>(c0 <= c1 ? lo : lo + 1));
  }
  const int wanted = nfetch;
  nfetch = min(nfetch, min(a.capacity, nfree));
  if (tid == 0) {
    a.num_missing[0] = m;
    a.num_indices[0] = nfetch;
    if (a.unserved && wanted > nfetch) atomicAdd(reinterpret_cast<unsigned long long*>(a.unserved),
                                                 static_cast<unsigned long long>(wanted - nfetch));
  }
  // admission, one miss after the other: the slot with the smallest (usage, slot)
  for (int idx = 0; idx < nfetch; ++idx) {
    uint64_t best = ~0ull;
    for (int s = tid; s < S; s += kLruThreads)
      best = min(best, (static_cast<uint64_t>(u[s] < 0 ? 0 : u[s]) << 13) | static_cast<uint64_t>(s));
    best = wave_min_u64(best);
    if (lane == 0) s_min[w] = best;
    __syncthreads();
    if (tid == 0) {
      uint64_t b = s_min[0];
      for (int v = 1; v < kLruWaves; ++v) b = min(b, s_min[v]);
      const int vic = static_cast<int>(b & 0x1FFFu);
      const int e = list[idx];
      const int old = a.id_of_slot[vic];
      if (old >= 0 && old < a.num_layers * E) a.slot_for_id[old] = -1;
      a.id_of_slot[vic] = base + e;
      a.slot_for_id[base + e] = vic;
      u[vic] = step;
      a.evict_slots[idx] = vic;
      a.src_indices[idx] = e;
    }
    __syncthreads();
  }
  for (int s = tid; s < S; s += kLruThreads) a.usage[s] = u[s];
  if (a.recency)
    for (int e = tid; e < E; e += kLruThreads)
      if (seen[e]) a.recency[e] = step;
  unsigned long long missed = 0;
  for (int i = tid; i < a.numel; i += kLruThreads) {
    const int e = a.ids[i];
    const bool valid = e >= 0 && e < E;
    if (valid && seen[e] == 2) ++missed;
    const int s = valid ? a.slot_for_id[base + e] : -1;
    a.ids[i] = s;
    if (a.cpu_ids) a.cpu_ids[i] = valid && s < 0 ? e : -1;
  }
  if (tid == 0) a.step[0] = step;
  if (a.stats) {
    const unsigned long long t_act = wave_sum_u64(static_cast<unsigned long long>(nact));
    const unsigned long long t_miss = wave_sum_u64(static_cast<unsigned long long>(nmiss));
    const unsigned long long t_missed = wave_sum_u64(missed);
    auto* st = reinterpret_cast<unsigned long long*>(a.stats);
    if (lane == 0) {
      if (t_act) atomicAdd(st + 0, t_act);
      if (t_miss) atomicAdd(st + 1, t_miss);
      if (t_missed) atomicAdd(st + 3, t_missed);
      if (tid == 0) atomicAdd(st + 2, 1ull);
    }
  }
}

size_t lru_lds_bytes(int num_experts, int cache_size, int sort_len) {
  return static_cast<size_t>(cache_size) * 8 + static_cast<size_t>(sort_len) * 8 +
         static_cast<size_t>(num_experts) * 4 + ((static_cast<size_t>(num_experts) + 15) / 16 * 16);
}

hipError_t launch_lru_ensure(const LruArgs& a, hipStream_t stream) {
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(lru_ensure_kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 4096);
    if (err != hipSuccess) return err;
    attr_set = true;
  }
  hipLaunchKernelGGL(lru_ensure_kernel, dim3(1), dim3(kLruThreads), lru_lds_bytes(a.num_experts, a.cache_size, a.sort_len),
                     stream, a);
  return hipGetLastError();
}

// ----------------------------------------------------------------------------
// Whole-layer placement for the prefill (reference: _materialize_layer_kernel,
// moe/offload_kernels.py:250-281): expert e of the layer goes to slot e.  Slots
// holding this layer's experts are emptied (usage 0: the next victims); the
// other layers' experts in slots [0, E) lose their mapping; step += 1; slots
// [0, E) get this layer's experts with usage = step and are listed as the
// entries (e -> e) of the gather.  Every slot is read before it is written by
// the same thread, and the slot_for_id rows written (other layers' unmaps,
// this layer's map) are disjoint, so one pass suffices.
// ----------------------------------------------------------------------------
__global__ void __launch_bounds__(kLruThreads) materialize_layer_kernel(PlaceArgs a) {
  const int E = a.num_experts, tid = threadIdx.x;
  const int base = a.layer * E;
  const long long step = a.step[0] + 1;
  for (int s = tid; s < a.cache_size; s += kLruThreads) {
    const int old = a.id_of_slot[s];
    const bool same = old >= base && old < base + E;
    if (same) {
      a.id_of_slot[s] = -1;
      a.usage[s] = 0;
    } else if (s < E && old >= 0 && old < a.num_layers * E) {
      a.slot_for_id[old] = -1;
    }
  }
  __syncthreads();
  for (int e = tid; e < E; e += kLruThreads) {
    a.id_of_slot[e] = base + e;
    a.slot_for_id[base + e] = e;
    a.usage[e] = step;
    a.evict_slots[e] = e;
    a.src_indices[e] = e;
  }
  if (tid == 0) {
    a.step[0] = step;
    a.num_indices[0] = E;
  }
}

// Release of slots [slot_begin, slot_end) (reference: _invalidate_prefill_buffer,
// moe/offload_cache.py:592-600): their experts lose their mapping, the slots
// become empty with usage 0.
__global__ void __launch_bounds__(kLruThreads) release_slots_kernel(PlaceArgs a) {
  for (int s = a.slot_begin + static_cast<int>(blockIdx.x * kLruThreads + threadIdx.x); s < a.slot_end;
       s += static_cast<int>(gridDim.x * kLruThreads)) {
    const int old = a.id_of_slot[s];
    if (old >= 0 && old < a.num_layers * a.num_experts) a.slot_for_id[old] = -1;
    a.id_of_slot[s] = -1;
    a.usage[s] = 0;
  }
}

hipError_t launch_materialize_layer(const PlaceArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(materialize_layer_kernel, dim3(1), dim3(kLruThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_release_slots(const PlaceArgs& a, hipStream_t stream) {
  const int n = a.slot_end - a.slot_begin;
  if (n <= 0) return hipSuccess;
  const int blocks = (n + kLruThreads - 1) / kLruThreads;
  hipLaunchKernelGGL(release_slots_kernel, dim3(blocks), dim3(kLruThreads), 0, stream, a);
  return hipGetLastError();
}

// ----------------------------------------------------------------------------
// Hit compaction of the prefill double buffer's hit/miss split (reference:
// prefill_hit_compact and its kernel, moe/offload_kernels.py:63-86): the
// experts of one layer resident outside the two buffers (slot >= threshold,
// the buffers own the slots below) are listed in ascending expert order as
// (buffer row dst_base + e, cache slot), for a device-to-device gather.  One
// workgroup; a block scan keeps the order.
// ----------------------------------------------------------------------------
__global__ void __launch_bounds__(kLruThreads) hit_compact_kernel(const int32_t* slot_row, int num_experts,
                                                                  int threshold, int dst_base, int32_t* dst_rows,
                                                                  int32_t* src_rows, int32_t* num) {
  __shared__ int s_tmp[2 * kLruWaves];
  const int per = (num_experts + kLruThreads - 1) / kLruThreads;  // contiguous experts per thread
  const int e0 = threadIdx.x * per;
  int mine = 0;
  for (int q = 0; q < per; ++q) {
    const int e = e0 + q;
    if (e < num_experts && slot_row[e] >= threshold) ++mine;
  }
  int total = 0;
  int pos = lru_block_scan(mine, s_tmp, &total);
  for (int q = 0; q < per; ++q) {
    const int e = e0 + q;
    if (e >= num_experts) break;
    const int s = slot_row[e];
    if (s >= threshold) {
      dst_rows[pos] = dst_base + e;
      src_rows[pos] = s;
      ++pos;
    }
  }
  if (threadIdx.x == 0) num[0] = total;
}

hipError_t launch_hit_compact(const int32_t* slot_row, int num_experts, int threshold, int dst_base, int32_t* dst_rows,
                              int32_t* src_rows, int32_t* num, hipStream_t stream) {
  hipLaunchKernelGGL(hit_compact_kernel, dim3(1), dim3(kLruThreads), 0, stream, slot_row, num_experts, threshold,
                     dst_base, dst_rows, src_rows, num);
  return hipGetLastError();
}

// ----------------------------------------------------------------------------
// Gather of admitted experts: entry i copies row src_indices[i] of every host
// bank to row evict_slots[i] of the matching slot bank, for i < num_indices[0]
// (reference: fast_index_copy_multi over the banks of copy_missing,
// moe/offload_cache.py:968-1010).  Work items are (entry, bank, 64 KiB chunk);
// a fixed grid walks them, each lane moving 16-byte pieces with a few loads in
// flight.  The host rows are read in place (pinned, mapped), so the copy is
// PCIe-bound.
// ----------------------------------------------------------------------------
constexpr int kFetchThreads = 256;
constexpr int kFetchChunk = 64 * 1024;

__global__ void __launch_bounds__(kFetchThreads) fetch_experts_kernel(FetchArgs a) {
  const int n = min(a.num_indices[0], a.max_entries);
  const long long items = static_cast<long long>(n) * a.chunks_per_entry;
  for (long long it = blockIdx.x; it < items; it += gridDim.x) {
    const int i = static_cast<int>(it / a.chunks_per_entry);
    int c = static_cast<int>(it % a.chunks_per_entry);
    int b = 0;
    while (b + 1 < a.nbanks && c >= a.chunk_start[b + 1]) ++b;
    c -= a.chunk_start[b];
    const uint64_t rb = a.row_bytes[b];
    const uint8_t* src = a.src[b] + static_cast<uint64_t>(a.src_indices[i]) * rb;
    uint8_t* dst = a.dst[b] + static_cast<uint64_t>(a.evict_slots[i]) * rb;
    const uint64_t lo = static_cast<uint64_t>(c) * kFetchChunk;
    const uint64_t hi = lo + kFetchChunk < rb ? lo + kFetchChunk : rb;
    constexpr int kAhead = 4;
    for (uint64_t off = lo + static_cast<uint64_t>(threadIdx.x) * 16; off < hi;
         off += static_cast<uint64_t>(kFetchThreads) * 16 * kAhead) {
      u32x4 v[kAhead];
#pragma unroll
      for (int k = 0; k < kAhead; ++k) {
        const uint64_t o = off + static_cast<uint64_t>(k) * kFetchThreads * 16;
        if (o < hi) v[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + o));
      }
#pragma unroll
      for (int k = 0; k < kAhead; ++k) {
        const uint64_t o = off + static_cast<uint64_t>(k) * kFetchThreads * 16;
        if (o < hi) *reinterpret_cast<u32x4*>(dst + o) = v[k];
      }
    }
  }
}

hipError_t launch_fetch_experts(const FetchArgs& a, int max_entries, hipStream_t stream) {
  const long long items = static_cast<long long>(max_entries) * a.chunks_per_entry;
  const int grid = static_cast<int>(items < 2048 ? (items > 0 ? items : 1) : 2048);
  hipLaunchKernelGGL(fetch_experts_kernel, dim3(grid), dim3(kFetchThreads), 0, stream, a);
  return hipGetLastError();
}

int fetch_chunks(uint64_t row_bytes) { return static_cast<int>((row_bytes + kFetchChunk - 1) / kFetchChunk); }

}  // namespace ftmoe
