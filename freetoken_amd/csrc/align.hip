// Deterministic token -> expert permutation (moe_align_block_size) with an
// optional expert-cache slot lookup in front of it.
//
// Contract (reference moe/fused.py:88-158, kernel/triton/moe_align.py:1-44):
//   effective_E = num_experts + 1, ids outside [0, effective_E) ignored;
//   counts padded to block_size, exclusive prefix sum -> region starts;
//   expert_ids per block; num_tokens_post_pad; sorted_ids filled with the
//   sentinel numel.  The reference ranks routes inside an expert with atomics;
//   here the order is the canonical stable one: ascending flat route index.
//
// Decode-sized calls (at most 64 routes, block size 1) take one wave
// (align_wave.h).  Otherwise one workgroup of 16 waves does everything
// (align_kernel; the multi-workgroup variant below for prefill).  The routes
// are cut into 16 contiguous chunks, one per wave.  Pass 1 counts per (wave,
// expert) with LDS atomics (order-free).  A scan over waves turns the counts
// into per-wave bases, a scan over experts gives the padded region starts.
// Pass 2 walks each chunk in 64-route batches in order; a 64-key bitonic sort
// of (expert << 6 | lane) inside the wave yields, for every route, its rank
// among the equal-expert routes of the batch, so the final position is
// region_start[e] + wave_base[w][e] + rank -- no atomics, fully deterministic.
#include <algorithm>

#include "align_wave.h"
#include "kernels.h"

namespace ftmoe {

constexpr int kAlignWaves = 16;
constexpr int kAlignThreads = kAlignWaves * kWave;


// Block-wide exclusive scan of v over all threads (returns prefix, total in *tot).
__device__ int block_exclusive_scan(int v, int* s_tmp, int* tot) {
  const int lane = lane_id();
  const int w = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  if (lane == kWave - 1) s_tmp[w] = x;
  __syncthreads();
  if (w == 0) {
    int s = (lane < kAlignWaves) ? s_tmp[lane] : 0;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int y = __shfl_up(s, off, kWave);
      if (lane >= off) s += y;
    }
    if (lane < kAlignWaves) s_tmp[kAlignWaves + lane] = s;  // inclusive per wave
  }
  __syncthreads();
  const int wave_prefix = (w == 0) ? 0 : s_tmp[kAlignWaves + w - 1];
  *tot = s_tmp[2 * kAlignWaves - 1];
  __syncthreads();
  return wave_prefix + x - v;
}

__global__ void __launch_bounds__(kAlignThreads) align_kernel(AlignArgs a) {
  extern __shared__ int lds[];
  const int eff = a.num_experts + 1;
  int* wcount = lds;                          // [kAlignWaves][eff]
  int* cum = wcount + kAlignWaves * eff;      // [eff + 1]
  int* cnt = cum + eff + 1;                   // [eff]
  int* seen = cnt + eff;                      // [table_size] (stats only)
  __shared__ int s_tmp[2 * kAlignWaves];

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int w = tid / kWave;
  // routes go to the first nw waves (64 or more each); the others only help
  // with the per-expert work
  const int nw = min(kAlignWaves, max(1, (a.numel + kWave - 1) / kWave));
  const int chunk = ((a.numel + nw - 1) / nw + kWave - 1) / kWave * kWave;
  const int c0 = min(a.numel, w * chunk);
  const int c1 = min(a.numel, c0 + chunk);

  for (int i = tid; i < nw * eff; i += kAlignThreads) wcount[i] = 0;
  if (a.stats)
    for (int i = tid; i < a.table_size; i += kAlignThreads) seen[i] = 0;
  __syncthreads();

  // ---- pass 0: optional slot lookup; pass 1: per-wave counts
  long long missed = 0;
  for (int i = c0 + lane; i < c1; i += kWave) {
    int e = a.ids[i];
    if (a.slot_for_id) {
      const bool valid = e >= 0 && e < a.table_size;
      const int s = valid ? a.slot_for_id[e] : -1;
      if (a.slot_ids) a.slot_ids[i] = s;
      if (a.miss_mask) a.miss_mask[i] = (valid && s < 0) ? 1 : 0;
      if (a.stats && valid) seen[e] = s < 0 ? 2 : 1;  // every writer of e stores the same value
      if (valid && s < 0) ++missed;
      e = s;
    }
    if (e >= 0 && e < eff) atomicAdd(&wcount[w * eff + e], 1);
  }
  __syncthreads();

  // ---- scan over waves (per expert) and padded scan over experts
  const int per = (eff + kAlignThreads - 1) / kAlignThreads;
  int local = 0, local_seg = 0;
  for (int q = 0; q < per; ++q) {
    const int e = tid * per + q;
    if (e < eff) {
      int acc = 0;
      for (int v = 0; v < nw; ++v) {
        const int t = wcount[v * eff + e];
        wcount[v * eff + e] = acc;
        acc += t;
      }
      cnt[e] = acc;
      local += (acc + a.block_size - 1) / a.block_size * a.block_size;
      if (a.seg_expert && e < a.num_experts) local_seg += (acc + a.seg_cap - 1) / a.seg_cap;
    }
  }
  int total = 0, total_seg = 0;
  int pre = block_exclusive_scan(local, s_tmp, &total);
  int pre_seg = block_exclusive_scan(local_seg, s_tmp, &total_seg);
  for (int q = 0; q < per; ++q) {
    const int e = tid * per + q;
    if (e < eff) {
      cum[e] = pre;
      if (a.cum_out) a.cum_out[e] = pre;
      const int c = cnt[e];
      if (a.seg_expert && e < a.num_experts) {
        for (int s0 = 0; s0 < c; s0 += a.seg_cap) {
          a.seg_expert[pre_seg] = e;
          a.seg_start[pre_seg] = pre + s0;
          a.seg_count[pre_seg] = min(a.seg_cap, c - s0);
          ++pre_seg;
        }
      }
      pre += (c + a.block_size - 1) / a.block_size * a.block_size;
    }
  }
  if (tid == 0) {
    cum[eff] = total;
    if (a.cum_out) a.cum_out[eff] = total;
    a.ntpp[0] = total;
    if (a.n_seg) a.n_seg[0] = total_seg;
  }
  // sentinel fill (ordered before the scatter by the barrier below)
  for (int i = tid; i < a.max_padded; i += kAlignThreads) a.sorted_ids[i] = a.numel;
  __syncthreads();
  // expert id of every used block; -1 for unused blocks (callers that read only
  // the segments pass no expert_ids)
  for (int b = tid; a.expert_ids && b < a.max_blocks; b += kAlignThreads) {
    int e = -1;
    if (b * a.block_size < total) {
      int lo = 0, hi = eff;  // largest e with cum[e] <= b*bs and cnt[e] > 0
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (cum[mid] <= b * a.block_size) lo = mid; else hi = mid;
      }
      e = lo;
    }
    a.expert_ids[b] = e;
  }
  if (a.stats) {
    // distinct active / missing experts (seen since the barrier after pass 1)
    // and missed routes: order-free integer sums straight into the counters
    unsigned long long act = 0, miss = 0;
    for (int e = tid; e < a.table_size; e += kAlignThreads) {
      act += seen[e] != 0;
      miss += seen[e] == 2;
    }
    const unsigned long long t_act = wave_sum_u64(act), t_miss = wave_sum_u64(miss);
    const unsigned long long t_missed = wave_sum_u64(static_cast<unsigned long long>(missed));
    auto* st = reinterpret_cast<unsigned long long*>(a.stats);
    if (lane == 0) {
      if (t_act) atomicAdd(st + 0, t_act);
      if (t_miss) atomicAdd(st + 1, t_miss);
      if (t_missed) atomicAdd(st + 3, t_missed);
      if (tid == 0) atomicAdd(st + 2, 1ull);
    }
  }

  // ---- pass 2: stable scatter, 64 routes at a time per wave
  for (int base = c0; base < c1; base += kWave) {
    const int i = base + lane;
    int e = -1;
    if (i < c1) {
      if (a.slot_for_id && a.slot_ids) {
        e = a.slot_ids[i];  // written by this lane in pass 1 (may alias ids)
      } else {
        e = a.ids[i];
        if (a.slot_for_id) e = (e >= 0 && e < a.table_size) ? a.slot_for_id[e] : -1;
      }
    }
    const bool valid = e >= 0 && e < eff;
    const uint32_t key = wave_sort64((static_cast<uint32_t>(valid ? e : 0xFFFFF) << 6) | static_cast<uint32_t>(lane));
    const int se = static_cast<int>(key >> 6);
    const int prev = __shfl(se, lane == 0 ? 0 : lane - 1, kWave);
    const int next = __shfl(se, lane == kWave - 1 ? lane : lane + 1, kWave);
    const bool head = lane == 0 || prev != se;
    const bool tail = lane == kWave - 1 || next != se;
    const unsigned long long heads = __ballot(head);
    const unsigned long long upto = (lane == kWave - 1) ? ~0ull : ((2ull << lane) - 1ull);
    const int run_start = kWave - 1 - __clzll(heads & upto);
    const int rank = lane - run_start;
    if (se < eff) {
      const int src_lane = static_cast<int>(key & 63u);
      const int pos = cum[se] + wcount[w * eff + se] + rank;
      a.sorted_ids[pos] = base + src_lane;
    }
    // A wave issues its LDS reads (above) before this write, so every lane saw
    // the base from before this batch.
    if (se < eff && tail) wcount[w * eff + se] += rank + 1;
  }
}

// ----------------------------------------------------------------------------
// Multi-workgroup align for large route counts (prefill): the same stable
// order, with the routes cut into B workgroups x 16 contiguous wave chunks.
//   align_count_kernel:   per (wave, expert) counts -> wcnt[B*16][eff] and per
//                         (workgroup, expert) totals -> btot[B][eff]; fills
//                         sorted_ids with the sentinel.
//   align_scan_kernel:    one workgroup: per expert, exclusive prefix of the
//                         workgroup totals; padded region starts; expert_ids;
//                         btot becomes the absolute base of every workgroup.
//   align_scatter_kernel: per workgroup, wave bases = workgroup base + prefix
//                         of the earlier waves' counts; each wave walks its
//                         chunk in 64-route batches, the 64-key bitonic rank
//                         giving every route its slot.
// ----------------------------------------------------------------------------
__device__ __forceinline__ void chunk_of(int numel, int gw, int waves, int& c0, int& c1) {
  const int chunk = ((numel + waves - 1) / waves + kWave - 1) / kWave * kWave;
  c0 = min(numel, gw * chunk);
  c1 = min(numel, c0 + chunk);
}

__global__ void __launch_bounds__(kAlignThreads) align_count_kernel(AlignArgs a, int32_t* wcnt, int32_t* btot) {
  extern __shared__ int lds[];
  const int eff = a.num_experts + 1;
  int* wcount = lds;  // [kAlignWaves][eff]
  const int tid = threadIdx.x, lane = lane_id(), w = tid / kWave;
  const int waves = gridDim.x * kAlignWaves, gw = blockIdx.x * kAlignWaves + w;
  for (int i = tid; i < kAlignWaves * eff; i += kAlignThreads) wcount[i] = 0;
  for (int i = blockIdx.x * kAlignThreads + tid; i < a.max_padded; i += gridDim.x * kAlignThreads)
    a.sorted_ids[i] = a.numel;
  __syncthreads();
  int c0, c1;
  chunk_of(a.numel, gw, waves, c0, c1);
  for (int i = c0 + lane; i < c1; i += kWave) {
    const int e = a.ids[i];
    if (e >= 0 && e < eff) atomicAdd(&wcount[w * eff + e], 1);
  }
  __syncthreads();
  for (int i = tid; i < kAlignWaves * eff; i += kAlignThreads)
    wcnt[static_cast<size_t>(blockIdx.x * kAlignWaves) * eff + i] = wcount[i];
  for (int e = tid; e < eff; e += kAlignThreads) {
    int t = 0;
#pragma unroll
    for (int v = 0; v < kAlignWaves; ++v) t += wcount[v * eff + e];
    btot[static_cast<size_t>(blockIdx.x) * eff + e] = t;
  }
}

__global__ void __launch_bounds__(kAlignThreads) align_scan_kernel(AlignArgs a, int32_t* btot, int blocks) {
  extern __shared__ int lds[];
  const int eff = a.num_experts + 1;
  int* cum = lds;            // [eff + 1]
  int* cnt = cum + eff + 1;  // [eff]
  __shared__ int s_tmp[2 * kAlignWaves];
  const int tid = threadIdx.x;
  for (int e = tid; e < eff; e += kAlignThreads) {
    int acc = 0;
    for (int b = 0; b < blocks; ++b) {
      const size_t at = static_cast<size_t>(b) * eff + e;
      const int t = btot[at];
      btot[at] = acc;
      acc += t;
    }
    cnt[e] = acc;
  }
  __syncthreads();
  const int per = (eff + kAlignThreads - 1) / kAlignThreads;
  int local = 0;
  for (int q = 0; q < per; ++q) {
    const int e = tid * per + q;
    if (e < eff) local += (cnt[e] + a.block_size - 1) / a.block_size * a.block_size;
  }
  int total = 0;
  int pre = block_exclusive_scan(local, s_tmp, &total);
  for (int q = 0; q < per; ++q) {
    const int e = tid * per + q;
    if (e < eff) {
      cum[e] = pre;
      if (a.cum_out) a.cum_out[e] = pre;
      pre += (cnt[e] + a.block_size - 1) / a.block_size * a.block_size;
    }
  }
  if (tid == 0) {
    cum[eff] = total;
    if (a.cum_out) a.cum_out[eff] = total;
    a.ntpp[0] = total;
  }
  __syncthreads();
  for (int b = tid; b < a.max_blocks; b += kAlignThreads) {
    int e = -1;
    if (b * a.block_size < total) {
      int lo = 0, hi = eff;  // largest e with cum[e] <= b*bs
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (cum[mid] <= b * a.block_size) lo = mid; else hi = mid;
      }
      e = lo;
    }
    a.expert_ids[b] = e;
  }
  for (int i = tid; i < blocks * eff; i += kAlignThreads) btot[i] += cum[i % eff];
}

__global__ void __launch_bounds__(kAlignThreads) align_scatter_kernel(AlignArgs a, const int32_t* wcnt,
                                                                      const int32_t* btot) {
  extern __shared__ int lds[];
  const int eff = a.num_experts + 1;
  int* wbase = lds;  // [kAlignWaves][eff]
  const int tid = threadIdx.x, lane = lane_id(), w = tid / kWave;
  const int waves = gridDim.x * kAlignWaves, gw = blockIdx.x * kAlignWaves + w;
  const int32_t* mine = wcnt + static_cast<size_t>(blockIdx.x * kAlignWaves) * eff;
  for (int e = tid; e < eff; e += kAlignThreads) {
    int acc = btot[static_cast<size_t>(blockIdx.x) * eff + e];
#pragma unroll
    for (int v = 0; v < kAlignWaves; ++v) {
      wbase[v * eff + e] = acc;
      acc += mine[v * eff + e];
    }
  }
  __syncthreads();
  int c0, c1;
  chunk_of(a.numel, gw, waves, c0, c1);
  for (int base = c0; base < c1; base += kWave) {
    const int i = base + lane;
    const int e = i < c1 ? a.ids[i] : -1;
    const bool valid = e >= 0 && e < eff;
    const uint32_t key = wave_sort64((static_cast<uint32_t>(valid ? e : 0xFFFFF) << 6) | static_cast<uint32_t>(lane));
    const int se = static_cast<int>(key >> 6);
    const int prev = __shfl(se, lane == 0 ? 0 : lane - 1, kWave);
    const int next = __shfl(se, lane == kWave - 1 ? lane : lane + 1, kWave);
    const bool head = lane == 0 || prev != se;
    const bool tail = lane == kWave - 1 || next != se;
    const unsigned long long heads = __ballot(head);
    const unsigned long long upto = (lane == kWave - 1) ? ~0ull : ((2ull << lane) - 1ull);
    const int run_start = kWave - 1 - __clzll(heads & upto);
    const int rank = lane - run_start;
    if (se < eff) a.sorted_ids[wbase[w * eff + se] + rank] = base + static_cast<int>(key & 63u);
    // the wave reads its bases (above) before this write
    if (se < eff && tail) wbase[w * eff + se] += rank + 1;
  }
}

int align_grid_blocks(int numel) {
  const int b = (numel + 4095) / 4096;  // ~4 K routes per workgroup (256 per wave)
  return b < 1 ? 1 : (b > 64 ? 64 : b);
}

size_t align_gcount_ints(int numel, int num_experts) {
  return static_cast<size_t>(align_grid_blocks(numel)) * (kAlignWaves + 1) * (num_experts + 1);
}

hipError_t launch_align_large(const AlignArgs& a, int32_t* gcount, hipStream_t stream) {
  const int eff = a.num_experts + 1;
  const int blocks = align_grid_blocks(a.numel);
  int32_t* wcnt = gcount;                                                   // [blocks * 16][eff]
  int32_t* btot = gcount + static_cast<size_t>(blocks) * kAlignWaves * eff;  // [blocks][eff]
  const size_t lds_w = sizeof(int) * static_cast<size_t>(kAlignWaves) * eff;
  const size_t lds_s = sizeof(int) * (2 * static_cast<size_t>(eff) + 1);
  static bool attr_set = false;
  if (!attr_set) {
    for (const void* f : {reinterpret_cast<const void*>(align_count_kernel),
                          reinterpret_cast<const void*>(align_scatter_kernel)}) {
      const hipError_t err = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 1024);
      if (err != hipSuccess) return err;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL(align_count_kernel, dim3(blocks), dim3(kAlignThreads), lds_w, stream, a, wcnt, btot);
  hipLaunchKernelGGL(align_scan_kernel, dim3(1), dim3(kAlignThreads), lds_s, stream, a, btot, blocks);
  hipLaunchKernelGGL(align_scatter_kernel, dim3(blocks), dim3(kAlignThreads), lds_w, stream, a,
                     static_cast<const int32_t*>(wcnt), static_cast<const int32_t*>(btot));
  return hipGetLastError();
}

// One-wave align for decode-sized calls (align_wave.h).
__global__ void __launch_bounds__(kWave) align_wave_kernel(AlignArgs a) { align_small(a, a.ids); }

// ----------------------------------------------------------------------------
// Decode-form align for banks of many rows (an expert cache of thousands of
// slots): block size 1, segments, no padding.  The counting kernel above keeps
// per-wave counts of every row in LDS; here the LDS holds one key per route
// instead, so the row count is free (up to kSortMaxRows) and the route count
// is bounded (kSortMaxRoutes).  One workgroup:
//   1. optional slot lookup (as pass 0 of align_kernel; distinct seen and
//      missing experts marked in LDS bitmaps), key = row << 14 | route, or
//      ~0 for routes outside [0, rows + 1);
//   2. ascending bitonic sort of the keys in LDS: the stable order, since
//      equal rows order by route;
//   3. position p of the sorted keys is the route's place (block size 1);
//      a row's run is found by binary search, segment starts are every
//      seg_cap-th place of a run, numbered by a block scan.
// The outputs are identical to align_kernel's for the same call.
// ----------------------------------------------------------------------------
constexpr int kSortShift = 14;
constexpr uint32_t kSortRouteMask = (1u << kSortShift) - 1u;

__device__ __forceinline__ int sorted_lower_bound(const uint32_t* keys, int n, uint32_t v) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (keys[mid] < v) lo = mid + 1; else hi = mid;
  }
  return lo;
}

__global__ void __launch_bounds__(kAlignThreads) align_sort_kernel(AlignArgs a, int P) {
  extern __shared__ __attribute__((aligned(16))) uint32_t skeys[];  // [P] keys, then the bitmaps
  const int words = a.stats && a.slot_for_id ? (a.table_size + 31) / 32 : 0;
  uint32_t* seen_bits = skeys + P;
  uint32_t* miss_bits = seen_bits + words;
  __shared__ int s_tmp[2 * kAlignWaves];
  const int tid = threadIdx.x, lane = lane_id();
  const int eff = a.num_experts + 1;
  for (int i = tid; i < words; i += kAlignThreads) {
    seen_bits[i] = 0;
    miss_bits[i] = 0;
  }
  __syncthreads();
  unsigned long long missed = 0;
  for (int i = tid; i < P; i += kAlignThreads) {
    uint32_t key = ~0u;
    if (i < a.numel) {
      int e = a.ids[i];
      if (a.slot_for_id) {
        const bool idv = e >= 0 && e < a.table_size;
        const int s = idv ? a.slot_for_id[e] : -1;
        if (a.slot_ids) a.slot_ids[i] = s;  // may alias ids: this thread read ids[i] above
        if (a.miss_mask) a.miss_mask[i] = (idv && s < 0) ? 1 : 0;
        if (words && idv) {
          atomicOr(&seen_bits[e >> 5], 1u << (e & 31));
          if (s < 0) atomicOr(&miss_bits[e >> 5], 1u << (e & 31));
        }
        if (idv && s < 0) ++missed;
        e = s;
      }
      if (e >= 0 && e < eff) key = (static_cast<uint32_t>(e) << kSortShift) | static_cast<uint32_t>(i);
    }
    skeys[i] = key;
  }
  __syncthreads();
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < P; i += kAlignThreads) {
        const int p = i ^ j;
        if (p > i) {
          const uint32_t x = skeys[i], y = skeys[p];
          if ((x > y) == ((i & k) == 0)) {
            skeys[i] = y;
            skeys[p] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  // places, run bounds and segment starts over contiguous chunks of places
  const int per = (a.numel + kAlignThreads - 1) / kAlignThreads;
  const int p0 = min(a.numel, tid * per), p1 = min(a.numel, p0 + per);
  int nstart = 0;
  for (int p = p0; p < p1; ++p) {
    const uint32_t key = skeys[p];
    if (key == ~0u) break;  // invalid keys sort last
    const int e = static_cast<int>(key >> kSortShift);
    a.sorted_ids[p] = static_cast<int>(key & kSortRouteMask);
    if (p + 1 == a.numel || skeys[p + 1] == ~0u) a.ntpp[0] = p + 1;
    if (a.seg_expert && e < a.num_experts) {
      const int run0 = sorted_lower_bound(skeys, a.numel, static_cast<uint32_t>(e) << kSortShift);
      if ((p - run0) % a.seg_cap == 0) ++nstart;
    }
  }
  if (tid == 0 && (a.numel == 0 || skeys[0] == ~0u)) a.ntpp[0] = 0;
  int nseg = 0;
  int si = block_exclusive_scan(nstart, s_tmp, &nseg);
  if (a.seg_expert) {
    for (int p = p0; p < p1; ++p) {
      const uint32_t key = skeys[p];
      if (key == ~0u) break;
      const int e = static_cast<int>(key >> kSortShift);
      if (e >= a.num_experts) continue;
      const int run0 = sorted_lower_bound(skeys, a.numel, static_cast<uint32_t>(e) << kSortShift);
      if ((p - run0) % a.seg_cap != 0) continue;
      const int run1 = sorted_lower_bound(skeys, a.numel, static_cast<uint32_t>(e + 1) << kSortShift);
      a.seg_expert[si] = e;
      a.seg_start[si] = p;
      a.seg_count[si] = min(a.seg_cap, run1 - p);
      ++si;
    }
    if (tid == 0) a.n_seg[0] = nseg;
  }
  if (a.stats) {
    unsigned long long act = 0, miss = 0;
    for (int i = tid; i < words; i += kAlignThreads) {
      act += __popc(seen_bits[i]);
      miss += __popc(miss_bits[i]);
    }
    const unsigned long long t_act = wave_sum_u64(act), t_miss = wave_sum_u64(miss);
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

// Whether a call takes align_sort_kernel: the decode form over a bank too
// large for the counting kernel's per-row LDS.
inline bool align_takes_sort(const AlignArgs& a) {
  return a.num_experts > kCountMaxRows && a.block_size == 1 && a.max_padded == 0 && !a.expert_ids &&
         !a.cum_out;
}

size_t align_sort_lds_bytes(const AlignArgs& a, int P) {
  const int words = a.stats && a.slot_for_id ? (a.table_size + 31) / 32 : 0;
  return sizeof(uint32_t) * (static_cast<size_t>(P) + 2 * static_cast<size_t>(words));
}

hipError_t launch_align_sort(const AlignArgs& a, hipStream_t stream) {
  int P = 1;
  while (P < a.numel) P <<= 1;
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(align_sort_kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 1024);
    if (err != hipSuccess) return err;
    attr_set = true;
  }
  hipLaunchKernelGGL(align_sort_kernel, dim3(1), dim3(kAlignThreads), align_sort_lds_bytes(a, P), stream, a, P);
  return hipGetLastError();
}

size_t align_lds_bytes(int num_experts, int table_size, bool stats) {
  const int eff = num_experts + 1;
  return sizeof(int) * (static_cast<size_t>(kAlignWaves) * eff + (eff + 1) + eff + (stats ? table_size : 0));
}

hipError_t launch_align(const AlignArgs& a, hipStream_t stream) {
  if (align_fits_wave(a)) {
    hipLaunchKernelGGL(align_wave_kernel, dim3(1), dim3(kWave), 0, stream, a);
    return hipGetLastError();
  }
  if (align_takes_sort(a)) return launch_align_sort(a, stream);
  const size_t lds = align_lds_bytes(a.num_experts, a.table_size, a.stats != nullptr);
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(align_kernel),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 1024);
    if (err != hipSuccess) return err;
    attr_set = true;
  }
  hipLaunchKernelGGL(align_kernel, dim3(1), dim3(kAlignThreads), lds, stream, a);
  return hipGetLastError();
}

}  // namespace ftmoe

namespace ftmoe {

// Standalone expert-cache lookup: slot_ids[i] = slot_for_id[ids[i]] (-1 when
// absent or out of range) with the accumulated counters of the reference's
// decode statistics (distinct active / distinct missing experts, calls, missed
// routes).  One workgroup; slot_ids may alias ids.
__global__ void __launch_bounds__(1024) slot_map_kernel(const int32_t* ids, int numel, const int32_t* slot_for_id,
                                                        int table_size, int32_t* slot_ids, uint8_t* miss_mask,
                                                        long long* stats) {
  extern __shared__ int seen[];  // per expert: 0 unseen, 1 resident, 2 missing
  const int tid = threadIdx.x;
  if (stats) {
    for (int i = tid; i < table_size; i += blockDim.x) seen[i] = 0;
    __syncthreads();
  }
  unsigned long long missed = 0;
  for (int i = tid; i < numel; i += blockDim.x) {
    const int e = ids[i];
    const bool valid = e >= 0 && e < table_size;
    const int s = valid ? slot_for_id[e] : -1;
    slot_ids[i] = s;
    if (miss_mask) miss_mask[i] = (valid && s < 0) ? 1 : 0;
    if (stats && valid) seen[e] = s < 0 ? 2 : 1;  // every writer of e stores the same value
    missed += (valid && s < 0) ? 1 : 0;
  }
  if (!stats) return;
  __syncthreads();
  unsigned long long act = 0, miss = 0;
  for (int e = tid; e < table_size; e += blockDim.x) {
    act += seen[e] != 0;
    miss += seen[e] == 2;
  }
  // order-free integer sums straight into the counters (no read-back)
  const unsigned long long t_act = wave_sum_u64(act), t_miss = wave_sum_u64(miss), t_missed = wave_sum_u64(missed);
  auto* st = reinterpret_cast<unsigned long long*>(stats);
  if (lane_id() == 0) {
    if (t_act) atomicAdd(st + 0, t_act);
    if (t_miss) atomicAdd(st + 1, t_miss);
    if (t_missed) atomicAdd(st + 3, t_missed);
    if (tid == 0) atomicAdd(st + 2, 1ull);
  }
}

hipError_t launch_slot_map(const int32_t* ids, int numel, const int32_t* slot_for_id, int table_size,
                           int32_t* slot_ids, uint8_t* miss_mask, long long* stats, hipStream_t stream) {
  const size_t lds = stats ? sizeof(int) * static_cast<size_t>(table_size) : 0;
  hipLaunchKernelGGL(slot_map_kernel, dim3(1), dim3(1024), lds, stream, ids, numel, slot_for_id, table_size,
                     slot_ids, miss_mask, stats);
  return hipGetLastError();
}

// Routing histogram: freq[e] += number of routes with id e, ids outside
// [0, num_experts) skipped.  Each workgroup counts its stride of the routes
// in LDS, then adds its nonzero bins to freq (integer atomics: the sums do
// not depend on the order).
__global__ void __launch_bounds__(256) route_histogram_kernel(const int32_t* ids, int numel, int num_experts,
                                                              unsigned long long* freq) {
  extern __shared__ int bins[];
  for (int e = threadIdx.x; e < num_experts; e += blockDim.x) bins[e] = 0;
  __syncthreads();
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < numel; i += gridDim.x * blockDim.x) {
    const int e = ids[i];
    if (e >= 0 && e < num_experts) atomicAdd(&bins[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < num_experts; e += blockDim.x)
    if (bins[e]) atomicAdd(freq + e, static_cast<unsigned long long>(bins[e]));
}

hipError_t launch_route_histogram(const int32_t* ids, int numel, int num_experts, long long* freq,
                                  hipStream_t stream) {
  const int blocks = std::max(1, std::min((numel + 1023) / 1024, 64));
  hipLaunchKernelGGL(route_histogram_kernel, dim3(blocks), dim3(256), sizeof(int) * static_cast<size_t>(num_experts),
                     stream, ids, numel, num_experts, reinterpret_cast<unsigned long long*>(freq));
  return hipGetLastError();
}

}  // namespace ftmoe
