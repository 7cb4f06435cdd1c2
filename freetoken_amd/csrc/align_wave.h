// Wave-level pieces of the token -> expert permutation shared by align.hip and
// the fused router + align of route.hip: a 64-key bitonic sort and the
// one-wave align for decode-sized calls.
#pragma once

#include "kernels.h"

namespace ftmoe {

// Ascending 64-key bitonic sort across the lanes of a wave (lane 0 gets the
// smallest key).
__device__ __forceinline__ uint32_t wave_sort64(uint32_t key) {
  const int lane = lane_id();
#pragma unroll
  for (int k = 2; k <= kWave; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const uint32_t other = __shfl_xor(key, j, kWave);
      const bool up = (lane & k) == 0;
      const bool lower = (lane & j) == 0;
      key = (lower == up) ? min(key, other) : max(key, other);
    }
  }
  return key;
}

// ----------------------------------------------------------------------------
// One-wave align for decode-sized calls (at most 64 routes, block size 1, no
// padding, no expert_ids or region starts requested): the same outputs as
// align_kernel (align.hip) without a barrier; ids may live in LDS.  Lane i
// takes route i; one 64-key sort of (aligned id, route) gives the stable order
// directly (with block size 1 a
// route's position is the number of valid routes sorting before it); runs of
// equal ids give the segments; a second sort of (expert id, missing, route)
// gives the distinct-expert counters.
// ----------------------------------------------------------------------------
__device__ __forceinline__ void align_wave(const AlignArgs& a, const int32_t* ids) {
  const int lane = lane_id();
  const int eff = a.num_experts + 1;
  const unsigned long long below = (1ull << lane) - 1ull;  // lanes before this one
  const unsigned long long upto = below | (1ull << lane);
  int e = -1, id = -1;
  bool idv = false, miss = false;
  if (lane < a.numel) {
    e = ids[lane];
    if (a.slot_for_id) {
      id = e;
      idv = e >= 0 && e < a.table_size;
      const int s = idv ? a.slot_for_id[e] : -1;
      if (a.slot_ids) a.slot_ids[lane] = s;
      if (a.miss_mask) a.miss_mask[lane] = (idv && s < 0) ? 1 : 0;
      miss = idv && s < 0;
      e = s;
    }
  }
  const bool valid = e >= 0 && e < eff;
  const uint32_t key = wave_sort64((static_cast<uint32_t>(valid ? e : 0xFFFFF) << 6) | static_cast<uint32_t>(lane));
  const int se = static_cast<int>(key >> 6);
  const bool placed = se < eff;
  if (placed) a.sorted_ids[lane] = static_cast<int>(key & 63u);
  const int prev = __shfl(se, lane == 0 ? 0 : lane - 1, kWave);
  const unsigned long long heads = __ballot(lane == 0 || prev != se);
  const int run_start = kWave - 1 - __clzll(heads & upto);
  const unsigned long long later = heads & ~upto;  // run heads after this lane
  const int run_end = later ? __ffsll(static_cast<long long>(later)) - 2 : kWave - 1;
  if (a.seg_expert) {
    const bool sstart = se < a.num_experts && (lane - run_start) % a.seg_cap == 0;
    const unsigned long long smask = __ballot(sstart);
    if (sstart) {
      const int si = __popcll(smask & below);
      a.seg_expert[si] = se;
      a.seg_start[si] = lane;
      a.seg_count[si] = min(a.seg_cap, run_end - lane + 1);
    }
    if (lane == 0) a.n_seg[0] = __popcll(smask);
  }
  const unsigned long long pmask = __ballot(placed);
  if (lane == 0) a.ntpp[0] = __popcll(pmask);
  if (a.stats) {
    unsigned long long t_act = 0, t_miss = 0, t_missed = 0;
    if (a.slot_for_id) {
      const uint32_t k2 = wave_sort64((static_cast<uint32_t>(idv ? id : 0xFFFFF) << 7) |
                                      (static_cast<uint32_t>(miss) << 6) | static_cast<uint32_t>(lane));
      const int sid = static_cast<int>(k2 >> 7);
      const int prev2 = __shfl(sid, lane == 0 ? 0 : lane - 1, kWave);
      const bool first = sid != 0xFFFFF && (lane == 0 || prev2 != sid);
      t_act = __popcll(__ballot(first));
      t_miss = __popcll(__ballot(first && ((k2 >> 6) & 1u)));
      t_missed = __popcll(__ballot(miss));
    }
    auto* st = reinterpret_cast<unsigned long long*>(a.stats);
    if (lane == 0) {
      if (t_act) atomicAdd(st + 0, t_act);
      if (t_miss) atomicAdd(st + 1, t_miss);
      if (t_missed) atomicAdd(st + 3, t_missed);
      atomicAdd(st + 2, 1ull);
    }
  }
}


// ----------------------------------------------------------------------------
// One-wave align by counting (the outputs of align_wave, at most 64 routes):
// lane i takes route i; one pass over the call's routes (their keys read
// with readlane, uniform j) counts, for every route, the valid routes whose
// (expert, route) key sorts before its own (its position), those of smaller
// experts (the start of its expert's run) and those of its own expert (the
// run's length); a second pass numbers the segment heads by position.  The
// counters' distinct experts come from the same first pass (first occurrence
// of an id).  No cross-lane sort: the dependent chain is two loops of
// independent compares, numel iterations each.  pre_slot (nullable, LDS): the
// slot of each route's id when the caller already looked it up.
// ----------------------------------------------------------------------------
__device__ __forceinline__ void align_rank_wave(const AlignArgs& a, const int32_t* ids,
                                                const int32_t* pre_slot = nullptr) {
  const int lane = lane_id();
  const int n = a.numel;
  const int eff = a.num_experts + 1;
  int e = -1, id = -1;
  bool idv = false, miss = false;
  if (lane < n) {
    e = ids[lane];
    if (a.slot_for_id) {
      id = e;
      idv = e >= 0 && e < a.table_size;
      const int s = idv ? (pre_slot ? pre_slot[lane] : a.slot_for_id[e]) : -1;
      if (a.slot_ids) a.slot_ids[lane] = s;
      if (a.miss_mask) a.miss_mask[lane] = (idv && s < 0) ? 1 : 0;
      miss = idv && s < 0;
      e = s;
    }
  }
  const bool valid = lane < n && e >= 0 && e < eff;
  // (expert << 6 | route): unique per valid route; invalid routes sort last
  const uint32_t key = valid ? (static_cast<uint32_t>(e) << 6) | static_cast<uint32_t>(lane) : 0xFFFFFFFFu;
  const uint32_t ex = key >> 6;
  const uint32_t idk = idv ? static_cast<uint32_t>(id) : 0xFFFFFFFFu;
  int pos = 0, before = 0, same = 0, dup = 0;
  for (int j = 0; j < n; ++j) {
    const uint32_t kj = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key), j));
    const uint32_t xj = kj >> 6;
    pos += kj < key;
    before += xj < ex;
    same += xj == ex;
    if (a.stats) {
      const uint32_t ij = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(idk), j));
      dup += (j < lane) && ij == idk;
    }
  }
  if (valid) a.sorted_ids[pos] = lane;
  const unsigned long long pmask = __ballot(valid);
  if (lane == 0) a.ntpp[0] = __popcll(pmask);
  if (a.seg_expert) {
    const bool head = valid && e < a.num_experts && (pos - before) % a.seg_cap == 0;
    const unsigned long long hmask = __ballot(head);
    int si = 0;
    for (unsigned long long m = hmask; m; m &= m - 1) {
      const int j = __ffsll(static_cast<long long>(m)) - 1;
      si += __builtin_amdgcn_readlane(pos, j) < pos;
    }
    if (head) {
      a.seg_expert[si] = e;
      a.seg_start[si] = pos;
      a.seg_count[si] = min(a.seg_cap, same - (pos - before));
    }
    if (lane == 0) a.n_seg[0] = __popcll(hmask);
  }
  if (a.stats) {
    unsigned long long t_act = 0, t_miss = 0, t_missed = 0;
    if (a.slot_for_id) {
      const bool first = idv && dup == 0;
      t_act = __popcll(__ballot(first));
      t_miss = __popcll(__ballot(first && miss));
      t_missed = __popcll(__ballot(miss));
    }
    auto* st = reinterpret_cast<unsigned long long*>(a.stats);
    if (lane == 0) {
      if (t_act) atomicAdd(st + 0, t_act);
      if (t_miss) atomicAdd(st + 1, t_miss);
      if (t_missed) atomicAdd(st + 3, t_missed);
      atomicAdd(st + 2, 1ull);
    }
  }
}

// The one-wave align of a decode-sized call: by counting up to
// kAlignCountRoutes routes (its loops are numel iterations long), by the
// sorts above that (their length is fixed).  Measured at C2 b = 1 (8 routes)
// 29.6 -> 27.8 us per layer with counting; at 64 routes counting was slower
// (C2 b = 8 62.0 -> 68.2 us).
constexpr int kAlignCountRoutes = 16;
__device__ __forceinline__ void align_small(const AlignArgs& a, const int32_t* ids) {
  if (a.numel <= kAlignCountRoutes) align_rank_wave(a, ids);
  else align_wave(a, ids);
}

// Whether a call qualifies for the one-wave align.
inline bool align_fits_wave(const AlignArgs& a) {
  return a.numel <= kWave && a.block_size == 1 && a.max_padded == 0 && !a.expert_ids && !a.cum_out &&
         a.num_experts < 0xFFFFF && a.table_size < 0xFFFFF;
}

}  // namespace ftmoe
