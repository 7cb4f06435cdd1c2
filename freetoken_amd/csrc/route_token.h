// Per-token router pieces shared by route.hip (router kernels, router +
// permutation) and decode.hip (router + permutation beside the shared expert's
// gate_up): softmax top-k and DeepSeek-V3 grouped sigmoid top-k for one token
// per wave.
//
// Expert e lives in lane (e % 64), register slot e / 64; PER = ceil(E / 64)
// slots per lane is a template parameter.  Selection is k rounds of: a
// wave-wide float maximum over the entries still available, then one ballot
// per slot for the entries holding it; the lowest expert index among them wins
// (the lowest-index tie rule of the reference's gpt-oss router,
// kernel/triton/mxfp4_moe.py:288-331; -0.0 equals +0.0).  The ballots and the
// winner are wave-uniform, so a round is one reduction plus scalar work.
#pragma once

#include "kernels.h"

namespace ftmoe {

constexpr int kRouteWaves = 4;

template <typename T>
__device__ __forceinline__ float load_logit(const T* p);
template <>
__device__ __forceinline__ float load_logit<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_logit<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

// Largest available value of v[PER] in the wave, the lowest index holding it
// (slot-major: index = 64 * slot + lane); -1 when nothing is available.
template <int PER>
__device__ __forceinline__ int wave_argmax(const float (&v)[PER], const bool (&live)[PER]) {
  float best = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (live[j]) best = fmaxf(best, v[j]);
  best = wave_max_f32(best);
  int win = -1;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const uint64_t b = __ballot(live[j] && v[j] == best);
    if (win < 0 && b != 0) win = j * kWave + __ffsll(static_cast<long long>(b)) - 1;
  }
  return win;
}

// k rounds of selection; returns the winner index of round r in lane r (lanes
// >= k, and rounds with nothing available: -1).
template <int PER>
__device__ __forceinline__ int select_topk(const float (&v)[PER], bool (&live)[PER], int k) {
  const int lane = lane_id();
  int mine = -1;
  for (int r = 0; r < k; ++r) {
    const int win = wave_argmax<PER>(v, live);
    if (win >= 0 && (win & (kWave - 1)) == lane) {
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (j == win / kWave) live[j] = false;
    }
    if (lane == r) mine = win;
  }
  return mine;
}

// fused_topk (reference moe/fused.py:38-85): selection on fp32 logits; with
// renormalize the weights are the softmax over the k selected logits, else the
// softmax over all experts evaluated at the selected ones.
template <typename T, int PER>
__device__ __forceinline__ int softmax_token(const T* __restrict__ row, int E, int k, int renorm,
                                             float* __restrict__ w_out, int32_t* __restrict__ ids_out) {
  const int lane = lane_id();
  float v[PER];
  bool live[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + j * kWave;
    v[j] = (e < E) ? load_logit<T>(row + e) : -INFINITY;
    live[j] = e < E;
  }
  const int my_idx = select_topk<PER>(v, live, k);
  const float my_val = (lane < k) ? load_logit<T>(row + my_idx) : -INFINITY;
  const float vmax = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(my_val), 0));  // rank 0
  float denom;
  if (renorm) {
    denom = wave_sum_f32((lane < k) ? expf(my_val - vmax) : 0.0f);
  } else {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (lane + j * kWave < E) s += expf(v[j] - vmax);
    denom = wave_sum_f32(s);
  }
  if (lane < k) {
    w_out[lane] = expf(my_val - vmax) / denom;
    ids_out[lane] = my_idx;
  }
  return my_idx;
}

// Multiset top-2 of two disjoint sets given as (largest, second largest).
__device__ __forceinline__ void top2_merge(float& a1, float& a2, float b1, float b2) {
  const float lo = fminf(a1, b1);
  a1 = fmaxf(a1, b1);
  a2 = fmaxf(lo, fmaxf(a2, b2));
}

template <int CTRL>
__device__ __forceinline__ void top2_dpp(float& a1, float& a2) {
  top2_merge(a1, a2, dpp_f32<CTRL>(a1), dpp_f32<CTRL>(a2));
}

// Top-2 of every aligned block of `per` lanes (per a power of two <= 64), left
// in all lanes of the block: butterflies over disjoint halves (DPP inside a
// 16-lane row, lane shuffles across rows).
__device__ __forceinline__ void block_top2(float& a1, float& a2, int per) {
  if (per >= 2) top2_dpp<0xB1>(a1, a2);   // quad_perm [1,0,3,2]
  if (per >= 4) top2_dpp<0x4E>(a1, a2);   // quad_perm [2,3,0,1]
  if (per >= 8) top2_dpp<0x141>(a1, a2);  // row_half_mirror
  if (per >= 16) top2_dpp<0x140>(a1, a2); // row_mirror
  if (per >= 32) top2_merge(a1, a2, __shfl_xor(a1, 16), __shfl_xor(a2, 16));
  if (per >= 64) top2_merge(a1, a2, __shfl_xor(a1, 32), __shfl_xor(a2, 32));
}

// Grouped sigmoid router (reference models/glm4_moe/moe.py:53-75):
//   s = sigmoid(l); c = s + bias; group score = top1(c) + top2(c) in the group;
//   keep topk_group groups; top-k of c over kept groups; w = s[id];
//   renorm w / (sum + 1e-20); times scale.  Uses det_sigmoid so the selection
//   is bit-identical to the CPU oracle.  Group scores: when the group size is a
//   power of two dividing 64 (DeepSeek-V3: 32) and E is a multiple of 64, a
//   group is an aligned lane block of one register slot and its top-2 is a
//   butterfly (block_top2); otherwise the wave stages c in LDS and lane g scans
//   group g.  The weights s[id] come from the lanes holding them (shuffles),
//   not from a second read of the logits.
template <int PER>
__device__ __forceinline__ int grouped_token(const float* __restrict__ row, const float* __restrict__ bias, int E,
                                             int n_group, int topk_group, int k, int renorm, float scale,
                                             float* s_c, float* __restrict__ w_out, int32_t* __restrict__ ids_out) {
  const int lane = lane_id();
  const int per = E / n_group;
  float sg[PER], c[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + j * kWave;
    if (e < E) {
      sg[j] = det_sigmoid(row[e]);
      c[j] = bias ? sg[j] + bias[e] : sg[j];
    } else {
      sg[j] = 0.0f;
      c[j] = -INFINITY;
    }
  }
  uint64_t gmask = ~0ull;
  const bool lane_groups = (E % kWave) == 0 && per <= kWave && (per & (per - 1)) == 0;
  if (n_group > 1 && lane_groups) {
    // group of (lane, slot j) = j * (64 / per) + lane / per
    // group of (lane, slot j) = j * (64 / per) + lane / per: ascending in
    // (slot, lane), so the lowest (slot, lane) holding the maximum is the
    // lowest group index
    const int gpl = kWave / per;
    float gs[PER];
    bool glive[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      float a1 = c[j], a2 = -INFINITY;
      block_top2(a1, a2, per);
      gs[j] = a1 + a2;
      glive[j] = lane % per == 0 && lane + j * kWave < E;
    }
    gmask = 0;
    for (int r = 0; r < topk_group; ++r) {
      const int win = wave_argmax<PER>(gs, glive);
      if (win < 0) break;
      const int wl = win & (kWave - 1), wj = win / kWave;
      if (wl == lane) {
#pragma unroll
        for (int j = 0; j < PER; ++j)
          if (j == wj) glive[j] = false;
      }
      gmask |= 1ull << (wj * gpl + wl / per);
    }
  } else if (n_group > 1) {
#pragma unroll
    for (int j = 0; j < PER; ++j) s_c[lane + j * kWave] = c[j];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    float gscore = -INFINITY;
    if (lane < n_group) {
      float a1 = -INFINITY, a2 = -INFINITY;  // top-2 with duplicates kept
      for (int i = 0; i < per; ++i) {
        const float x = s_c[lane * per + i];
        if (x > a1) {
          a2 = a1;
          a1 = x;
        } else if (x > a2) {
          a2 = x;
        }
      }
      gscore = a1 + a2;
    }
    float gv[1] = {gscore};
    bool glive[1] = {lane < n_group};
    gmask = 0;
    for (int r = 0; r < topk_group; ++r) {
      const int win = wave_argmax<1>(gv, glive);
      if (win < 0) break;
      if (lane == win) glive[0] = false;
      gmask |= 1ull << win;
    }
  }
  float sel[PER];
  bool live[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = lane + j * kWave;
    const bool kept = (gmask >> ((e < E ? e : 0) / per)) & 1ull;
    sel[j] = kept ? c[j] : -INFINITY;
    live[j] = e < E;
  }
  const int my_idx = select_topk<PER>(sel, live, k);
  float w = 0.0f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const float t = __shfl(sg[j], my_idx & (kWave - 1));
    if (lane < k && (my_idx >> 6) == j) w = t;
  }
  if (renorm) {
    float tot = 0.0f;  // sequential sum in rank order, as the oracle does
    for (int r = 0; r < k; ++r) tot += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(w), r));
    w = w / (tot + 1e-20f);
  }
  w = w * scale;
  if (lane < k) {
    w_out[lane] = w;
    ids_out[lane] = my_idx;
  }
  return my_idx;
}

}  // namespace ftmoe
