// Router top-k kernels: softmax top-k and DeepSeek-V3 grouped sigmoid top-k.
//
// One wave per token.  Expert e lives in lane (e % 64), register slot e / 64,
// so E <= 64 * kMaxPerLane.  Selection is k rounds of a wave-wide maximum over
// 64-bit keys (order_key(value) << 32 | ~index): the larger value wins and on
// equal values the lower expert index wins -- the lowest-index tie rule of the
// reference's gpt-oss router (kernel/triton/mxfp4_moe.py:288-331).
#include "kernels.h"

namespace ftmoe {

constexpr int kMaxPerLane = 16;  // E <= 1024

__device__ __forceinline__ uint64_t pack_key(float v, int e) {
  return (static_cast<uint64_t>(order_key(v)) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(e));
}

template <typename T>
__device__ __forceinline__ float load_logit(const T* p);
template <>
__device__ __forceinline__ float load_logit<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_logit<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

// fused_topk (reference moe/fused.py:38-85): selection on fp32 logits; with
// renormalize the weights are the softmax over the k selected logits, else the
// softmax over all experts evaluated at the selected ones.
template <typename T>
__global__ void __launch_bounds__(256) softmax_topk_kernel(const T* __restrict__ logits, int M, int E,
                                                           int k, int renorm, float* __restrict__ out_w,
                                                           int32_t* __restrict__ out_ids) {
  const int lane = lane_id();
  const int tok = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (tok >= M) return;
  const T* row = logits + static_cast<size_t>(tok) * E;
  float v[kMaxPerLane];
  uint32_t taken = 0;
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    const int e = lane + j * kWave;
    v[j] = (e < E) ? load_logit<T>(row + e) : -INFINITY;
  }
  float my_val = 0.0f;
  int my_idx = -1;
  for (int r = 0; r < k; ++r) {
    uint64_t best = 0;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      const int e = lane + j * kWave;
      if (e < E && !((taken >> j) & 1u)) {
        const uint64_t key = pack_key(v[j], e);
        best = key > best ? key : best;
      }
    }
    best = wave_max_u64(best);
    const int win = static_cast<int>(~static_cast<uint32_t>(best));
    if ((win & (kWave - 1)) == lane) taken |= 1u << (win / kWave);
    // value of the winner, broadcast from its owner lane
    float wv = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j)
      if (j == win / kWave) wv = v[j];
    wv = __shfl(wv, win & (kWave - 1), kWave);
    if (lane == r) {
      my_val = wv;
      my_idx = win;
    }
  }
  const float vmax = __shfl(my_val, 0, kWave);  // rank 0 holds the maximum
  float denom;
  if (renorm) {
    const float ex = (lane < k) ? expf(my_val - vmax) : 0.0f;
    denom = wave_sum_f32(ex);
  } else {
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      const int e = lane + j * kWave;
      if (e < E) s += expf(v[j] - vmax);
    }
    denom = wave_sum_f32(s);
  }
  if (lane < k) {
    out_w[static_cast<size_t>(tok) * k + lane] = expf(my_val - vmax) / denom;
    out_ids[static_cast<size_t>(tok) * k + lane] = my_idx;
  }
}

// Grouped sigmoid router (reference models/glm4_moe/moe.py:53-75):
//   s = sigmoid(l); c = s + bias; group score = top1(c) + top2(c) in the group;
//   keep topk_group groups; top-k of c over kept groups; w = s[id];
//   renorm w / (sum + 1e-20); times scale.  Uses det_sigmoid so the selection
//   is bit-identical to the CPU oracle.
__global__ void __launch_bounds__(256) grouped_sigmoid_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int M, int E, int n_group,
    int topk_group, int k, int renorm, float scale, float* __restrict__ out_w,
    int32_t* __restrict__ out_ids) {
  const int lane = lane_id();
  const int tok = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (tok >= M) return;
  const float* row = logits + static_cast<size_t>(tok) * E;
  const int per = E / n_group;
  float c[kMaxPerLane];
#pragma unroll
  for (int j = 0; j < kMaxPerLane; ++j) {
    const int e = lane + j * kWave;
    if (e < E) {
      const float s = det_sigmoid(row[e]);
      c[j] = bias ? s + bias[e] : s;
    } else {
      c[j] = -INFINITY;
    }
  }
  if (n_group > 1) {
    // group g's score lands in lane g (n_group <= 64)
    float gscore = -INFINITY;
    for (int g = 0; g < n_group; ++g) {
      float a1 = -INFINITY, a2 = -INFINITY;  // local top-2 of c in group g
#pragma unroll
      for (int j = 0; j < kMaxPerLane; ++j) {
        const int e = lane + j * kWave;
        if (e < E && e / per == g) {
          const float x = c[j];
          if (x > a1) {
            a2 = a1;
            a1 = x;
          } else if (x > a2) {
            a2 = x;
          }
        }
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        const float b1 = __shfl_xor(a1, off, kWave);
        const float b2 = __shfl_xor(a2, off, kWave);
        const float n1 = fmaxf(a1, b1);
        const float n2 = fmaxf(fminf(a1, b1), fmaxf(a2, b2));
        a1 = n1;
        a2 = n2;
      }
      if (lane == g) gscore = a1 + a2;
    }
    uint64_t gmask = 0;
    bool kept = false;
    for (int r = 0; r < topk_group; ++r) {
      const uint64_t key = (lane < n_group && !kept) ? pack_key(gscore, lane) : 0;
      const uint64_t best = wave_max_u64(key);
      const int win = static_cast<int>(~static_cast<uint32_t>(best));
      if (lane == win) kept = true;
      gmask |= 1ull << win;
    }
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      const int e = lane + j * kWave;
      if (e < E && !((gmask >> (e / per)) & 1ull)) c[j] = -INFINITY;
    }
  }
  uint32_t taken = 0;
  int my_idx = -1;
  for (int r = 0; r < k; ++r) {
    uint64_t best = 0;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
      const int e = lane + j * kWave;
      if (e < E && !((taken >> j) & 1u)) {
        const uint64_t key = pack_key(c[j], e);
        best = key > best ? key : best;
      }
    }
    best = wave_max_u64(best);
    const int win = static_cast<int>(~static_cast<uint32_t>(best));
    if ((win & (kWave - 1)) == lane) taken |= 1u << (win / kWave);
    if (lane == r) my_idx = win;
  }
  float w = (lane < k) ? det_sigmoid(row[my_idx]) : 0.0f;
  if (renorm) {
    float tot = 0.0f;  // sequential sum in rank order, as the oracle does
    for (int r = 0; r < k; ++r) tot += __shfl(w, r, kWave);
    w = w / (tot + 1e-20f);
  }
  w = w * scale;
  if (lane < k) {
    out_w[static_cast<size_t>(tok) * k + lane] = w;
    out_ids[static_cast<size_t>(tok) * k + lane] = my_idx;
  }
}

hipError_t launch_softmax_topk(const void* logits, int logits_bf16, int M, int E, int k, int renorm,
                               float* w, int32_t* ids, hipStream_t stream) {
  const int waves = 4;
  dim3 grid((M + waves - 1) / waves), block(waves * kWave);
  if (logits_bf16)
    hipLaunchKernelGGL(softmax_topk_kernel<uint16_t>, grid, block, 0, stream,
                       static_cast<const uint16_t*>(logits), M, E, k, renorm, w, ids);
  else
    hipLaunchKernelGGL(softmax_topk_kernel<float>, grid, block, 0, stream,
                       static_cast<const float*>(logits), M, E, k, renorm, w, ids);
  return hipGetLastError();
}

hipError_t launch_grouped_sigmoid(const float* logits, const float* bias, int M, int E, int n_group,
                                  int topk_group, int k, int renorm, float scale, float* w, int32_t* ids,
                                  hipStream_t stream) {
  const int waves = 4;
  dim3 grid((M + waves - 1) / waves), block(waves * kWave);
  hipLaunchKernelGGL(grouped_sigmoid_kernel, grid, block, 0, stream, logits, bias, M, E, n_group,
                     topk_group, k, renorm, scale, w, ids);
  return hipGetLastError();
}

}  // namespace ftmoe
