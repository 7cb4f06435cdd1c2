// Router top-k kernels: softmax top-k and DeepSeek-V3 grouped sigmoid top-k,
// one wave per token (the per-token routines are in route_token.h), and the
// router + permutation launch of decode-sized calls.
#include "align_wave.h"
#include "kernels.h"
#include "route_token.h"

namespace ftmoe {

template <typename T, int PER>
__global__ void __launch_bounds__(kRouteWaves * kWave) softmax_topk_kernel(const T* __restrict__ logits, int M,
                                                                            int E, int k, int renorm,
                                                                            float* __restrict__ out_w,
                                                                            int32_t* __restrict__ out_ids) {
  const int tok = blockIdx.x * kRouteWaves + threadIdx.x / kWave;
  if (tok >= M) return;
  softmax_token<T, PER>(logits + static_cast<size_t>(tok) * E, E, k, renorm, out_w + static_cast<size_t>(tok) * k,
                        out_ids + static_cast<size_t>(tok) * k);
}

template <int PER>
__global__ void __launch_bounds__(kRouteWaves * kWave) grouped_sigmoid_kernel(
    const float* __restrict__ logits, const float* __restrict__ bias, int M, int E, int n_group, int topk_group,
    int k, int renorm, float scale, float* __restrict__ out_w, int32_t* __restrict__ out_ids) {
  __shared__ float s_c[kRouteWaves][PER * kWave];
  const int wave = threadIdx.x / kWave;
  const int tok = blockIdx.x * kRouteWaves + wave;
  if (tok >= M) return;
  grouped_token<PER>(logits + static_cast<size_t>(tok) * E, bias, E, n_group, topk_group, k, renorm, scale, s_c[wave],
                     out_w + static_cast<size_t>(tok) * k, out_ids + static_cast<size_t>(tok) * k);
}

template <int PER>
static void launch_softmax_per(const void* logits, int bf16, int M, int E, int k, int renorm, float* w, int32_t* ids,
                               hipStream_t stream) {
  dim3 grid((M + kRouteWaves - 1) / kRouteWaves), block(kRouteWaves * kWave);
  if (bf16)
    hipLaunchKernelGGL((softmax_topk_kernel<uint16_t, PER>), grid, block, 0, stream,
                       static_cast<const uint16_t*>(logits), M, E, k, renorm, w, ids);
  else
    hipLaunchKernelGGL((softmax_topk_kernel<float, PER>), grid, block, 0, stream, static_cast<const float*>(logits),
                       M, E, k, renorm, w, ids);
}

hipError_t launch_softmax_topk(const void* logits, int logits_bf16, int M, int E, int k, int renorm, float* w,
                               int32_t* ids, hipStream_t stream) {
  const int per = (E + kWave - 1) / kWave;
  if (per <= 1) launch_softmax_per<1>(logits, logits_bf16, M, E, k, renorm, w, ids, stream);
  else if (per <= 2) launch_softmax_per<2>(logits, logits_bf16, M, E, k, renorm, w, ids, stream);
  else if (per <= 4) launch_softmax_per<4>(logits, logits_bf16, M, E, k, renorm, w, ids, stream);
  else if (per <= 8) launch_softmax_per<8>(logits, logits_bf16, M, E, k, renorm, w, ids, stream);
  else launch_softmax_per<16>(logits, logits_bf16, M, E, k, renorm, w, ids, stream);
  return hipGetLastError();
}

template <int PER>
static void launch_grouped_per(const float* logits, const float* bias, int M, int E, int n_group, int topk_group,
                               int k, int renorm, float scale, float* w, int32_t* ids, hipStream_t stream) {
  dim3 grid((M + kRouteWaves - 1) / kRouteWaves), block(kRouteWaves * kWave);
  hipLaunchKernelGGL((grouped_sigmoid_kernel<PER>), grid, block, 0, stream, logits, bias, M, E, n_group, topk_group,
                     k, renorm, scale, w, ids);
}

hipError_t launch_grouped_sigmoid(const float* logits, const float* bias, int M, int E, int n_group, int topk_group,
                                  int k, int renorm, float scale, float* w, int32_t* ids, hipStream_t stream) {
  const int per = (E + kWave - 1) / kWave;
  if (per <= 1) launch_grouped_per<1>(logits, bias, M, E, n_group, topk_group, k, renorm, scale, w, ids, stream);
  else if (per <= 2) launch_grouped_per<2>(logits, bias, M, E, n_group, topk_group, k, renorm, scale, w, ids, stream);
  else if (per <= 4) launch_grouped_per<4>(logits, bias, M, E, n_group, topk_group, k, renorm, scale, w, ids, stream);
  else if (per <= 8) launch_grouped_per<8>(logits, bias, M, E, n_group, topk_group, k, renorm, scale, w, ids, stream);
  else launch_grouped_per<16>(logits, bias, M, E, n_group, topk_group, k, renorm, scale, w, ids, stream);
  return hipGetLastError();
}


// ----------------------------------------------------------------------------
// Router + permutation in one launch for decode-sized calls (at most 16 tokens,
// at most 64 routes): wave t routes token t, writing the router outputs and
// the ids into LDS; after one barrier wave 0 runs the one-wave align on them.
// Saves the permutation's launch and the ids' round trip through memory.
// ----------------------------------------------------------------------------
constexpr int kFrontWaves = 16;

template <int GROUPED, typename T, int PER>
__global__ void __launch_bounds__(kFrontWaves * kWave) route_align_kernel(RouteArgs r, AlignArgs a) {
  __shared__ int s_ids[kWave];
  __shared__ float s_c[GROUPED ? kFrontWaves * PER * kWave : 1];
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int tok = wave;
  if (tok < r.M) {
    int id;
    if constexpr (GROUPED) {
      id = grouped_token<PER>(static_cast<const float*>(r.logits) + static_cast<size_t>(tok) * r.E, r.bias, r.E,
                              r.n_group, r.topk_group, r.k, r.renorm, r.scale, s_c + wave * PER * kWave,
                              r.out_w + static_cast<size_t>(tok) * r.k, r.out_ids + static_cast<size_t>(tok) * r.k);
    } else {
      id = softmax_token<T, PER>(static_cast<const T*>(r.logits) + static_cast<size_t>(tok) * r.E, r.E, r.k, r.renorm,
                                 r.out_w + static_cast<size_t>(tok) * r.k, r.out_ids + static_cast<size_t>(tok) * r.k);
    }
    if (lane < r.k) s_ids[tok * r.k + lane] = id;
  }
  __syncthreads();
  if (wave == 0) align_small(a, s_ids);
}

template <int GROUPED, typename T, int PER>
static void launch_front(const RouteArgs& r, const AlignArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((route_align_kernel<GROUPED, T, PER>), dim3(1), dim3(kFrontWaves * kWave), 0, stream, r, a);
}

hipError_t launch_route_align(const RouteArgs& r, const AlignArgs& a, hipStream_t stream) {
  const int per = (r.E + kWave - 1) / kWave;
  const bool fused = align_fits_wave(a) && r.M <= kFrontWaves && r.M * r.k <= kWave && (r.grouped ? per <= 4 : true);
  if (!fused) {
    const hipError_t err =
        r.grouped ? launch_grouped_sigmoid(static_cast<const float*>(r.logits), r.bias, r.M, r.E, r.n_group,
                                           r.topk_group, r.k, r.renorm, r.scale, r.out_w, r.out_ids, stream)
                  : launch_softmax_topk(r.logits, r.logits_bf16, r.M, r.E, r.k, r.renorm, r.out_w, r.out_ids, stream);
    if (err != hipSuccess) return err;
    return launch_align(a, stream);
  }
  if (r.grouped) {
    if (per <= 1) launch_front<1, float, 1>(r, a, stream);
    else if (per <= 2) launch_front<1, float, 2>(r, a, stream);
    else launch_front<1, float, 4>(r, a, stream);
  } else if (r.logits_bf16) {
    if (per <= 1) launch_front<0, uint16_t, 1>(r, a, stream);
    else if (per <= 2) launch_front<0, uint16_t, 2>(r, a, stream);
    else if (per <= 4) launch_front<0, uint16_t, 4>(r, a, stream);
    else if (per <= 8) launch_front<0, uint16_t, 8>(r, a, stream);
    else launch_front<0, uint16_t, 16>(r, a, stream);
  } else {
    if (per <= 1) launch_front<0, float, 1>(r, a, stream);
    else if (per <= 2) launch_front<0, float, 2>(r, a, stream);
    else if (per <= 4) launch_front<0, float, 4>(r, a, stream);
    else if (per <= 8) launch_front<0, float, 8>(r, a, stream);
    else launch_front<0, float, 16>(r, a, stream);
  }
  return hipGetLastError();
}

}  // namespace ftmoe
