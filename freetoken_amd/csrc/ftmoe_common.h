// Shared device helpers for the gfx950 MoE-layer kernels.
//
// Conventions used by every kernel in this directory:
//   * wave64: a "wave" is 64 lanes; workgroups are multiples of 64 threads.
//   * bf16 values travel as uint16_t bit patterns; conversions are explicit.
//   * fp8 is OCP e4m3fn and fp4 is OCP e2m1, the native gfx950 formats.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ftmoe {

constexpr int kWave = 64;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float32 -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Monotone map float32 -> uint32 (IEEE order on non-NaN values); -0.0 is
// folded onto +0.0 first so equal values get equal keys.
__device__ __forceinline__ uint32_t order_key(float v) {
  uint32_t u = __float_as_uint(v);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Deterministic float32 exp/sigmoid.  Bit-identical to oracle/numerics.py
// (exp_det / sigmoid_det): Cody-Waite reduction with ln2 split into a 16-bit
// head (exact products) and a tail, degree-6 Taylor polynomial in Horner form,
// exact ldexp.  Contraction is disabled so every step is one IEEE operation.
__device__ __forceinline__ float det_exp(float y) {
#pragma clang fp contract(off)
  y = fminf(fmaxf(y, -87.0f), 87.0f);
  const float n = rintf(y * 0x1.715476p+0f);
  float r = y - n * 0x1.62e4p-1f;
  r = r - n * 0x1.7f7d1cp-20f;
  float p = 0x1.6c16c2p-10f;
  p = p * r + 0x1.111112p-7f;
  p = p * r + 0x1.555556p-5f;
  p = p * r + 0x1.555556p-3f;
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  return ldexpf(p, static_cast<int>(n));
}

__device__ __forceinline__ float det_sigmoid(float x) {
#pragma clang fp contract(off)
  const float e = det_exp(-x);
  return __fdiv_rn(1.0f, 1.0f + e);
}

// Activations of the *_and_mul epilogue (reference kernel/triton/activation.py).
enum Act : int { ACT_SILU = 0, ACT_GELU = 1, ACT_GELU_TANH = 2 };

__device__ __forceinline__ float act_apply(int act, float g) {
  if (act == ACT_SILU) return g / (1.0f + __expf(-g));
  if (act == ACT_GELU) return 0.5f * g * (1.0f + erff(g * 0.7071067811865476f));
  const float inner = 0.7978845608028654f * (g + 0.044715f * g * g * g);
  return 0.5f * g * (1.0f + tanhf(inner));
}

// 64-bit wave max via xor shuffles (all lanes end with the maximum).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), off, kWave);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), off, kWave);
    const uint64_t o = (static_cast<uint64_t>(hi) << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

}  // namespace ftmoe
