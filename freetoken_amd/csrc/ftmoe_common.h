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

// Round-to-nearest-even float32 -> bf16: the __bf16 conversion, one
// v_cvt_pk_bf16_f32 on gfx950.  Checked on MI355X over all 2^32 inputs against
// the integer rounding (u + 0x7fff + ((u >> 16) & 1)) >> 16 that the CPU
// oracle uses: equal for every finite and infinite input, NaN stays NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two values rounded to bf16 and packed (a in the low half): one instruction.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

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

// Clamped SwiGLU inputs (DeepSeek-V4 ds_fp4, kernel/triton/dsv4/fused_moe.py:121-141):
// the gate capped at lim and the up value clamped to [-lim, lim]; lim = 0
// leaves both as they are.
__device__ __forceinline__ void swiglu_clamp(float lim, float& g, float& u) {
  if (lim > 0.f) {
    g = fminf(g, lim);
    u = fminf(fmaxf(u, -lim), lim);
  }
}

// Cross-lane reductions: DPP butterflies inside each 16-lane row (quad_perm
// xor1 / xor2, row_half_mirror, row_mirror leave every lane of a row with the
// row's result), then the four row results are combined from readlanes.  This
// keeps the dependent chain at a few VALU latencies instead of the LDS-latency
// permutes of generic shuffles.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), CTRL, 0xF, 0xF,
                                                           false));
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = dpp_u32<CTRL>(static_cast<uint32_t>(v));
  const uint32_t hi = dpp_u32<CTRL>(static_cast<uint32_t>(v >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(v), lane);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(v >> 32), lane);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Wave-wide maximum of a 64-bit key; the result is uniform across the wave.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  v = max_u64(v, dpp_u64<0xB1>(v));   // quad_perm [1,0,3,2]
  v = max_u64(v, dpp_u64<0x4E>(v));   // quad_perm [2,3,0,1]
  v = max_u64(v, dpp_u64<0x141>(v));  // row_half_mirror
  v = max_u64(v, dpp_u64<0x140>(v));  // row_mirror
  return max_u64(max_u64(readlane_u64(v, 0), readlane_u64(v, 16)),
                 max_u64(readlane_u64(v, 32), readlane_u64(v, 48)));
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v)));
}

__device__ __forceinline__ float wave_sum_f32(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x141>(v);
  v += dpp_f32<0x140>(v);
  const float a = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
  const float b = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16));
  const float c = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 32));
  const float d = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 48));
  return (a + b) + (c + d);
}

// Wave-wide sum of small non-negative counts (the result is uniform).
__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) {
  uint32_t x = static_cast<uint32_t>(v);
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) x += static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), off, kWave));
  return x;
}

__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  const float a = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0));
  const float b = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16));
  const float c = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 32));
  const float d = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// ---- raw buffer loads ---------------------------------------------------------
// A descriptor covers [base, base + bytes); a lane offset at or beyond `bytes`
// reads zeros without touching memory (kOutOfRange is beyond every range the
// library builds: callers keep ranges below 2 GiB).
constexpr uint32_t kOutOfRange = 0x80000000u;
constexpr int kBufDword3 = 0x00020000;  // gfx9 raw-buffer descriptor word 3

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufDword3);
}

__device__ __forceinline__ u32x4 buf_x4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

__device__ __forceinline__ float buf_f32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}

__device__ __forceinline__ uint2 buf_x2(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
  return uint2{static_cast<uint32_t>(v[0]), static_cast<uint32_t>(v[1])};
}

__device__ __forceinline__ uint32_t buf_u8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b8(r, voff, soff, 0));
}

}  // namespace ftmoe
