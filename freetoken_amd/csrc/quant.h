// Activation quantisation of one 128-value group and the activations of the
// fused *_and_mul epilogues, shared by the quantisation kernel, the gate/up
// GEMM epilogue (both must give identical bytes) and the test helper that
// checks the division below exhaustively.
//
//   MODE 0: float scale s = max(amax, 1e-10) / 448, q = e4m3(clamp(x / s))
//           (reference per_token_group_quant_fp8, kernel/triton/fp8_block_linear.py:53-59)
//   MODE 1: e8m0 scale 2^ceil(log2(max(amax, 1e-4) * (1/448))), q = e4m3(x / 2^e),
//           codes stored as uint8; MODE 2: the same with codes stored as uint32
//           (the grouped GEMM copies them to LDS in 4-byte units)
#pragma once

#include "ftmoe_common.h"

namespace ftmoe {

// Scale of one group with absolute maximum amax.
// MODE 0: returns s and sets mul = RN(1/s), the rounded reciprocal that
// quant_value's division uses;
// MODE 1/2: returns the e8m0 code e+127 as a float and sets mul = 2^-e.
template <int MODE>
__device__ __forceinline__ float group_scale(float amax, float& mul) {
  if (MODE == 0) {
    const float s = fmaxf(amax, 1e-10f) / 448.0f;
    mul = __fdiv_rn(1.0f, s);
    return s;
  }
  const float t = fmaxf(amax, 1e-4f) * 0x1.24924ap-9f;  // * (1/448) rounded to float
  const uint32_t bits = __float_as_uint(t);
  const int e = static_cast<int>((bits >> 23) & 0xff) - 127 + ((bits & 0x7fffff) ? 1 : 0);
  mul = ldexpf(1.0f, -e);
  return static_cast<float>(e + 127);
}

// The value to convert to e4m3, clamped to +-448.
// MODE 0: x / s without a division instruction (Markstein's correction): with
// r = RN(1/s), q = RN(x r) and the residual e = x - q s (exact through the
// FMA), RN(q + e r) is the correctly rounded quotient unless the residual
// underflows; the sign is copied from x so that -0 stays -0.  Over the whole
// domain of the callers (x and amax bf16 values, |x| <= amax, s as above) it
// equals the IEEE quotient x / s except where x is so small that the residual
// underflows; all those quotients are below 2^-71 (e4m3's smallest subnormal
// is 2^-9) and convert to the zero code of x's sign either way: checked
// exhaustively against __fdiv_rn on the GPU and against C's division on the
// CPU.  Three VALU operations instead of the ten of the IEEE division sequence
// with its reciprocal.
template <int MODE>
__device__ __forceinline__ float quant_value(float x, float s, float mul) {
  float y;
  if (MODE == 0) {
    const float q = x * mul;
    const float e = __builtin_fmaf(-q, s, x);
    y = __builtin_fmaf(e, mul, q);
    y = __uint_as_float((__float_as_uint(y) & 0x7fffffffu) | (__float_as_uint(x) & 0x80000000u));
  } else {
    y = x * mul;
  }
  return fminf(fmaxf(y, -448.0f), 448.0f);
}

// Activation with its kind fixed at compile time, for epilogues that hoist
// the runtime choice out of their per-value loops.  SiLU multiplies by the
// hardware reciprocal (within 1 ulp) instead of dividing: its result is
// rounded to bf16 next, and the exponential is the hardware one either way,
// so the IEEE division bought no exactness (the other kinds are act_apply).
template <int ACT>
__device__ __forceinline__ float act_fixed(float g) {
  if constexpr (ACT == ACT_SILU) return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
  else return act_apply(ACT, g);
}

}  // namespace ftmoe
