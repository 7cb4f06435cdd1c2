// Test helper (not part of libftmoe.so): the library's activation
// quantisation of a float32-scaled group (group_scale<0> / quant_value<0> of
// quant.h, a division by the scale done as a multiplication with an FMA
// correction) against the IEEE division __fdiv_rn(x, s), for every pair of
// bf16 values with 0 <= amax finite and |x| <= amax, the whole domain on which
// the kernels call it (amax is the group's absolute maximum, x one of its
// values, both bf16).  Counted per pair: e4m3 codes that differ (through the
// conversion instruction the kernels use), float32 results that differ where
// the IEEE quotient is at least 2^-64, and float32 results that differ at all.
#include <cstdint>

#include "quant.h"

namespace {

__global__ void quant_division_kernel(uint32_t a_base, unsigned long long* counts) {
  const uint32_t ab = a_base + blockIdx.y;  // amax bit pattern (upper half of a float)
  const uint32_t xb = blockIdx.x * blockDim.x + threadIdx.x;
  if (ab >= 0x7f80u || xb > 0xffffu) return;
  const float amax = __uint_as_float(ab << 16);
  const float x = __uint_as_float(xb << 16);
  if (!(fabsf(x) <= amax)) return;
  float r;
  const float s = ftmoe::group_scale<0>(amax, r);
  const float y = ftmoe::quant_value<0>(x, s, r);
  const float ref = fminf(fmaxf(__fdiv_rn(x, s), -448.0f), 448.0f);
  const int cy = __builtin_amdgcn_cvt_pk_fp8_f32(y, y, 0, false) & 0xff;
  const int cr = __builtin_amdgcn_cvt_pk_fp8_f32(ref, ref, 0, false) & 0xff;
  const bool diff = __float_as_uint(y) != __float_as_uint(ref);
  if (cy != cr) atomicAdd(counts + 0, 1ull);
  if (diff && fabsf(ref) >= 0x1p-64f) atomicAdd(counts + 1, 1ull);
  if (diff) atomicAdd(counts + 2, 1ull);
}

}  // namespace

// counts[0]: e4m3 code mismatches, counts[1]: float32 mismatches with
// |x / s| >= 2^-64, counts[2]: float32 mismatches.  Returns 0, or a HIP error.
extern "C" int ftmoe_test_quant_division(unsigned long long* counts) {
  unsigned long long* d = nullptr;
  hipError_t e = hipMalloc(&d, 3 * sizeof(unsigned long long));
  if (e != hipSuccess) return static_cast<int>(e);
  e = hipMemset(d, 0, 3 * sizeof(unsigned long long));
  const uint32_t per_launch = 0x3fc0;  // amax patterns per launch (grid y)
  for (uint32_t a = 0; e == hipSuccess && a < 0x7f80u; a += per_launch) {
    hipLaunchKernelGGL(quant_division_kernel, dim3(0x10000 / 256, per_launch), dim3(256), 0, 0, a, d);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipDeviceSynchronize();
  }
  unsigned long long h[3] = {0, 0, 0};
  if (e == hipSuccess) e = hipMemcpy(h, d, sizeof(h), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  for (int i = 0; i < 3; ++i) counts[i] = h[i];
  return static_cast<int>(e);
}
