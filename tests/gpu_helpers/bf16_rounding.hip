// Test helper (not part of libftmoe.so): the library's device float32 -> bf16
// rounding, f32_to_bf16 and pack_bf16x2 of ftmoe_common.h, against the integer
// round-to-nearest-even formula the CPU oracle uses (oracle/numerics.py
// bf16_round), over every float32 bit pattern.  Mismatches among finite and
// infinite inputs, and NaN inputs whose result is not a NaN, are counted.
#include <cstdint>

#include "ftmoe_common.h"

namespace {

__device__ __forceinline__ uint16_t rne_formula(uint32_t u) {
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__global__ void bf16_check_kernel(uint32_t base, unsigned long long* counts) {
  const uint32_t u = base + blockIdx.x * blockDim.x + threadIdx.x;
  const float f = __uint_as_float(u);
  const uint16_t h = ftmoe::f32_to_bf16(f);
  // the packed form, with the neighbouring pattern in the other half
  const uint32_t p = ftmoe::pack_bf16x2(f, __uint_as_float(u ^ 1u));
  const bool nan = (u & 0x7fffffffu) > 0x7f800000u;
  unsigned long long m = 0;
  if (!nan) {
    if (h != rne_formula(u) || static_cast<uint16_t>(p & 0xffffu) != rne_formula(u) ||
        static_cast<uint16_t>(p >> 16) != rne_formula(u ^ 1u))
      m = 1;
  } else if ((h & 0x7fffu) <= 0x7f80u) {
    m = 1ull << 32;
  }
  if (m) atomicAdd(counts, m);
}

}  // namespace

// counts[0]: finite / infinite mismatches, counts[1]: NaNs not kept NaN.
// Returns 0, or a HIP error code.
extern "C" int ftmoe_test_bf16_rounding(unsigned long long* counts) {
  unsigned long long* d = nullptr;
  hipError_t e = hipMalloc(&d, sizeof(unsigned long long));
  if (e != hipSuccess) return static_cast<int>(e);
  e = hipMemset(d, 0, sizeof(unsigned long long));
  const uint32_t chunk = 1u << 28;
  for (uint64_t b = 0; e == hipSuccess && b < (1ull << 32); b += chunk) {
    hipLaunchKernelGGL(bf16_check_kernel, dim3(chunk / 256), dim3(256), 0, 0, static_cast<uint32_t>(b), d);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipDeviceSynchronize();
  }
  unsigned long long h = 0;
  if (e == hipSuccess) e = hipMemcpy(&h, d, sizeof(h), hipMemcpyDeviceToHost);
  (void)hipFree(d);
  counts[0] = h & 0xffffffffull;
  counts[1] = h >> 32;
  return static_cast<int>(e);
}
