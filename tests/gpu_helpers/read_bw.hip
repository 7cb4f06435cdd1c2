// Test helper (not part of libftmoe.so): the HBM read bandwidth a plain
// streaming kernel reaches on this GPU, the practical ceiling against which
// the decode GEMVs' bandwidth is read.  Each thread XORs 16-byte loads of a
// buffer far larger than the caches (grid-stride, U loads in flight per
// thread, nontemporal or not) into one register and writes it once; the best
// rate over a few grid sizes and load depths is returned.
#include <cstdint>

#include <hip/hip_runtime.h>

namespace {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

template <int U, bool NT>
__global__ void __launch_bounds__(256) read_kernel(const u32x4_t* __restrict__ p, size_t n, unsigned* out) {
  size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) * U + threadIdx.x;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x * U;
  unsigned acc = 0;
  for (; i + (U - 1) * blockDim.x < n; i += stride) {
    u32x4_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(p + i + u * blockDim.x) : p[i + u * blockDim.x];
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

template <int U, bool NT>
hipError_t time_read(const u32x4_t* d, size_t n, unsigned* out, int grid, int reps, double* tbs) {
  hipEvent_t a, b;
  hipError_t e = hipEventCreate(&a);
  if (e != hipSuccess) return e;
  e = hipEventCreate(&b);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((read_kernel<U, NT>), dim3(grid), dim3(256), 0, 0, d, n, out);  // warm-up
  e = hipEventRecord(a);
  for (int r = 0; e == hipSuccess && r < reps; ++r) {
    hipLaunchKernelGGL((read_kernel<U, NT>), dim3(grid), dim3(256), 0, 0, d, n, out);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipEventRecord(b);
  if (e == hipSuccess) e = hipEventSynchronize(b);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  if (e == hipSuccess) *tbs = static_cast<double>(n) * 16.0 * reps / (ms * 1e-3) / 1e12;
  return e;
}

}  // namespace

// best[0]: the best rate in TB/s over grids {1024, 2048, 4096, 8192} x
// {8, 16 loads in flight} x {nontemporal, plain}; best[1]: its grid, best[2]:
// its depth, best[3]: 1 if nontemporal.  Reads a 4 GiB buffer.  Returns 0, or
// a HIP error code.
extern "C" int ftmoe_test_read_bandwidth(double* best) {
  const size_t bytes = size_t{4} << 30, n = bytes / 16;
  u32x4_t* d = nullptr;
  unsigned* out = nullptr;
  hipError_t e = hipMalloc(&d, bytes);
  if (e != hipSuccess) return static_cast<int>(e);
  e = hipMalloc(&out, size_t{8192} * 256 * sizeof(unsigned));
  if (e == hipSuccess) e = hipMemset(d, 1, bytes);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  best[0] = best[1] = best[2] = best[3] = 0.0;
  const int grids[] = {1024, 2048, 4096, 8192};
  for (int grid : grids) {
    double r[4] = {0, 0, 0, 0};
    if (e == hipSuccess) e = time_read<8, true>(d, n, out, grid, 8, &r[0]);
    if (e == hipSuccess) e = time_read<16, true>(d, n, out, grid, 8, &r[1]);
    if (e == hipSuccess) e = time_read<8, false>(d, n, out, grid, 8, &r[2]);
    if (e == hipSuccess) e = time_read<16, false>(d, n, out, grid, 8, &r[3]);
    for (int k = 0; k < 4; ++k)
      if (r[k] > best[0]) {
        best[0] = r[k];
        best[1] = grid;
        best[2] = (k & 1) ? 16 : 8;
        best[3] = k < 2 ? 1 : 0;
      }
  }
  (void)hipFree(d);
  (void)hipFree(out);
  return static_cast<int>(e);
}
