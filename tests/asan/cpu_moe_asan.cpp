// Host-side AddressSanitizer run of the CPU baseline's restatement of the
// reference CPU executor (oracle/cpu_moe/cpu_moe.cpp): exact-size banks in
// bf16 and MXFP4, skipped and out-of-range routes, repeated pools.  Exit
// status 0 and "asan cpu_moe ok" on success.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

extern "C" {
void* cpumoe_create(int H, int I, int top_k, int num_experts, int fmt, const int* cpus, int ncpus);
void cpumoe_set_bank(void* h, const void* gate_up, const void* down, const void* gu_scale, const void* dn_scale);
void cpumoe_run(void* h, const void* x, const float* w, const int32_t* ids, int M, void* y);
void cpumoe_destroy(void* h);
void cpumoe_fill_bf16(void* dst, size_t n, float a, uint64_t seed, int nthreads);
}

int main() {
  std::mt19937 rng(99);
  const int cpus[] = {0, 0, 0};
  for (int fmt : {0, 1}) {
    const int E = 6, H = 256, I = 384, k = 4;
    std::vector<uint8_t> gu, dn, gus, dns;
    if (fmt == 0) {
      gu.resize(size_t(E) * 2 * I * H * 2);
      dn.resize(size_t(E) * H * I * 2);
      cpumoe_fill_bf16(gu.data(), gu.size() / 2, 0.05f, 1, 2);
      cpumoe_fill_bf16(dn.data(), dn.size() / 2, 0.05f, 2, 2);
    } else {
      gu.resize(size_t(E) * 2 * I * H / 2);
      dn.resize(size_t(E) * H * I / 2);
      for (auto& v : gu) v = uint8_t(rng());
      for (auto& v : dn) v = uint8_t(rng());
      gus.assign(size_t(E) * 2 * I * (H / 32), 120);
      dns.assign(size_t(E) * H * (I / 32), 120);
    }
    for (int rep = 0; rep < 3; ++rep) {
      void* p = cpumoe_create(H, I, k, E, fmt, cpus, 1 + rep);
      cpumoe_set_bank(p, gu.data(), dn.data(), gus.empty() ? nullptr : gus.data(), dns.empty() ? nullptr : dns.data());
      for (int M : {1, 5}) {
        std::vector<uint16_t> x(size_t(M) * H), y(size_t(M) * H);
        cpumoe_fill_bf16(x.data(), x.size(), 1.0f, 3 + M, 1);
        std::vector<float> w(size_t(M) * k, 0.25f);
        std::vector<int32_t> ids(size_t(M) * k);
        for (auto& v : ids) v = int(rng() % (E + 3)) - 1;  // -1 and ids >= E are skipped
        cpumoe_run(p, x.data(), w.data(), ids.data(), M, y.data());
        for (uint16_t v : y) {
          uint32_t u = uint32_t(v) << 16;
          float f;
          std::memcpy(&f, &u, 4);
          if (!std::isfinite(f)) return 1;
        }
      }
      cpumoe_destroy(p);
    }
  }
  std::puts("asan cpu_moe ok");
  return 0;
}
