// Host-side AddressSanitizer run of the hybrid decode's CPU expert executor
// (freetoken_amd/csrc/cpu_experts.hip, synchronous entry point only: no HIP
// call is made).  Every bank lives in a heap buffer of its exact size, so a
// read past an expert's rows, past a scale table or past the activations is
// reported.  Exercises all three formats, ragged batches with skipped and
// out-of-range routes, the activation variants, the watchdog failure path and
// repeated create/destroy of the pool.  Exit status 0 and "asan executor ok"
// on success.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "ftmoe.h"

namespace ftmoe {
int report_error(int code, const char* msg) {
  std::fprintf(stderr, "ftmoe error %d: %s\n", code, msg);
  return code;
}
}  // namespace ftmoe

namespace {

uint16_t f2b(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return static_cast<uint16_t>((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

float b2f(uint16_t b) {
  const uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

struct HostBank {
  std::vector<uint8_t> gu, dn, gus, dns;
  ftmoe_bank b{};
};

HostBank make_bank(int fmt, int E, int H, int I, std::mt19937& rng) {
  HostBank hb;
  std::uniform_int_distribution<int> byte(0, 255);
  const size_t ngu = static_cast<size_t>(E) * 2 * I * H, ndn = static_cast<size_t>(E) * H * I;
  if (fmt == FTMOE_FMT_BF16) {
    std::normal_distribution<float> nd(0.f, 0.05f);
    hb.gu.resize(ngu * 2);
    hb.dn.resize(ndn * 2);
    auto* g = reinterpret_cast<uint16_t*>(hb.gu.data());
    auto* d = reinterpret_cast<uint16_t*>(hb.dn.data());
    for (size_t i = 0; i < ngu; ++i) g[i] = f2b(nd(rng));
    for (size_t i = 0; i < ndn; ++i) d[i] = f2b(nd(rng));
  } else if (fmt == FTMOE_FMT_FP8_B128) {
    hb.gu.resize(ngu);
    hb.dn.resize(ndn);
    for (auto& v : hb.gu) v = static_cast<uint8_t>(byte(rng) & 0x77);  // finite e4m3 codes
    for (auto& v : hb.dn) v = static_cast<uint8_t>(byte(rng) & 0x77);
    const size_t sgu = static_cast<size_t>(E) * (2 * I / 128) * (H / 128), sdn = static_cast<size_t>(E) * (H / 128) * (I / 128);
    hb.gus.resize(sgu * 4);
    hb.dns.resize(sdn * 4);
    for (size_t i = 0; i < sgu; ++i) reinterpret_cast<float*>(hb.gus.data())[i] = 1e-3f;
    for (size_t i = 0; i < sdn; ++i) reinterpret_cast<float*>(hb.dns.data())[i] = 1e-3f;
  } else {
    hb.gu.resize(ngu / 2);
    hb.dn.resize(ndn / 2);
    for (auto& v : hb.gu) v = static_cast<uint8_t>(byte(rng));
    for (auto& v : hb.dn) v = static_cast<uint8_t>(byte(rng));
    hb.gus.resize(static_cast<size_t>(E) * 2 * I * (H / 32));
    hb.dns.resize(static_cast<size_t>(E) * H * (I / 32));
    for (auto& v : hb.gus) v = static_cast<uint8_t>(118 + byte(rng) % 4);
    for (auto& v : hb.dns) v = static_cast<uint8_t>(118 + byte(rng) % 4);
  }
  hb.b.format = fmt;
  hb.b.num_rows = E;
  hb.b.hidden = H;
  hb.b.inter = I;
  hb.b.gate_up = hb.gu.data();
  hb.b.down = hb.dn.data();
  hb.b.gate_up_scale = hb.gus.empty() ? nullptr : hb.gus.data();
  hb.b.down_scale = hb.dns.empty() ? nullptr : hb.dns.data();
  return hb;
}

int run_case(ftmoe_cpu_executor* ex, const HostBank& hb, int M, int k, int act, std::mt19937& rng) {
  const int H = hb.b.hidden, E = hb.b.num_rows;
  std::vector<uint16_t> x(static_cast<size_t>(M) * H), y(static_cast<size_t>(M) * H, 0xFFFF);
  std::normal_distribution<float> nd(0.f, 1.f);
  for (auto& v : x) v = f2b(nd(rng));
  std::vector<float> w(static_cast<size_t>(M) * k, 0.25f);
  std::vector<int32_t> ids(static_cast<size_t>(M) * k);
  std::uniform_int_distribution<int> pick(-2, E + 1);  // skipped and out-of-range routes included
  for (auto& v : ids) v = pick(rng);
  const int rc = ftmoe_cpu_experts(ex, &hb.b, x.data(), w.data(), ids.data(), M, k, act, y.data());
  if (rc != FTMOE_OK) return rc;
  for (uint16_t v : y)
    if (!std::isfinite(b2f(v))) return -100;
  return 0;
}

}  // namespace

int main() {
  std::mt19937 rng(1234);
  const int fmts[] = {FTMOE_FMT_BF16, FTMOE_FMT_FP8_B128, FTMOE_FMT_MXFP4};
  ftmoe_cpu_executor* ex = ftmoe_cpu_executor_create(3);
  // (experts, hidden, inter): a larger bank, and a small one whose FP8 / MXFP4
  // buffers are small heap blocks with redzones right after their last row
  const int shapes[][3] = {{5, 256, 384}, {2, 128, 128}};
  for (const auto& sh : shapes)
  for (int fmt : fmts) {
    const HostBank hb = make_bank(fmt, sh[0], sh[1], sh[2], rng);
    for (int M : {1, 3, 9})
      for (int k : {1, 4, 8})
        for (int act : {FTMOE_ACT_SILU, FTMOE_ACT_GELU, FTMOE_ACT_GELU_TANH}) {
          const int rc = run_case(ex, hb, M, k, act, rng);
          if (rc) {
            std::fprintf(stderr, "case fmt %d M %d k %d act %d failed: %d\n", fmt, M, k, act, rc);
            return 1;
          }
        }
  }
  // the watchdog: a held pool fails the job after the period, then fails at once
  const HostBank small = make_bank(FTMOE_FMT_BF16, 2, 128, 128, rng);
  ftmoe_cpu_executor_set_watchdog(ex, 100);
  ftmoe_cpu_executor_hold(ex, 1);
  if (run_case(ex, small, 2, 2, FTMOE_ACT_SILU, rng) != FTMOE_ERR_TIMEOUT) return 2;
  if (ftmoe_cpu_executor_healthy(ex) != FTMOE_ERR_TIMEOUT) return 3;
  ftmoe_cpu_executor_hold(ex, 0);
  if (run_case(ex, small, 2, 2, FTMOE_ACT_SILU, rng) != FTMOE_ERR_TIMEOUT) return 4;
  if (ftmoe_cpu_executor_destroy(ex, 0) != FTMOE_OK) return 5;
  // pool lifecycle: threads started and joined cleanly, jobs in between
  for (int i = 0; i < 20; ++i) {
    ftmoe_cpu_executor* e = ftmoe_cpu_executor_create(1 + i % 4);
    if (i % 2 && run_case(e, small, 1 + i % 3, 2, FTMOE_ACT_SILU, rng)) return 6;
    if (ftmoe_cpu_executor_destroy(e, 0) != FTMOE_OK) return 7;
  }
  std::puts("asan executor ok");
  return 0;
}
