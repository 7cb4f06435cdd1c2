// CPU MoE decode executor -- restatement of FreeToken's CPU MoE-offload path,
// used as the CPU baseline timed beside the GPU and as a second checker of the
// bf16 expert math.  TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
//
// Algorithm restated from kernel/csrc/cpu_moe/cpu_moe_ext.cpp of the reference:
//   * two passes over a persistent pool of pinned worker threads, one per
//     physical core (moe/cpu_executor.py:91-140);
//   * pass 1, work unit (token, route, 32-row I tile): gate row i and up row I+i
//     dotted with the token's activations in fp32, SwiGLU, bf16 intermediate
//     (cpu_moe_ext.cpp:1574-1627, IBLK = 32 at :1096);
//   * spin barrier between the passes (:1833-1857);
//   * pass 2, work unit (token, 32-row H tile): down rows dotted with each route's
//     intermediate, times the router weight, summed over the routes, bf16 out
//     (:1629-1668, HBLK = 32 at :1097);
//   * work is grabbed with an atomic counter (:1833-1857);
//   * ISA ladder avx512bf16 > avx512f > avx2 > scalar chosen once (:671-706);
//   * the row-major MXFP4 ("ds_fp4") format decodes e2m1 * 2^(e8m0-127) per 32
//     values inside the dot (:1745-1832), here with bf16 activations (no FP8
//     activation round trip) and no SwiGLU clamp.
// The code is this build's own; only the algorithm is restated.
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <unistd.h>

#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

namespace {

using bf16 = uint16_t;

inline float b2f(bf16 v) {
  uint32_t u = static_cast<uint32_t>(v) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

inline bf16 f2b(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<bf16>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<bf16>(u >> 16);
}

constexpr int kTile = 32;  // IBLK = HBLK = 32

const float kE2M1[16] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f, -0.f, -.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f};

// ---------------------------------------------------------------- bf16 dots
float dot_scalar(const bf16* w, const bf16* x, int n) {
  float acc = 0.f;
  for (int i = 0; i < n; ++i) acc += b2f(w[i]) * b2f(x[i]);
  return acc;
}

__attribute__((target("avx2,fma"))) float dot_avx2(const bf16* w, const bf16* x, int n) {
  __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
  int i = 0;
  for (; i + 32 <= n; i += 32) {
    for (int u = 0; u < 4; ++u) {
      const __m256i wv = _mm256_cvtepu16_epi32(_mm_loadu_si128(reinterpret_cast<const __m128i*>(w + i + 8 * u)));
      const __m256i xv = _mm256_cvtepu16_epi32(_mm_loadu_si128(reinterpret_cast<const __m128i*>(x + i + 8 * u)));
      acc[u] = _mm256_fmadd_ps(_mm256_castsi256_ps(_mm256_slli_epi32(wv, 16)),
                               _mm256_castsi256_ps(_mm256_slli_epi32(xv, 16)), acc[u]);
    }
  }
  __m256 s = _mm256_add_ps(_mm256_add_ps(acc[0], acc[1]), _mm256_add_ps(acc[2], acc[3]));
  float t[8];
  _mm256_storeu_ps(t, s);
  float r = t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6] + t[7];
  for (; i < n; ++i) r += b2f(w[i]) * b2f(x[i]);
  return r;
}

__attribute__((target("avx512f"))) float dot_avx512(const bf16* w, const bf16* x, int n) {
  __m512 acc[4] = {_mm512_setzero_ps(), _mm512_setzero_ps(), _mm512_setzero_ps(), _mm512_setzero_ps()};
  int i = 0;
  for (; i + 64 <= n; i += 64) {
    for (int u = 0; u < 4; ++u) {
      const __m512i wv = _mm512_cvtepu16_epi32(_mm256_loadu_si256(reinterpret_cast<const __m256i*>(w + i + 16 * u)));
      const __m512i xv = _mm512_cvtepu16_epi32(_mm256_loadu_si256(reinterpret_cast<const __m256i*>(x + i + 16 * u)));
      acc[u] = _mm512_fmadd_ps(_mm512_castsi512_ps(_mm512_slli_epi32(wv, 16)),
                               _mm512_castsi512_ps(_mm512_slli_epi32(xv, 16)), acc[u]);
    }
  }
  float r = _mm512_reduce_add_ps(_mm512_add_ps(_mm512_add_ps(acc[0], acc[1]), _mm512_add_ps(acc[2], acc[3])));
  for (; i < n; ++i) r += b2f(w[i]) * b2f(x[i]);
  return r;
}

__attribute__((target("avx512f,avx512bf16"))) float dot_avx512bf16(const bf16* w, const bf16* x, int n) {
  __m512 acc[4] = {_mm512_setzero_ps(), _mm512_setzero_ps(), _mm512_setzero_ps(), _mm512_setzero_ps()};
  int i = 0;
  for (; i + 128 <= n; i += 128) {
    for (int u = 0; u < 4; ++u) {
      const __m512i wv = _mm512_loadu_si512(w + i + 32 * u);
      const __m512i xv = _mm512_loadu_si512(x + i + 32 * u);
      acc[u] = _mm512_dpbf16_ps(acc[u], (__m512bh)wv, (__m512bh)xv);
    }
  }
  float r = _mm512_reduce_add_ps(_mm512_add_ps(_mm512_add_ps(acc[0], acc[1]), _mm512_add_ps(acc[2], acc[3])));
  for (; i < n; ++i) r += b2f(w[i]) * b2f(x[i]);
  return r;
}

// ---------------------------------------------------------------- ds_fp4 dots
// w: packed row (n/2 bytes, low nibble = even k), s: e8m0 codes (n/32), x: bf16 [n]
float dot_fp4_scalar(const uint8_t* w, const uint8_t* s, const bf16* x, int n) {
  float acc = 0.f;
  for (int b = 0; b < n / 32; ++b) {
    float part = 0.f;
    for (int j = 0; j < 16; ++j) {
      const uint8_t byte = w[b * 16 + j];
      part += kE2M1[byte & 15] * b2f(x[b * 32 + 2 * j]) + kE2M1[byte >> 4] * b2f(x[b * 32 + 2 * j + 1]);
    }
    acc += part * std::ldexp(1.0f, static_cast<int>(s[b]) - 127);
  }
  return acc;
}

__attribute__((target("avx512f,avx512bw"))) float dot_fp4_avx512(const uint8_t* w, const uint8_t* s, const bf16* x,
                                                                 int n) {
  const __m512 lut = _mm512_loadu_ps(kE2M1);
  __m512 acc = _mm512_setzero_ps();
  for (int b = 0; b < n / 32; ++b) {
    // 16 bytes -> 32 codes in k order: interleave low/high nibbles
    const __m128i raw = _mm_loadu_si128(reinterpret_cast<const __m128i*>(w + b * 16));
    const __m512i bytes = _mm512_cvtepu8_epi32(raw);
    const __m512i lo = _mm512_and_si512(bytes, _mm512_set1_epi32(15));
    const __m512i hi = _mm512_srli_epi32(bytes, 4);
    const __m512 wlo = _mm512_permutexvar_ps(lo, lut);  // even k
    const __m512 whi = _mm512_permutexvar_ps(hi, lut);  // odd k
    // x pairs (even, odd) as one 32-bit lane each
    const __m512i xp = _mm512_loadu_si512(x + b * 32);
    const __m512 xe = _mm512_castsi512_ps(_mm512_slli_epi32(xp, 16));
    const __m512 xo = _mm512_castsi512_ps(_mm512_and_si512(xp, _mm512_set1_epi32(static_cast<int>(0xffff0000u))));
    const __m512 part = _mm512_fmadd_ps(wlo, xe, _mm512_mul_ps(whi, xo));
    acc = _mm512_fmadd_ps(part, _mm512_set1_ps(std::ldexp(1.0f, static_cast<int>(s[b]) - 127)), acc);
  }
  return _mm512_reduce_add_ps(acc);
}

using dot_fn = float (*)(const bf16*, const bf16*, int);
using dot4_fn = float (*)(const uint8_t*, const uint8_t*, const bf16*, int);

struct Pool;

void pin_to_cpu(int cpu) {
  cpu_set_t set;
  CPU_ZERO(&set);
  CPU_SET(cpu, &set);
  pthread_setaffinity_np(pthread_self(), sizeof(set), &set);
}

struct Pool {
  // configuration
  int H, I, k, E, fmt, nthreads;
  dot_fn dot = dot_scalar;
  dot4_fn dot4 = dot_fp4_scalar;
  const char* isa = "scalar";
  // banks
  const uint8_t* gate_up = nullptr;   // bf16 [E, 2I, H] or packed [E, 2I, H/2]
  const uint8_t* down = nullptr;      // bf16 [E, H, I] or packed [E, H, I/2]
  const uint8_t* gu_scale = nullptr;  // [E, 2I, H/32]
  const uint8_t* dn_scale = nullptr;  // [E, H, I/32]
  std::vector<int> cpus;
  // task
  const bf16* x = nullptr;
  const float* w = nullptr;
  const int32_t* ids = nullptr;
  bf16* y = nullptr;
  int M = 0;
  std::vector<bf16> g;  // [M*k, I] intermediate
  std::atomic<int64_t> p1{0}, p2{0};
  int64_t p1_total = 0, p2_total = 0;
  std::atomic<int> bar{0};
  std::atomic<uint64_t> gen{0};
  std::atomic<int> done{0};
  std::atomic<bool> stop{false};
  std::vector<std::thread> threads;

  const bf16* row_bf16(const uint8_t* base, size_t rows_per_e, int e, int r, int len) const {
    return reinterpret_cast<const bf16*>(base) + (static_cast<size_t>(e) * rows_per_e + r) * len;
  }

  float row_dot(bool first, int e, int r, const bf16* act, int len) const {
    const size_t rows = first ? 2 * static_cast<size_t>(I) : static_cast<size_t>(H);
    const uint8_t* base = first ? gate_up : down;
    if (fmt == 0) return dot(row_bf16(base, rows, e, r, len), act, len);
    const uint8_t* sb = first ? gu_scale : dn_scale;
    const size_t ridx = static_cast<size_t>(e) * rows + r;
    return dot4(base + ridx * (len / 2), sb + ridx * (len / 32), act, len);
  }

  void pass1(int64_t p) {
    const int n_iblk = (I + kTile - 1) / kTile;
    const int ib = static_cast<int>(p % n_iblk);
    const int64_t tk = p / n_iblk;
    const int r = static_cast<int>(tk % k), t = static_cast<int>(tk / k);
    const int e = ids[static_cast<size_t>(t) * k + r];
    if (e < 0 || e >= E) return;
    const bf16* xr = x + static_cast<size_t>(t) * H;
    bf16* gr = g.data() + (static_cast<size_t>(t) * k + r) * I;
    for (int i = ib * kTile; i < std::min(I, (ib + 1) * kTile); ++i) {
      const float gate = b2f(f2b(row_dot(true, e, i, xr, H)));
      const float up = b2f(f2b(row_dot(true, e, I + i, xr, H)));
      gr[i] = f2b(gate / (1.0f + std::exp(-gate)) * up);
    }
  }

  void pass2(int64_t p) {
    const int n_hblk = (H + kTile - 1) / kTile;
    const int hb = static_cast<int>(p % n_hblk);
    const int t = static_cast<int>(p / n_hblk);
    bf16* yr = y + static_cast<size_t>(t) * H;
    for (int h = hb * kTile; h < std::min(H, (hb + 1) * kTile); ++h) {
      float acc = 0.f;
      for (int r = 0; r < k; ++r) {
        const int e = ids[static_cast<size_t>(t) * k + r];
        if (e < 0 || e >= E) continue;
        const bf16* gr = g.data() + (static_cast<size_t>(t) * k + r) * I;
        acc += b2f(f2b(row_dot(false, e, h, gr, I) * w[static_cast<size_t>(t) * k + r]));
      }
      yr[h] = f2b(acc);
    }
  }

  void spin_barrier(uint64_t round) {
    // sense-free barrier on a monotone counter: round r completes at (r+1)*n arrivals
    bar.fetch_add(1, std::memory_order_acq_rel);
    const int target = static_cast<int>((round + 1) * nthreads);
    while (bar.load(std::memory_order_acquire) < target) _mm_pause();
  }

  void body(uint64_t round_base) {
    for (;;) {
      const int64_t p = p1.fetch_add(1, std::memory_order_relaxed);
      if (p >= p1_total) break;
      pass1(p);
    }
    spin_barrier(round_base);
    for (;;) {
      const int64_t p = p2.fetch_add(1, std::memory_order_relaxed);
      if (p >= p2_total) break;
      pass2(p);
    }
  }

  void worker(int tid) {
    if (tid < static_cast<int>(cpus.size())) pin_to_cpu(cpus[tid]);
    uint64_t seen = 0;
    for (;;) {
      uint64_t cur;
      while ((cur = gen.load(std::memory_order_acquire)) == seen) {
        if (stop.load(std::memory_order_acquire)) return;
        _mm_pause();
      }
      seen = cur;
      body(cur - 1);
      done.fetch_add(1, std::memory_order_acq_rel);
    }
  }

  void run(const bf16* x_, const float* w_, const int32_t* ids_, int M_, bf16* y_) {
    x = x_;
    w = w_;
    ids = ids_;
    y = y_;
    M = M_;
    const size_t need = static_cast<size_t>(M) * k * I;
    if (g.size() < need) g.resize(need);
    p1_total = static_cast<int64_t>(M) * k * ((I + kTile - 1) / kTile);
    p2_total = static_cast<int64_t>(M) * ((H + kTile - 1) / kTile);
    p1.store(0);
    p2.store(0);
    done.store(0);
    const uint64_t round = gen.load();
    bar.store(static_cast<int>(round * nthreads));
    gen.store(round + 1, std::memory_order_release);
    while (done.load(std::memory_order_acquire) < nthreads) _mm_pause();
  }
};

void choose_isa(Pool* p) {
  const char* force = std::getenv("FTMOE_CPU_ISA");
  __builtin_cpu_init();
  const bool bf = __builtin_cpu_supports("avx512bf16");
  const bool f = __builtin_cpu_supports("avx512f");
  const bool bw = __builtin_cpu_supports("avx512bw");
  const bool a2 = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
  auto want = [&](const char* s) { return !force || std::strcmp(force, s) == 0; };
  if (bf && want("avx512bf16")) {
    p->dot = dot_avx512bf16;
    p->isa = "avx512bf16";
  } else if (f && want("avx512f")) {
    p->dot = dot_avx512;
    p->isa = "avx512f";
  } else if (a2 && want("avx2")) {
    p->dot = dot_avx2;
    p->isa = "avx2";
  }
  if (f && bw && (!force || std::strcmp(force, "scalar") != 0)) p->dot4 = dot_fp4_avx512;
}

}  // namespace

extern "C" {

// One thread per listed CPU (the caller lists one logical CPU per physical core).
void* cpumoe_create(int H, int I, int top_k, int num_experts, int fmt, const int* cpus, int ncpus) {
  auto* p = new Pool();
  p->H = H;
  p->I = I;
  p->k = top_k;
  p->E = num_experts;
  p->fmt = fmt;
  p->nthreads = ncpus > 0 ? ncpus : 1;
  for (int i = 0; i < ncpus; ++i) p->cpus.push_back(cpus[i]);
  choose_isa(p);
  for (int t = 0; t < p->nthreads; ++t) p->threads.emplace_back(&Pool::worker, p, t);
  return p;
}

const char* cpumoe_isa(void* h) { return static_cast<Pool*>(h)->isa; }

void cpumoe_set_bank(void* h, const void* gate_up, const void* down, const void* gu_scale, const void* dn_scale) {
  auto* p = static_cast<Pool*>(h);
  p->gate_up = static_cast<const uint8_t*>(gate_up);
  p->down = static_cast<const uint8_t*>(down);
  p->gu_scale = static_cast<const uint8_t*>(gu_scale);
  p->dn_scale = static_cast<const uint8_t*>(dn_scale);
}

// Synchronous decode (the reference's run_task, submit + sync).
void cpumoe_run(void* h, const void* x, const float* w, const int32_t* ids, int M, void* y) {
  static_cast<Pool*>(h)->run(static_cast<const bf16*>(x), w, ids, M, static_cast<bf16*>(y));
}

void cpumoe_destroy(void* h) {
  auto* p = static_cast<Pool*>(h);
  p->stop.store(true, std::memory_order_release);
  for (auto& t : p->threads) t.join();
  delete p;
}

// Fills n bf16 values ~ U(-a, a) from a counter hash, in parallel (bench banks).
void cpumoe_fill_bf16(void* dst, size_t n, float a, uint64_t seed, int nthreads) {
  auto* out = static_cast<bf16*>(dst);
  std::vector<std::thread> ts;
  const int T = nthreads > 0 ? nthreads : 1;
  for (int t = 0; t < T; ++t)
    ts.emplace_back([=] {
      const size_t b = n * t / T, e = n * (t + 1) / T;
      for (size_t i = b; i < e; ++i) {
        uint64_t z = (i + seed * 0x9E3779B97F4A7C15ull) * 0xBF58476D1CE4E5B9ull;
        z ^= z >> 31;
        z *= 0x94D049BB133111EBull;
        z ^= z >> 29;
        const float u = static_cast<float>(z >> 40) * (1.0f / 16777216.0f);
        out[i] = f2b((2.0f * u - 1.0f) * a);
      }
    });
  for (auto& t : ts) t.join();
}

}  // extern "C"
