// Host-side expert executor of the hybrid decode: the routes whose experts are
// neither resident nor fetched this call are computed on the CPU from the
// pinned host banks while the GPU computes the others (reference: the hybrid
// backend, layers/moe.py:325-372, with its CPU pool, moe/cpu_executor.py).
//
// Math per route (the decode rounding points of the GPU path): g = W_gate x,
// u = W_up x in fp32 (FP8: per 128-deep K block partial times the block scale;
// MXFP4: e2m1 * 2^(e8m0 - 127)), rounded to bf16; act = bf16(silu(g) * u);
// d = W_down act the same way, times the router weight, rounded to bf16; the
// token's output is bf16 of the fp32 sum of its CPU routes in route order.
//
// Work: the routes are grouped by expert, so that every weight row is read
// once per step for all the tokens routed to its expert (up to kMaxVec at a
// time): pass 1 over (expert, 32 rows of I) -> act; pass 2 over (expert, 32
// rows of H) -> the weighted, bf16-rounded down output of each route; pass 3
// over tokens sums its routes in route order.  A route's numbers do not depend
// on the grouping.  Units come from an atomic counter; a driver thread runs
// the passes of one job after the other and works in them beside a pool of
// workers, which spin briefly on the pass generation between passes.  The
// stream sees the job through two
// host-function nodes: "submit" hands the job to the driver and returns at
// once, "wait" blocks the stream until the job is done -- so the CPU work
// overlaps whatever the stream runs between them (the GPU's share of the
// layer), and both nodes replay in a captured graph.
//
// Flag handshake (set_handshake(1), the reference's default where stream
// memory operations work, moe/cpu_executor.py:32-50): "submit" is a stream
// write of the job's ready flag (mapped pinned memory), a coordinator thread
// polls the flags of the armed jobs and hands a ready job to the driver, the
// driver raises the job's done flag when it ends, and "wait" is a stream wait
// on that flag followed by its reset -- no host function, so no runtime
// callback round trip.  The coordinator also runs the watchdog of these jobs
// (their waits are on the GPU, not in a host function): a job without pool
// progress for the watchdog period is failed and its done flag raised, so a
// stream never waits for ever.
#include <hip/hip_runtime.h>
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <type_traits>
#include <cstdlib>
#include <deque>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "ftmoe.h"
#include "kernels.h"

namespace ftmoe_cpu {

using bf16 = uint16_t;

inline float b2f(bf16 v) {
  const uint32_t u = static_cast<uint32_t>(v) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

inline bf16 f2b(float f) {  // round to nearest even
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<bf16>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<bf16>(u >> 16);
}

inline float rb(float f) { return b2f(f2b(f)); }

// e4m3 (bias 7, no infinities, S.1111.111 NaN) and e2m1 value tables
struct Tables {
  float e4m3[256];
  float e2m1[16];
  Tables() {
    for (int c = 0; c < 256; ++c) {
      const int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
      float v = e == 0 ? std::ldexp(static_cast<float>(m), -9) : std::ldexp(1.0f + m / 8.0f, e - 7);
      if (e == 15 && m == 7) v = NAN;
      e4m3[c] = s ? -v : v;
    }
    const float p[8] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
    for (int c = 0; c < 16; ++c) e2m1[c] = c & 8 ? -p[c & 7] : p[c & 7];
  }
};
const Tables kT;

// ---------------------------------------------------------------- row dots
// dot of weight row n (K values) with x (fp32, K), in the format's
// accumulation order: bf16 one pass; FP8 per 128-block partial * scale;
// MXFP4 per 32-block with its power-of-two scale.
struct Mat {
  int format;
  int K;
  const uint8_t* w;  // [N, K * bytes per value]
  const void* s;     // FP8 float [N/128, K/128]; MXFP4 uint8 [N, K/32]
};

constexpr int kMaxVec = 8;  // activation vectors per pass over a weight row

// dots of weight row n with nx activation vectors xs[] (each K fp32), in the
// format's accumulation order: bf16 one pass; FP8 per 128-block partial times
// the block scale; MXFP4 per 32-block times its power-of-two scale.
void dot_scalar(const Mat& m, int n, const float* const* xs, int nx, float* out) {
  for (int v = 0; v < nx; ++v) {
    const float* x = xs[v];
    float acc = 0.f;
    if (m.format == FTMOE_FMT_BF16) {
      const bf16* w = reinterpret_cast<const bf16*>(m.w) + static_cast<size_t>(n) * m.K;
      for (int k = 0; k < m.K; ++k) acc += b2f(w[k]) * x[k];
    } else if (m.format == FTMOE_FMT_FP8_B128) {
      const uint8_t* w = m.w + static_cast<size_t>(n) * m.K;
      const float* s = static_cast<const float*>(m.s) + static_cast<size_t>(n / 128) * (m.K / 128);
      for (int kb = 0; kb < m.K / 128; ++kb) {
        float part = 0.f;
        for (int k = 0; k < 128; ++k) part += kT.e4m3[w[kb * 128 + k]] * x[kb * 128 + k];
        acc += part * s[kb];
      }
    } else {
      const uint8_t* w = m.w + static_cast<size_t>(n) * (m.K / 2);
      const uint8_t* s = static_cast<const uint8_t*>(m.s) + static_cast<size_t>(n) * (m.K / 32);
      for (int kb = 0; kb < m.K / 32; ++kb) {
        float part = 0.f;
        for (int k = 0; k < 32; k += 2) {
          const uint8_t b = w[kb * 16 + k / 2];
          part += kT.e2m1[b & 15] * x[kb * 32 + k] + kT.e2m1[b >> 4] * x[kb * 32 + k + 1];
        }
        acc += part * std::ldexp(1.0f, static_cast<int>(s[kb]) - 127);
      }
    }
    out[v] = acc;
  }
}

// AVX-512: each 32 weights are decoded to fp32 once and used for every
// vector.  FP8 codes widen to 16 bits and become fp16 by a shift (sign to bit
// 15, exponent and mantissa under fp16's, exact for every finite e4m3 value
// including subnormals: the fp16 holds value / 2^8), then fp32 by vcvtph2ps;
// the 2^8 rides on the block scale, so the block partial times (scale * 2^8)
// is the same product.  MXFP4 looks its values up with one permute and
// interleaves the low / high nibbles back into k order.
template <int FMT, int NX>
__attribute__((target("avx512f,avx512bw"))) void dot_avx512_t(const Mat& m, int n, const float* const* xs,
                                                               float* out) {
  // A independent accumulator chains per vector: few vectors would otherwise
  // wait on the FMA latency
  constexpr int A = NX <= 4 ? 2 : 1;
  __m512 acc[A][NX];
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int v = 0; v < NX; ++v) acc[a][v] = _mm512_setzero_ps();
  if constexpr (FMT == FTMOE_FMT_BF16) {
    const bf16* w = reinterpret_cast<const bf16*>(m.w) + static_cast<size_t>(n) * m.K;
    for (int k = 0; k < m.K; k += 32) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const __m512 wv = _mm512_castsi512_ps(_mm512_slli_epi32(
            _mm512_cvtepu16_epi32(_mm256_loadu_si256(reinterpret_cast<const __m256i*>(w + k + 16 * c))), 16));
#pragma unroll
        for (int v = 0; v < NX; ++v)
          acc[c % A][v] = _mm512_fmadd_ps(wv, _mm512_loadu_ps(xs[v] + k + 16 * c), acc[c % A][v]);
      }
    }
  } else if constexpr (FMT == FTMOE_FMT_FP8_B128) {
    const uint8_t* w = m.w + static_cast<size_t>(n) * m.K;
    const float* s = static_cast<const float*>(m.s) + static_cast<size_t>(n / 128) * (m.K / 128);
    const __m512i sgn = _mm512_set1_epi16(0x80), mag = _mm512_set1_epi16(0x7F);
    for (int kb = 0; kb < m.K / 128; ++kb) {
      __m512 part[A][NX];
#pragma unroll
      for (int a = 0; a < A; ++a)
#pragma unroll
        for (int v = 0; v < NX; ++v) part[a][v] = _mm512_setzero_ps();
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int k = kb * 128 + 32 * c;
        const __m512i b = _mm512_cvtepu8_epi16(_mm256_loadu_si256(reinterpret_cast<const __m256i*>(w + k)));
        const __m512i h = _mm512_or_si512(_mm512_slli_epi16(_mm512_and_si512(b, sgn), 8),
                                          _mm512_slli_epi16(_mm512_and_si512(b, mag), 7));
        const __m512 w0 = _mm512_cvtph_ps(_mm512_castsi512_si256(h));
        const __m512 w1 = _mm512_cvtph_ps(_mm512_extracti64x4_epi64(h, 1));
#pragma unroll
        for (int v = 0; v < NX; ++v) {
          part[0][v] = _mm512_fmadd_ps(w0, _mm512_loadu_ps(xs[v] + k), part[0][v]);
          part[A - 1][v] = _mm512_fmadd_ps(w1, _mm512_loadu_ps(xs[v] + k + 16), part[A - 1][v]);
        }
      }
      const __m512 sc = _mm512_set1_ps(s[kb] * 256.0f);
#pragma unroll
      for (int v = 0; v < NX; ++v) {
        const __m512 p = A == 2 ? _mm512_add_ps(part[0][v], part[A - 1][v]) : part[0][v];
        acc[kb % A][v] = _mm512_fmadd_ps(p, sc, acc[kb % A][v]);
      }
    }
  } else {
    const uint8_t* w = m.w + static_cast<size_t>(n) * (m.K / 2);
    const uint8_t* s = static_cast<const uint8_t*>(m.s) + static_cast<size_t>(n) * (m.K / 32);
    const __m512 lut = _mm512_loadu_ps(kT.e2m1);
    const __m512i il0 = _mm512_setr_epi32(0, 16, 1, 17, 2, 18, 3, 19, 4, 20, 5, 21, 6, 22, 7, 23);
    const __m512i il1 = _mm512_setr_epi32(8, 24, 9, 25, 10, 26, 11, 27, 12, 28, 13, 29, 14, 30, 15, 31);
    for (int kb = 0; kb < m.K / 32; ++kb) {
      // 16 bytes = 32 values; even k in the low nibble
      const __m512i b = _mm512_cvtepu8_epi32(_mm_loadu_si128(reinterpret_cast<const __m128i*>(w + kb * 16)));
      const __m512 lo = _mm512_permutexvar_ps(_mm512_and_si512(b, _mm512_set1_epi32(15)), lut);
      const __m512 hi = _mm512_permutexvar_ps(_mm512_srli_epi32(b, 4), lut);
      const __m512 w0 = _mm512_permutex2var_ps(lo, il0, hi), w1 = _mm512_permutex2var_ps(lo, il1, hi);
      const __m512 sc = _mm512_set1_ps(std::ldexp(1.0f, static_cast<int>(s[kb]) - 127));
#pragma unroll
      for (int v = 0; v < NX; ++v) {
        const __m512 p = _mm512_fmadd_ps(w1, _mm512_loadu_ps(xs[v] + kb * 32 + 16),
                                         _mm512_mul_ps(w0, _mm512_loadu_ps(xs[v] + kb * 32)));
        acc[kb % A][v] = _mm512_fmadd_ps(p, sc, acc[kb % A][v]);
      }
    }
  }
#pragma unroll
  for (int v = 0; v < NX; ++v)
    out[v] = _mm512_reduce_add_ps(A == 2 ? _mm512_add_ps(acc[0][v], acc[A - 1][v]) : acc[0][v]);
}

template <int FMT>
void dot_avx512_f(const Mat& m, int n, const float* const* xs, int nx, float* out) {
  switch (nx) {
    case 1: return dot_avx512_t<FMT, 1>(m, n, xs, out);
    case 2: return dot_avx512_t<FMT, 2>(m, n, xs, out);
    case 3: return dot_avx512_t<FMT, 3>(m, n, xs, out);
    case 4: return dot_avx512_t<FMT, 4>(m, n, xs, out);
    case 5: return dot_avx512_t<FMT, 5>(m, n, xs, out);
    case 6: return dot_avx512_t<FMT, 6>(m, n, xs, out);
    case 7: return dot_avx512_t<FMT, 7>(m, n, xs, out);
    default: return dot_avx512_t<FMT, 8>(m, n, xs, out);
  }
}

void dot_avx512(const Mat& m, int n, const float* const* xs, int nx, float* out) {
  if (m.format == FTMOE_FMT_BF16) return dot_avx512_f<FTMOE_FMT_BF16>(m, n, xs, nx, out);
  if (m.format == FTMOE_FMT_FP8_B128) return dot_avx512_f<FTMOE_FMT_FP8_B128>(m, n, xs, nx, out);
  dot_avx512_f<FTMOE_FMT_MXFP4>(m, n, xs, nx, out);
}

static_assert(kMaxVec == 8, "dot_avx512_f dispatches 1..8 vectors");

// AVX512-BF16: the activation vectors stay bf16 and vdpbf16ps multiplies 32
// weight / activation pairs per instruction.  Every weight value is exact in
// bf16 (FP8 and e2m1 values have at most 4 significant bits; FP8 goes through
// the same fp16 shift as above, then fp32, then bf16 exactly), so the products
// are the fp32 ones; only the summation order differs (pairs, then lanes).
// The instruction treats bf16 subnormal inputs as zero: FP8 weights at 2^-8
// scale are normal, activations that small contribute below bf16 resolution.
__attribute__((target("avx512f,avx512bw,avx512bf16"))) inline __m512bh load_bh(const bf16* p) {
  return (__m512bh)_mm512_loadu_si512(p);
}

template <int FMT, int NX>
__attribute__((target("avx512f,avx512bw,avx512bf16"))) void dot_bf16_t(const Mat& m, int n, const bf16* const* xs,
                                                                        float* out) {
  constexpr int A = NX <= 4 ? 2 : 1;
  __m512 acc[A][NX];
#pragma unroll
  for (int a = 0; a < A; ++a)
#pragma unroll
    for (int v = 0; v < NX; ++v) acc[a][v] = _mm512_setzero_ps();
  if constexpr (FMT == FTMOE_FMT_BF16) {
    const bf16* w = reinterpret_cast<const bf16*>(m.w) + static_cast<size_t>(n) * m.K;
    for (int k = 0; k < m.K; k += 64) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const __m512bh wv = (__m512bh)_mm512_loadu_si512(w + k + 32 * c);
#pragma unroll
        for (int v = 0; v < NX; ++v) acc[c % A][v] = _mm512_dpbf16_ps(acc[c % A][v], wv, load_bh(xs[v] + k + 32 * c));
      }
    }
  } else if constexpr (FMT == FTMOE_FMT_FP8_B128) {
    const uint8_t* w = m.w + static_cast<size_t>(n) * m.K;
    const float* s = static_cast<const float*>(m.s) + static_cast<size_t>(n / 128) * (m.K / 128);
    const __m512i sgn = _mm512_set1_epi16(0x80), mag = _mm512_set1_epi16(0x7F);
    for (int kb = 0; kb < m.K / 128; ++kb) {
      __m512 part[A][NX];
#pragma unroll
      for (int a = 0; a < A; ++a)
#pragma unroll
        for (int v = 0; v < NX; ++v) part[a][v] = _mm512_setzero_ps();
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int k = kb * 128 + 32 * c;
        const __m512i b = _mm512_cvtepu8_epi16(_mm256_loadu_si256(reinterpret_cast<const __m256i*>(w + k)));
        const __m512i h = _mm512_or_si512(_mm512_slli_epi16(_mm512_and_si512(b, sgn), 8),
                                          _mm512_slli_epi16(_mm512_and_si512(b, mag), 7));
        const __m512bh wv = _mm512_cvtne2ps_pbh(_mm512_cvtph_ps(_mm512_extracti64x4_epi64(h, 1)),
                                                _mm512_cvtph_ps(_mm512_castsi512_si256(h)));
#pragma unroll
        for (int v = 0; v < NX; ++v) part[c % A][v] = _mm512_dpbf16_ps(part[c % A][v], wv, load_bh(xs[v] + k));
      }
      const __m512 sc = _mm512_set1_ps(s[kb] * 256.0f);
#pragma unroll
      for (int v = 0; v < NX; ++v) {
        const __m512 p = A == 2 ? _mm512_add_ps(part[0][v], part[A - 1][v]) : part[0][v];
        acc[kb % A][v] = _mm512_fmadd_ps(p, sc, acc[kb % A][v]);
      }
    }
  } else {
    const uint8_t* w = m.w + static_cast<size_t>(n) * (m.K / 2);
    const uint8_t* s = static_cast<const uint8_t*>(m.s) + static_cast<size_t>(n) * (m.K / 32);
    // e2m1 -> bf16 bits, indexed by the code
    alignas(64) static const uint16_t kLut[32] = {0x0000, 0x3F00, 0x3F80, 0x3FC0, 0x4000, 0x4040, 0x4080, 0x40C0,
                                                  0x8000, 0xBF00, 0xBF80, 0xBFC0, 0xC000, 0xC040, 0xC080, 0xC0C0};
    const __m512i lut = _mm512_load_si512(kLut);
    for (int kb = 0; kb < m.K / 32; ++kb) {
      // 16 bytes = 32 values; byte j holds k = 2j (low nibble) and 2j + 1, so
      // (low | high << 16) per 32-bit lane is k order
      const __m512i b = _mm512_cvtepu8_epi32(_mm_loadu_si128(reinterpret_cast<const __m128i*>(w + kb * 16)));
      const __m512i idx = _mm512_or_si512(_mm512_and_si512(b, _mm512_set1_epi32(15)),
                                          _mm512_slli_epi32(_mm512_srli_epi32(b, 4), 16));
      const __m512bh wv = (__m512bh)_mm512_permutexvar_epi16(idx, lut);
      const __m512 sc = _mm512_set1_ps(std::ldexp(1.0f, static_cast<int>(s[kb]) - 127));
#pragma unroll
      for (int v = 0; v < NX; ++v)
        acc[kb % A][v] = _mm512_fmadd_ps(_mm512_dpbf16_ps(_mm512_setzero_ps(), wv, load_bh(xs[v] + kb * 32)), sc, acc[kb % A][v]);
    }
  }
#pragma unroll
  for (int v = 0; v < NX; ++v)
    out[v] = _mm512_reduce_add_ps(A == 2 ? _mm512_add_ps(acc[0][v], acc[A - 1][v]) : acc[0][v]);
}

template <int FMT>
void dot_bf16_f(const Mat& m, int n, const bf16* const* xs, int nx, float* out) {
  switch (nx) {
    case 1: return dot_bf16_t<FMT, 1>(m, n, xs, out);
    case 2: return dot_bf16_t<FMT, 2>(m, n, xs, out);
    case 3: return dot_bf16_t<FMT, 3>(m, n, xs, out);
    case 4: return dot_bf16_t<FMT, 4>(m, n, xs, out);
    case 5: return dot_bf16_t<FMT, 5>(m, n, xs, out);
    case 6: return dot_bf16_t<FMT, 6>(m, n, xs, out);
    case 7: return dot_bf16_t<FMT, 7>(m, n, xs, out);
    default: return dot_bf16_t<FMT, 8>(m, n, xs, out);
  }
}

void dot_bf16(const Mat& m, int n, const bf16* const* xs, int nx, float* out) {
  if (m.format == FTMOE_FMT_BF16) return dot_bf16_f<FTMOE_FMT_BF16>(m, n, xs, nx, out);
  if (m.format == FTMOE_FMT_FP8_B128) return dot_bf16_f<FTMOE_FMT_FP8_B128>(m, n, xs, nx, out);
  dot_bf16_f<FTMOE_FMT_MXFP4>(m, n, xs, nx, out);
}

using dot_fn = void (*)(const Mat&, int, const float* const*, int, float*);

float silu(float g) { return g / (1.0f + std::exp(-g)); }
float gelu(float g) { return 0.5f * g * (1.0f + std::erf(g * 0.70710678118654752f)); }
float gelu_tanh(float g) {
  return 0.5f * g * (1.0f + std::tanh(0.7978845608028654f * (g + 0.044715f * g * g * g)));
}

class Executor;

struct Job {
  Executor* ex;
  int slot = -1;           // flag handshake: this record's flag slot (fixed for its life)
  bool flagged = false;    // the current use rides the flag handshake
  bool armed = false;      // flag handshake: the coordinator watches the ready flag
  bool started = false;    // flag handshake: handed to the driver, not yet done
  ftmoe_bank bank;  // host pointers
  const bf16* x;    // [M, H]
  const float* w;   // [M, k]
  const int32_t* ids;  // [M, k] bank rows; < 0 or >= num_rows skipped
  int M, k, activation;
  bf16* y;          // [M, H]
  bool permanent = false;
  bool done = true;
  bool failed = false;     // poisoned by the watchdog (or refused by an unhealthy executor)
  // poisoned while the driver held it: never recycled, and the pool stops
  // taking its work units and writes nothing more to its y
  std::atomic<bool> abandoned{false};
};

class Executor {
 public:
  explicit Executor(int threads) : nthreads_(threads < 1 ? 1 : threads) {
    dot_ = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") ? dot_avx512 : dot_scalar;
    const char* want = std::getenv("FTMOE_CPU_DOT");  // "fp32" keeps the fp32 dots (measurement)
    bf16_dot_ = dot_ == dot_avx512 && __builtin_cpu_supports("avx512bf16") && !(want && !std::strcmp(want, "fp32"));
    const char* wd = std::getenv("FTMOE_CPU_WATCHDOG_S");  // seconds without progress; 0 turns it off
    watchdog_ms_ = wd ? static_cast<int>(std::atof(wd) * 1000.0) : 10000;
    for (int t = 1; t < nthreads_; ++t) workers_.emplace_back([this] { worker(); });  // the driver is the other one
    driver_ = std::thread([this] { drive(); });
    pin_workers();
  }
  ~Executor() {
    {
      std::lock_guard<std::mutex> g(m_);
      hold_ = false;
    }
    cv_job_.notify_all();
    {
      // queued and running jobs finish first (a worker leaving mid-pass would
      // leave the driver waiting for it); after the watchdog fired the queue
      // was failed and only a running job is waited for
      std::unique_lock<std::mutex> g(m_);
      cv_done_.wait(g, [this] { return queue_.empty() && !busy_; });
      stop_ = true;
    }
    cv_job_.notify_all();
    cv_work_.notify_all();
    driver_.join();
    for (auto& t : workers_) t.join();
    if (coord_.joinable()) coord_.join();
    if (flags_) {
      // release any wait still enqueued on a stream (callers synchronise first)
      for (int s = 0; s < kFlagSlots; ++s) flag_store(done_flag(s), 1);
      (void)hipHostFree(flags_);
    }
    for (Job* j : jobs_) delete j;
  }

  // ---- flag handshake ------------------------------------------------------
  static constexpr int kFlagSlots = 256;
  // Turns the flag handshake on after a functional probe of stream memory
  // operations on a private stream of the current device (write seen by the
  // host, wait on a host write, and the same under graph capture); returns 0,
  // or FTMOE_ERR_UNSUPPORTED with the host-function handshake kept.
  int enable_flags() {
    std::lock_guard<std::mutex> g(flag_mu_);
    if (flags_) return 0;
    int dev = 0, can = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&can, hipDeviceAttributeCanUseStreamWaitValue, dev) != hipSuccess || !can)
      return FTMOE_ERR_UNSUPPORTED;
    void* host = nullptr;
    const size_t bytes = (2 * kFlagSlots + 16) * sizeof(uint64_t);
    if (hipHostMalloc(&host, bytes, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess)
      return FTMOE_ERR_UNSUPPORTED;
    std::memset(host, 0, bytes);
    void* devp = nullptr;
    if (hipHostGetDevicePointer(&devp, host, 0) != hipSuccess || !devp) {
      (void)hipHostFree(host);
      return FTMOE_ERR_UNSUPPORTED;
    }
    flags_ = static_cast<uint64_t*>(host);
    dflags_ = static_cast<uint64_t*>(devp);
    if (!probe_flags()) {
      // a probe stream that may still wait is left as it is (never reused)
      flags_ = nullptr;
      dflags_ = nullptr;
      if (!probe_hung_) (void)hipHostFree(host);
      return FTMOE_ERR_UNSUPPORTED;
    }
    slot_job_.assign(kFlagSlots, nullptr);
    coord_ = std::thread([this] { coordinate(); });
    return 0;
  }
  bool flags_on() const { return flags_ != nullptr && use_flags_; }
  void use_flags(bool on) { use_flags_ = on; }
  bool flags_capturable() const { return flags_capturable_; }
  // Binds a flag slot to the record (kept for its life); false when none is left.
  bool bind_slot(Job* j) {
    std::lock_guard<std::mutex> g(m_);
    if (j->slot >= 0) return true;
    for (int s = 0; s < kFlagSlots; ++s)
      if (!slot_job_[s]) {
        slot_job_[s] = j;
        j->slot = s;
        nslots_.store(std::max(nslots_.load(), s + 1));
        return true;
      }
    return false;
  }
  // a submit that failed to enqueue: the record goes back unused
  void disarm(Job* j) {
    std::lock_guard<std::mutex> g(m_);
    j->armed = false;
    j->flagged = false;
    if (!j->permanent) free_.push_back(j);
  }
  // submit side: the record waits for its ready flag (the coordinator polls it)
  void arm(Job* j) {
    std::lock_guard<std::mutex> g(m_);
    j->flagged = true;
    j->done = false;
    j->failed = false;
    j->armed = true;
  }
  uint64_t* ready_dev(const Job* j) const { return dflags_ + j->slot; }
  uint64_t* done_dev(const Job* j) const { return dflags_ + kFlagSlots + j->slot; }
  // Jobs captured into graphs: their records are replayed by the graphs, so
  // the executor must outlive them.
  int captured_jobs() {
    std::lock_guard<std::mutex> g(m_);
    return captured_;
  }
  bool healthy() const { return !unhealthy_.load(); }
  // The watchdog abandoned a job that the driver is still computing (a wedged
  // pool): the threads cannot be joined, so the executor must not be freed.
  bool wedged() {
    std::lock_guard<std::mutex> g(m_);
    return unhealthy_.load() && busy_;
  }
  void set_watchdog_ms(int ms) { watchdog_ms_ = ms; }
  // Maintenance and tests of the watchdog: mode 1 holds the driver before its
  // next job; mode 2 lets the driver take its next job and stall inside it,
  // before its first work unit, as a wedged pool would (until mode 0).
  void hold(int mode) {
    {
      std::lock_guard<std::mutex> g(m_);
      hold_ = mode == 1;
      stall_.store(mode == 2);
    }
    cv_job_.notify_all();
  }
  // The driver and the workers one per CPU of the process's affinity mask, on
  // the last CPUs of the mask (the first ones stay free for the threads that
  // enqueue GPU work and run the stream's host functions), while there are at
  // least as many CPUs as threads (the reference pins its pool to physical
  // cores, moe/cpu_executor.py:91-140); FTMOE_CPU_PIN=0 leaves the scheduler
  // free.
  void pin_workers() {
    const char* pin = std::getenv("FTMOE_CPU_PIN");
    if (pin && !std::strcmp(pin, "0")) return;
    cpu_set_t allowed;
    if (sched_getaffinity(0, sizeof(allowed), &allowed) != 0 || CPU_COUNT(&allowed) < nthreads_) return;
    int t = 0, skip = CPU_COUNT(&allowed) - nthreads_;
    for (int c = 0; c < CPU_SETSIZE && t < nthreads_; ++c) {
      if (!CPU_ISSET(c, &allowed) || skip-- > 0) continue;
      cpu_set_t one;
      CPU_ZERO(&one);
      CPU_SET(c, &one);
      std::thread& th = t == 0 ? driver_ : workers_[t - 1];
      pthread_setaffinity_np(th.native_handle(), sizeof(one), &one);
      ++t;
    }
  }
  const char* isa() const { return bf16_dot_ ? "avx512bf16" : dot_ == dot_avx512 ? "avx512f" : "scalar"; }

  Job* new_job(bool permanent) {
    std::lock_guard<std::mutex> g(m_);
    Job* j = nullptr;
    if (!permanent && !free_.empty()) {
      j = free_.back();
      free_.pop_back();
    } else {
      j = new Job();
      jobs_.push_back(j);
    }
    j->ex = this;
    j->flagged = false;
    j->armed = false;
    j->started = false;
    j->permanent = permanent;
    if (permanent) ++captured_;
    return j;
  }
  // host node: queue the job for the driver (an unhealthy executor fails it at once)
  void start(Job* j) {
    {
      std::lock_guard<std::mutex> g(m_);
      start_locked(j);
    }
    cv_job_.notify_all();
    cv_done_.notify_all();
  }
  void start_locked(Job* j) {
    if (unhealthy_.load()) {
      j->done = true;
      j->failed = true;
      if (j->flagged) flag_store(done_flag(j->slot), 1);
    } else {
      j->done = false;
      j->failed = false;
      j->started = j->flagged;
      queue_.push_back(j);
    }
  }
  // a job record that was never started goes back to the free list
  void discard(Job* j) {
    std::lock_guard<std::mutex> g(m_);
    if (!j->permanent) free_.push_back(j);
  }
  // host node: block until the job is done, or until the watchdog finds the
  // driver and workers without progress for watchdog_ms (the reference's
  // flag watchdog, moe/cpu_executor.py:602-656: a dead or wedged coordinator
  // must not block the stream forever); recycle the record unless a graph
  // holds it.  Returns false for a failed job.
  bool finish(Job* j) {
    std::unique_lock<std::mutex> g(m_);
    if (watchdog_ms_ <= 0) {
      cv_done_.wait(g, [j] { return j->done; });
    } else {
      uint64_t seen = progress_.load(std::memory_order_relaxed);
      auto since = std::chrono::steady_clock::now();
      while (!cv_done_.wait_for(g, std::chrono::milliseconds(20), [j] { return j->done; })) {
        const uint64_t p = progress_.load(std::memory_order_relaxed);
        const auto now = std::chrono::steady_clock::now();
        if (p != seen) {
          seen = p;
          since = now;
        } else if (now - since >= std::chrono::milliseconds(watchdog_ms_)) {
          poison(j);
          break;
        }
      }
    }
    const bool ok = !j->failed;
    if (!j->permanent && !j->abandoned) free_.push_back(j);
    return ok;
  }

 private:
  // One pass over `units`: the driver and every worker take units from an
  // atomic counter; the driver then spins until each worker has finished.
  // Workers spin on the pass generation for a while before sleeping, so the
  // passes of a job follow one another without wake-ups (the reference's
  // pool uses a spin barrier between its passes, cpu_moe_ext.cpp:1833-1857).
  void parallel(int units, const std::function<void(int)>& fn) {
    fn_ = &fn;
    units_ = units;
    next_.store(0, std::memory_order_relaxed);
    left_.store(static_cast<int>(workers_.size()), std::memory_order_relaxed);
    {
      std::lock_guard<std::mutex> g(m_);
      gen_.fetch_add(1, std::memory_order_release);  // publishes fn_, units_, the counters
    }
    cv_work_.notify_all();
    for (int u = next_.fetch_add(1); u < units; u = next_.fetch_add(1)) {
      fn(u);
      progress_.fetch_add(1, std::memory_order_relaxed);
    }
    while (left_.load(std::memory_order_acquire) != 0) _mm_pause();
    fn_ = nullptr;
  }
  // The watchdog fired on j (m_ held): the executor is unhealthy for good, j
  // and every queued job fail now so their waiters return; a job the driver
  // is computing is abandoned (its record is never reused).
  void poison(Job* j) {
    unhealthy_.store(true);
    const auto it = std::find(queue_.begin(), queue_.end(), j);
    if (it != queue_.end()) queue_.erase(it);
    else j->abandoned = true;
    j->failed = true;
    j->done = true;
    j->started = false;
    if (j->flagged) flag_store(done_flag(j->slot), 1);  // the stream's wait must end
    for (Job* q : queue_) {
      q->failed = true;
      q->done = true;
      q->started = false;
      if (q->flagged) flag_store(done_flag(q->slot), 1);
    }
    queue_.clear();
    cv_done_.notify_all();
  }

  // Bounded wait for a stream's queued work: true when it drained within ms.
  static bool drained(hipStream_t s, int ms) {
    const auto t0 = std::chrono::steady_clock::now();
    for (;;) {
      const hipError_t e = hipStreamQuery(s);
      if (e == hipSuccess) return true;
      if (e != hipErrorNotReady) return false;
      if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(ms)) return false;
      std::this_thread::sleep_for(std::chrono::microseconds(200));
    }
  }
  // Polls a host flag for a value (true when seen within ms).
  static bool seen(const uint64_t* p, uint64_t v, int ms) {
    const auto t0 = std::chrono::steady_clock::now();
    while (flag_load(p) != v) {
      if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(ms)) return false;
      std::this_thread::sleep_for(std::chrono::microseconds(100));
    }
    return true;
  }
  // The functional probe of the flag handshake on a private stream: a stream
  // write reaches the host; a stream wait holds the stream until the host
  // writes the value (every wait is released from the host, so none can stay
  // blocked); and the same write / wait / reset sequence captured in a graph.
  bool probe_flags() {
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return false;
    uint64_t* hp = flags_ + 2 * kFlagSlots;
    uint64_t* dp = dflags_ + 2 * kFlagSlots;
    // a device-to-host copy enqueued before the write has landed when the
    // host sees the flag (the CPU share's inputs travel that way)
    void* dword = nullptr;
    const uint64_t val = 29;
    bool ok = hipMalloc(&dword, sizeof(uint64_t)) == hipSuccess &&
              hipMemcpy(dword, &val, sizeof(val), hipMemcpyHostToDevice) == hipSuccess &&
              hipMemcpyAsync(hp + 8, dword, sizeof(uint64_t), hipMemcpyDeviceToHost, s) == hipSuccess &&
              hipStreamWriteValue64(s, dp, 5, 0) == hipSuccess && seen(hp, 5, 2000) && flag_load(hp + 8) == val &&
              drained(s, 2000);
    if (dword) (void)hipFree(dword);
    if (ok) {
      const bool q = hipStreamWaitValue64(s, dp + 1, 7, hipStreamWaitValueEq, ~0ull) == hipSuccess &&
                     hipStreamWriteValue64(s, dp + 2, 9, 0) == hipSuccess;
      std::this_thread::sleep_for(std::chrono::milliseconds(2));
      const bool held = flag_load(hp + 2) == 0;
      flag_store(hp + 1, 7);  // releases the wait
      if (!drained(s, 2000)) {
        probe_hung_ = true;  // the stream is left waiting: never destroyed or reused
        return false;
      }
      ok = q && held && flag_load(hp + 2) == 9;
    }
    if (ok) flags_capturable_ = probe_capture(s, hp + 3, dp + 3);
    if (!probe_hung_) (void)hipStreamDestroy(s);
    return ok;
  }
  // The captured sequence also copies a device word to the host before the
  // ready write (as the CPU share's inputs are copied out), which the host must
  // see when it sees the flag, and a host word to the device and back after
  // the wait (as the CPU share's result is copied back), which must see the
  // host's write made before it released the wait.
  bool probe_capture(hipStream_t s, uint64_t* hp, uint64_t* dp) {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    void* dword = nullptr;
    if (hipMalloc(&dword, 2 * sizeof(uint64_t)) != hipSuccess) return false;
    const uint64_t init[2] = {0, 23};
    if (hipMemcpy(dword, init, sizeof(init), hipMemcpyHostToDevice) != hipSuccess ||
        hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) {
      (void)hipFree(dword);
      return false;
    }
    const bool q = hipMemcpyAsync(hp + 5, static_cast<uint64_t*>(dword) + 1, sizeof(uint64_t), hipMemcpyDeviceToHost,
                                  s) == hipSuccess &&
                   hipStreamWriteValue64(s, dp, 11, 0) == hipSuccess &&
                   hipStreamWaitValue64(s, dp + 1, 13, hipStreamWaitValueEq, ~0ull) == hipSuccess &&
                   hipStreamWriteValue64(s, dp + 1, 0, 0) == hipSuccess &&
                   hipStreamWriteValue64(s, dp + 2, 17, 0) == hipSuccess &&
                   hipMemcpyAsync(dword, hp + 3, sizeof(uint64_t), hipMemcpyHostToDevice, s) == hipSuccess &&
                   hipMemcpyAsync(hp + 4, dword, sizeof(uint64_t), hipMemcpyDeviceToHost, s) == hipSuccess;
    const bool ended = hipStreamEndCapture(s, &graph) == hipSuccess && graph;
    bool ok = q && ended && hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess;
    if (ok && hipGraphLaunch(exec, s) == hipSuccess) {
      ok = seen(hp, 11, 2000) && flag_load(hp + 5) == 23;  // the copy before the flag has landed
      std::this_thread::sleep_for(std::chrono::milliseconds(2));
      ok = ok && flag_load(hp + 2) == 0;  // the wait holds the replay
      flag_store(hp + 3, 19);  // the host's data, written before the release
      flag_store(hp + 1, 13);  // releases the wait whatever happened
      if (!drained(s, 2000)) {
        probe_hung_ = true;
        ok = false;
      } else {
        // the writes and the copies after the wait ran after it
        ok = ok && flag_load(hp + 1) == 0 && flag_load(hp + 2) == 17 && flag_load(hp + 4) == 19;
      }
    } else {
      ok = false;
    }
    if (exec && !probe_hung_) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (!probe_hung_) (void)hipFree(dword);
    return ok;
  }
  // The coordinator of the flag handshake: hands each armed job whose ready
  // flag the stream raised to the driver, returns eager records to the free
  // list once the stream has consumed their done flag, and runs the watchdog
  // of the flag jobs (their waits are stream waits, not host functions).
  // Busy-polls only while a submitted job waits for its ready flag; while the
  // pool computes, or nothing is submitted, it sleeps between sweeps, so that
  // it does not take a CPU from the pool.
  void coordinate() {
    int idle = 0;
    uint64_t seen_progress = progress_.load(std::memory_order_relaxed);
    auto since = std::chrono::steady_clock::now();
    while (!stop_.load(std::memory_order_relaxed)) {
      bool any = false, waiting = false, awaiting_ready = false;
      {
        std::lock_guard<std::mutex> g(m_);
        const int n = nslots_.load();
        for (int s = 0; s < n; ++s) {
          Job* j = slot_job_[s];
          if (!j || !j->armed) continue;
          if (flag_load(ready_flag(s)) == 1) {
            flag_store(ready_flag(s), 0);
            start_locked(j);
            any = true;
          } else if (!j->permanent && j->done && !j->started && flag_load(done_flag(s)) == 0) {
            j->armed = false;  // the stream consumed the done flag: the record is free again
            if (!j->abandoned) free_.push_back(j);
          }
          waiting |= j->started && !j->done;
          awaiting_ready |= !j->permanent && j->armed && !j->started && !j->done;
        }
        if (waiting && watchdog_ms_ > 0) {
          const uint64_t p = progress_.load(std::memory_order_relaxed);
          const auto now = std::chrono::steady_clock::now();
          if (p != seen_progress) {
            seen_progress = p;
            since = now;
          } else if (now - since >= std::chrono::milliseconds(watchdog_ms_)) {
            for (int s = 0; s < n; ++s) {
              Job* j = slot_job_[s];
              if (j && j->armed && j->started && !j->done) poison(j);
            }
          }
        } else {
          seen_progress = progress_.load(std::memory_order_relaxed);
          since = std::chrono::steady_clock::now();
        }
      }
      if (any) {
        cv_job_.notify_all();
        cv_done_.notify_all();
        idle = 0;
      } else if (!awaiting_ready || ++idle > (1 << 16)) {
        std::this_thread::sleep_for(std::chrono::microseconds(20));
      } else {
        _mm_pause();
      }
    }
  }
  void worker() {
    constexpr int kSpin = 4096;  // pauses before sleeping (~0.1 ms)
    uint64_t seen = 0;
    for (;;) {
      uint64_t g = gen_.load(std::memory_order_acquire);
      for (int spin = 0; g == seen && spin < kSpin && !stop_.load(std::memory_order_relaxed); ++spin) {
        _mm_pause();
        g = gen_.load(std::memory_order_acquire);
      }
      if (g == seen) {
        std::unique_lock<std::mutex> lk(m_);
        cv_work_.wait(lk, [&] { return stop_.load() || gen_.load(std::memory_order_acquire) != seen; });
        if (stop_.load()) return;
        g = gen_.load(std::memory_order_acquire);
      }
      seen = g;
      const std::function<void(int)>* fn = fn_;
      const int units = units_;
      for (int u = next_.fetch_add(1); u < units; u = next_.fetch_add(1)) {
        (*fn)(u);
        progress_.fetch_add(1, std::memory_order_relaxed);
      }
      left_.fetch_sub(1, std::memory_order_acq_rel);
    }
  }
  void drive() {
    for (;;) {
      Job* j;
      {
        std::unique_lock<std::mutex> g(m_);
        cv_job_.wait(g, [this] { return stop_ || (!hold_ && !queue_.empty()); });
        if (stop_) return;
        j = queue_.front();
        queue_.pop_front();
        busy_ = true;
      }
      compute(*j);
      progress_.fetch_add(1, std::memory_order_relaxed);
      {
        std::lock_guard<std::mutex> g(m_);
        const bool already = j->done;  // poisoned while computed: its flag was raised then
        j->done = true;
        j->started = false;
        if (j->flagged && !already) flag_store(done_flag(j->slot), 1);
        busy_ = false;
      }
      cv_done_.notify_all();
    }
  }
  void compute(const Job& j) {
    if (bf16_dot_) compute_t<true>(j);
    else compute_t<false>(j);
  }

  // BF: the activation vectors are bf16 (the input rows and a bf16 act) for
  // the bf16 dot; otherwise fp32 copies for the fp32 dots
  template <bool BF>
  void compute_t(const Job& j) {
    using X = std::conditional_t<BF, bf16, float>;
    const int H = j.bank.hidden, I = j.bank.inter, R = j.M * j.k;
    const Mat gu{j.bank.format, H, static_cast<const uint8_t*>(j.bank.gate_up), j.bank.gate_up_scale};
    const Mat dn{j.bank.format, I, static_cast<const uint8_t*>(j.bank.down), j.bank.down_scale};
    const size_t gu_rows = static_cast<size_t>(2) * I, dn_rows = H;
    const auto rowmat = [&](const Mat& m, size_t rows, int e) {
      Mat r = m;
      const size_t row_bytes = m.format == FTMOE_FMT_MXFP4 ? m.K / 2 : m.format == FTMOE_FMT_BF16 ? m.K * 2 : m.K;
      r.w = m.w + static_cast<size_t>(e) * rows * row_bytes;
      if (m.format == FTMOE_FMT_FP8_B128)
        r.s = static_cast<const float*>(m.s) + static_cast<size_t>(e) * (rows / 128) * (m.K / 128);
      else if (m.format == FTMOE_FMT_MXFP4)
        r.s = static_cast<const uint8_t*>(m.s) + static_cast<size_t>(e) * rows * (m.K / 32);
      return r;
    };
    const auto valid = [&](int r) { return j.ids[r] >= 0 && j.ids[r] < j.bank.num_rows; };
    // routes grouped by expert (ascending expert, then route), split into
    // groups of at most kMaxVec routes
    order_.clear();
    for (int r = 0; r < R; ++r)
      if (valid(r)) order_.push_back(r);
    std::stable_sort(order_.begin(), order_.end(), [&](int a, int b) { return j.ids[a] < j.ids[b]; });
    group_.clear();
    for (size_t i = 0; i < order_.size(); ++i)
      if (i == 0 || j.ids[order_[i]] != j.ids[order_[i - 1]] || i - group_.back() == kMaxVec)
        group_.push_back(static_cast<int>(i));
    const int G = static_cast<int>(group_.size());
    group_.push_back(static_cast<int>(order_.size()));
    if constexpr (!BF) {
      xf_.resize(static_cast<size_t>(j.M) * H);
      for (size_t i = 0; i < xf_.size(); ++i) xf_[i] = b2f(j.x[i]);
      act_.resize(static_cast<size_t>(R) * I);
    } else {
      act16_.resize(static_cast<size_t>(R) * I);
    }
    while (stall_.load(std::memory_order_relaxed)) std::this_thread::sleep_for(std::chrono::milliseconds(1));
    // an abandoned job's remaining work units return at once, and pass 3, the
    // only writer of the caller's y, writes no row once the job is abandoned
    const auto dropped = [&] { return j.abandoned.load(std::memory_order_relaxed); };
    const X* const xin = BF ? reinterpret_cast<const X*>(j.x) : reinterpret_cast<const X*>(xf_.data());
    X* const act = BF ? reinterpret_cast<X*>(act16_.data()) : reinterpret_cast<X*>(act_.data());
    const auto dot = [&](const Mat& m, int n, const X* const* xs, int nv, float* o) {
      if constexpr (BF) dot_bf16(m, n, xs, nv, o);
      else dot_(m, n, xs, nv, o);
    };
    dout_.resize(static_cast<size_t>(R) * H);
    constexpr int kTile = 32;
    // pass 1: gate and up rows of (group, 32 rows of I) -> bf16 act
    const int tiles1 = I / kTile;
    const float lim = j.bank.swiglu_limit;
    parallel(G * tiles1, [&](int u) {
      if (dropped()) return;
      const int g = u / tiles1, i0 = (u % tiles1) * kTile;
      const int* rs = order_.data() + group_[g];
      const int nv = group_[g + 1] - group_[g];
      const Mat m = rowmat(gu, gu_rows, j.ids[rs[0]]);
      const X* xs[kMaxVec];
      for (int v = 0; v < nv; ++v) xs[v] = xin + static_cast<size_t>(rs[v] / j.k) * H;
      float gv[kMaxVec], uv[kMaxVec];
      for (int i = i0; i < i0 + kTile; ++i) {
        dot(m, i, xs, nv, gv);
        dot(m, I + i, xs, nv, uv);
        for (int v = 0; v < nv; ++v) {
          float g = rb(gv[v]), up = rb(uv[v]);
          if (lim > 0.f) {  // clamped SwiGLU (cpu_moe_ext.cpp:1769-1781)
            g = std::min(g, lim);
            up = std::min(std::max(up, -lim), lim);
          }
          const float a = j.activation == FTMOE_ACT_SILU ? silu(g) : j.activation == FTMOE_ACT_GELU ? gelu(g)
                                                                                                  : gelu_tanh(g);
          if constexpr (BF) act[static_cast<size_t>(rs[v]) * I + i] = f2b(a * up);
          else act[static_cast<size_t>(rs[v]) * I + i] = rb(a * up);
        }
      }
    });
    // pass 2: down rows of (group, 32 rows of H) -> bf16(down * router weight) per route
    const int tiles2 = H / kTile;
    parallel(G * tiles2, [&](int u) {
      if (dropped()) return;
      const int g = u / tiles2, h0 = (u % tiles2) * kTile;
      const int* rs = order_.data() + group_[g];
      const int nv = group_[g + 1] - group_[g];
      const Mat m = rowmat(dn, dn_rows, j.ids[rs[0]]);
      const X* xs[kMaxVec];
      for (int v = 0; v < nv; ++v) xs[v] = act + static_cast<size_t>(rs[v]) * I;
      float dv[kMaxVec];
      for (int h = h0; h < h0 + kTile; ++h) {
        dot(m, h, xs, nv, dv);
        for (int v = 0; v < nv; ++v) dout_[static_cast<size_t>(rs[v]) * H + h] = rb(dv[v] * j.w[rs[v]]);
      }
    });
    // pass 3: each token's routes summed in route order
    parallel(j.M, [&](int t) {
      if (dropped()) return;
      bf16* y = j.y + static_cast<size_t>(t) * H;
      for (int h = 0; h < H; ++h) {
        float s = 0.f;
        for (int q = 0; q < j.k; ++q)
          if (valid(t * j.k + q)) s += dout_[static_cast<size_t>(t * j.k + q) * H + h];
        y[h] = f2b(s);
      }
    });
  }

  int nthreads_;
  dot_fn dot_;
  std::vector<std::thread> workers_;
  std::thread driver_;
  std::mutex m_;
  std::condition_variable cv_job_, cv_done_, cv_work_;
  std::deque<Job*> queue_;
  std::vector<Job*> jobs_, free_;
  const std::function<void(int)>* fn_ = nullptr;
  int units_ = 0;
  std::atomic<int> left_{0};
  std::atomic<uint64_t> gen_{0};
  std::atomic<int> next_{0};
  std::atomic<bool> stop_{false};
  bool busy_ = false;  // the driver is computing a job
  bool hold_ = false;  // the driver takes no new job
  std::atomic<bool> stall_{false};  // the driver stalls inside its job (tests of a wedged pool)
  int captured_ = 0;   // permanent (graph-captured) job records
  // flag handshake: pinned host flags (ready [kFlagSlots], done [kFlagSlots],
  // probe words) and their device addresses; the record bound to each slot
  std::mutex flag_mu_;
  uint64_t* flags_ = nullptr;
  uint64_t* dflags_ = nullptr;
  bool flags_capturable_ = false;
  bool probe_hung_ = false;
  bool use_flags_ = false;
  std::vector<Job*> slot_job_;
  std::atomic<int> nslots_{0};
  std::thread coord_;
  uint64_t* ready_flag(int s) { return flags_ + s; }
  uint64_t* done_flag(int s) { return flags_ + kFlagSlots + s; }
  static void flag_store(uint64_t* p, uint64_t v) { __atomic_store_n(p, v, __ATOMIC_RELEASE); }
  static uint64_t flag_load(const uint64_t* p) { return __atomic_load_n(p, __ATOMIC_ACQUIRE); }
  int watchdog_ms_ = 10000;
  std::atomic<uint64_t> progress_{0};  // work units and jobs completed
  std::atomic<bool> unhealthy_{false};
  std::vector<float> xf_, act_, dout_;
  std::vector<bf16> act16_;
  bool bf16_dot_ = false;
  std::vector<int> order_, group_;
};

void host_start(void* p) {
  Job* j = static_cast<Job*>(p);
  j->ex->start(j);
}
void host_finish(void* p) {
  Job* j = static_cast<Job*>(p);
  j->ex->finish(j);
}

int check_job(const ftmoe_bank* b, const void* x, const float* w, const int32_t* ids, int M, int k, int act,
              const void* y) {
  if (!b || !x || !w || !ids || !y || !b->gate_up || !b->down)
    return ftmoe::report_error(FTMOE_ERR_INVALID, "cpu_experts: NULL pointer");
  if (b->format < FTMOE_FMT_BF16 || b->format > FTMOE_FMT_MXFP4 || b->hidden <= 0 || b->inter <= 0 ||
      b->hidden % 128 || b->inter % 128 || b->num_rows <= 0 ||
      (b->format != FTMOE_FMT_BF16 && (!b->gate_up_scale || !b->down_scale)))
    return ftmoe::report_error(FTMOE_ERR_UNSUPPORTED, "cpu_experts: bank format/shape");
  if (M <= 0 || k <= 0 || act < FTMOE_ACT_SILU || act > FTMOE_ACT_GELU_TANH)
    return ftmoe::report_error(FTMOE_ERR_UNSUPPORTED, "cpu_experts: M/k/activation");
  if (!std::isfinite(b->swiglu_limit) || b->swiglu_limit < 0.f)
    return ftmoe::report_error(FTMOE_ERR_INVALID, "cpu_experts: swiglu_limit (finite, >= 0)");
  if (b->swiglu_limit > 0.f && act != FTMOE_ACT_SILU)
    return ftmoe::report_error(FTMOE_ERR_UNSUPPORTED, "cpu_experts: swiglu_limit > 0 needs the silu activation");
  return FTMOE_OK;
}

void fill(Job* j, const ftmoe_bank* b, const void* x, const float* w, const int32_t* ids, int M, int k, int act,
          void* y) {
  j->bank = *b;
  j->x = static_cast<const bf16*>(x);
  j->w = w;
  j->ids = ids;
  j->M = M;
  j->k = k;
  j->activation = act;
  j->y = static_cast<bf16*>(y);
}

}  // namespace ftmoe_cpu

extern "C" {

ftmoe_cpu_executor* ftmoe_cpu_executor_create(int threads) {
  if (threads <= 0) {  // the CPUs this process may run on, not the machine's count
    cpu_set_t set;
    threads = sched_getaffinity(0, sizeof(set), &set) == 0 ? CPU_COUNT(&set)
                                                             : static_cast<int>(std::thread::hardware_concurrency());
  }
  return reinterpret_cast<ftmoe_cpu_executor*>(new ftmoe_cpu::Executor(threads));
}

int ftmoe_cpu_executor_destroy(ftmoe_cpu_executor* ex, int graphs_released) {
  if (!ex) return FTMOE_OK;
  auto* e = reinterpret_cast<ftmoe_cpu::Executor*>(ex);
  if (!graphs_released && e->captured_jobs() > 0) {
    char msg[160];
    std::snprintf(msg, sizeof(msg), "cpu_executor_destroy: %d job(s) captured into graphs may still replay",
                  e->captured_jobs());
    return ftmoe::report_error(FTMOE_ERR_BUSY, msg);
  }
  if (e->wedged())
    return ftmoe::report_error(FTMOE_ERR_BUSY, "cpu_executor_destroy: the watchdog abandoned a job the pool is still "
                               "computing; its threads cannot be joined, so the executor is kept");
  delete e;
  return FTMOE_OK;
}

int ftmoe_cpu_executor_healthy(ftmoe_cpu_executor* ex) {
  if (!ex) return FTMOE_ERR_INVALID;
  return reinterpret_cast<ftmoe_cpu::Executor*>(ex)->healthy() ? FTMOE_OK : FTMOE_ERR_TIMEOUT;
}

void ftmoe_cpu_executor_set_watchdog(ftmoe_cpu_executor* ex, int ms) {
  if (ex) reinterpret_cast<ftmoe_cpu::Executor*>(ex)->set_watchdog_ms(ms);
}

int ftmoe_cpu_executor_set_handshake(ftmoe_cpu_executor* ex, int mode) {
  if (!ex || mode < 0 || mode > 1) return ftmoe::report_error(FTMOE_ERR_INVALID, "cpu_executor_set_handshake: mode");
  auto* e = reinterpret_cast<ftmoe_cpu::Executor*>(ex);
  if (mode == 0) {
    e->use_flags(false);
    return FTMOE_OK;
  }
  const int rc = e->enable_flags();
  if (rc) return ftmoe::report_error(rc, "cpu_executor_set_handshake: stream memory operations failed their probe "
                                         "on this device; the host-function handshake stays");
  e->use_flags(true);
  return FTMOE_OK;
}

int ftmoe_cpu_executor_handshake(ftmoe_cpu_executor* ex) {
  if (!ex) return -1;
  auto* e = reinterpret_cast<ftmoe_cpu::Executor*>(ex);
  return e->flags_on() ? (e->flags_capturable() ? 2 : 1) : 0;
}

void ftmoe_cpu_executor_hold(ftmoe_cpu_executor* ex, int hold) {
  if (ex) reinterpret_cast<ftmoe_cpu::Executor*>(ex)->hold(hold);
}

const char* ftmoe_cpu_executor_isa(ftmoe_cpu_executor* ex) {
  return ex ? reinterpret_cast<ftmoe_cpu::Executor*>(ex)->isa() : "";
}

int ftmoe_cpu_experts(ftmoe_cpu_executor* ex, const ftmoe_bank* bank, const void* x, const float* w,
                      const int32_t* ids, int M, int k, int activation, void* y) {
  if (!ex) return ftmoe::report_error(FTMOE_ERR_INVALID, "cpu_experts: NULL executor");
  const int rc = ftmoe_cpu::check_job(bank, x, w, ids, M, k, activation, y);
  if (rc) return rc;
  auto* e = reinterpret_cast<ftmoe_cpu::Executor*>(ex);
  ftmoe_cpu::Job* j = e->new_job(false);
  ftmoe_cpu::fill(j, bank, x, w, ids, M, k, activation, y);
  e->start(j);
  if (!e->finish(j))
    return ftmoe::report_error(FTMOE_ERR_TIMEOUT, "cpu_experts: the executor's watchdog fired (no progress); "
                               "the executor is unhealthy");
  return FTMOE_OK;
}

int ftmoe_cpu_experts_submit(ftmoe_cpu_executor* ex, const ftmoe_bank* bank, const void* x, const float* w,
                             const int32_t* ids, int M, int k, int activation, void* y, ftmoe_stream_t stream,
                             void** job) {
  if (!ex || !job) return ftmoe::report_error(FTMOE_ERR_INVALID, "cpu_experts_submit: NULL executor or job");
  const int rc = ftmoe_cpu::check_job(bank, x, w, ids, M, k, activation, y);
  if (rc) return rc;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (stream && hipStreamIsCapturing(stream, &cs) != hipSuccess)
    return ftmoe::report_error(FTMOE_ERR_HIP, "cpu_experts_submit: stream query failed");
  auto* e = reinterpret_cast<ftmoe_cpu::Executor*>(ex);
  const bool capturing = cs != hipStreamCaptureStatusNone;
  // a job captured into a graph is replayed with the same record: never recycled
  ftmoe_cpu::Job* j = e->new_job(capturing);
  ftmoe_cpu::fill(j, bank, x, w, ids, M, k, activation, y);
  if (e->flags_on() && (!capturing || e->flags_capturable()) && e->bind_slot(j)) {
    // flag handshake: the stream raises the job's ready flag
    e->arm(j);
    if (hipStreamWriteValue64(stream, e->ready_dev(j), 1, 0) != hipSuccess) {
      e->disarm(j);
      return ftmoe::report_error(FTMOE_ERR_HIP, "cpu_experts_submit: hipStreamWriteValue64 failed");
    }
    *job = j;
    return FTMOE_OK;
  }
  if (hipLaunchHostFunc(stream, ftmoe_cpu::host_start, j) != hipSuccess) {
    e->discard(j);
    return ftmoe::report_error(FTMOE_ERR_HIP, "cpu_experts_submit: hipLaunchHostFunc failed");
  }
  *job = j;
  return FTMOE_OK;
}

int ftmoe_cpu_experts_wait(ftmoe_cpu_executor* ex, void* job, ftmoe_stream_t stream) {
  if (!ex || !job) return ftmoe::report_error(FTMOE_ERR_INVALID, "cpu_experts_wait: NULL executor or job");
  auto* j = static_cast<ftmoe_cpu::Job*>(job);
  if (j->flagged) {
    // flag handshake: wait for the job's done flag, then reset it for the next use
    auto* e = reinterpret_cast<ftmoe_cpu::Executor*>(ex);
    if (hipStreamWaitValue64(stream, e->done_dev(j), 1, hipStreamWaitValueEq, ~0ull) != hipSuccess ||
        hipStreamWriteValue64(stream, e->done_dev(j), 0, 0) != hipSuccess)
      return ftmoe::report_error(FTMOE_ERR_HIP, "cpu_experts_wait: stream memory operation failed");
    return FTMOE_OK;
  }
  if (hipLaunchHostFunc(stream, ftmoe_cpu::host_finish, job) != hipSuccess)
    return ftmoe::report_error(FTMOE_ERR_HIP, "cpu_experts_wait: hipLaunchHostFunc failed");
  return FTMOE_OK;
}

}  // extern "C"
