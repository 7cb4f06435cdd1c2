// Prefill (grouped GEMM) path: activation quantisation, the two grouped GEMMs
// with fused epilogues, on CDNA4 matrix cores.
//
// Formats
//   FMT_FP8   W8A8: activations e4m3 with one float32 scale per row per 128 K
//             (s = amax/448, reference per_token_group_quant_fp8,
//             kernel/triton/fp8_block_linear.py:38-82), weights e4m3 with float32
//             128x128 block scales.  One v_mfma_f32_16x16x128_f8f6f4 covers exactly
//             one 128-deep scale block, so each MFMA result is folded into the
//             accumulator with the product of both scales (reference
//             _prefill_fp8_moe_kernel: acc += dot(a, w) * a_s * w_s).
//   FMT_MXFP4 activations e4m3 with a power-of-two scale per row per 128 K (the
//             DSV4 act_quant round trip of routed_experts_fp4_prefill), weights e2m1
//             with e8m0 per 32 K: v_mfma_scale_f32_16x16x128_f8f6f4 applies both
//             scales in hardware and accumulates directly.
//   FMT_BF16  bf16 activations and weights, v_mfma_f32_16x16x32_bf16.
//
// The quantised formats (FP8, MXFP4) run prefill_qgemm_kernel, whose tiling,
// copies and schedule are described at its section below; the rest of this
// header describes the bf16 grouped GEMM (prefill_gemm_kernel).
//
// Tiling (bf16): a workgroup computes a 128 (weight rows) x 128 (routes) tile with 4 waves
// (2 x 2), each 64 x 64 = 4 x 4 MFMA blocks.  Weights are the MFMA A operand, so a
// lane's four accumulators are four consecutive output features of one route and
// stores are 8-byte vectors.  K advances 128 per step; global->LDS copies of the
// next step overlap the MFMAs of the current one (double-buffered LDS).
//
// Gate/up: the weight tile holds gate rows [n0, n0+64) and up rows [I+n0, I+n0+64);
// wave column wn owns gate and up rows n0+32wn..+32, so SwiGLU pairs registers.
//
// Schedule: workgroups are ordered expert-major -- for each expert, each N tile,
// all M blocks of that expert -- so the blocks sharing a weight tile run together
// and read it from HBM about once; the expert's activation rows stay hot in the
// memory-side cache across its N tiles.  Shared-expert blocks come last.
#include <algorithm>
#include <type_traits>

#include "kernels.h"
#include "quant.h"

namespace ftmoe {

constexpr int kPBM = 128;   // routes per tile
constexpr int kPBN = 128;   // weight rows per tile
constexpr int kPThreads = 256;

// ----------------------------------------------------------------------------
// Activation quantisation: one wave per row, 2 values per lane per 128-group
// (group_scale / quant_value of quant.h).
// ----------------------------------------------------------------------------
// Maximum over each 16-lane row of the wave (DPP inside the row), in every lane.
__device__ __forceinline__ float row16_max_f32(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x141>(v));  // row_half_mirror
  return fmaxf(v, dpp_f32<0x140>(v));  // row_mirror
}

// One wave per row.  Lane l of load i holds 8 values (16 bytes) at
// 8 * (64 i + l): the 16 lanes of a row of the wave cover one 128-value group,
// whose amax is a DPP reduction inside the row.  kAhead loads of the row are
// in flight together; x is read once (nontemporal).
template <int MODE>
__global__ void __launch_bounds__(256) act_quant_kernel(const uint16_t* __restrict__ x, int rows, int K,
                                                        uint8_t* __restrict__ q, void* __restrict__ scales) {
  const int lane = lane_id();
  const int row = blockIdx.x * 4 + threadIdx.x / kWave;
  if (row >= rows) return;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + static_cast<size_t>(row) * K);
  uint2* qr = reinterpret_cast<uint2*>(q + static_cast<size_t>(row) * K);
  const int ng = K / 128;
  const int nv = K / 8;                  // 16-byte pieces of the row
  const int nload = (nv + kWave - 1) / kWave;
  constexpr int kAhead = 8;
  for (int i0 = 0; i0 < nload; i0 += kAhead) {
    u32x4 v[kAhead];
#pragma unroll
    for (int u = 0; u < kAhead; ++u) {
      const int p = (i0 + u) * kWave + lane;
      v[u] = (i0 + u < nload && p < nv) ? __builtin_nontemporal_load(xr + p) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kAhead; ++u) {
      if (i0 + u >= nload) break;
      const int p = (i0 + u) * kWave + lane;
      const int gi = p / 16;  // the row's 16 lanes form group gi (uniform inside the row)
      float f[8];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        f[2 * w] = bf16_to_f32(static_cast<uint16_t>(v[u][w] & 0xffffu));
        f[2 * w + 1] = bf16_to_f32(static_cast<uint16_t>(v[u][w] >> 16));
      }
      float m = 0.f;
#pragma unroll
      for (int w = 0; w < 8; ++w) m = fmaxf(m, fabsf(f[w]));
      const float amax = row16_max_f32(m);
      if (p >= nv) continue;  // whole rows of lanes past the end (K not a multiple of 512)
      float mul;
      const float sc = group_scale<MODE>(amax, mul);
      uint32_t pk[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float q0 = quant_value<MODE>(f[4 * h], sc, mul), q1 = quant_value<MODE>(f[4 * h + 1], sc, mul);
        const float q2 = quant_value<MODE>(f[4 * h + 2], sc, mul), q3 = quant_value<MODE>(f[4 * h + 3], sc, mul);
        uint32_t w4 = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(q0, q1, 0, false));
        w4 = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(q2, q3, static_cast<int>(w4), true));
        pk[h] = w4;
      }
      qr[p] = uint2{pk[0], pk[1]};
      if ((lane & 15) == 0) {
        const size_t at = static_cast<size_t>(row) * ng + gi;
        if (MODE == 0) static_cast<float*>(scales)[at] = sc;
        else if (MODE == 1) static_cast<uint8_t*>(scales)[at] = static_cast<uint8_t>(sc);
        else static_cast<uint32_t*>(scales)[at] = static_cast<uint32_t>(sc);
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Grouped GEMM
// ----------------------------------------------------------------------------

template <int FMT>
struct TileCfg;
template <>
struct TileCfg<FMT_FP8> {
  static constexpr int kWRow = 128;  // bytes of a weight row per K step
  static constexpr int kXRow = 128;
};
template <>
struct TileCfg<FMT_MXFP4> {
  static constexpr int kWRow = 64;
  static constexpr int kXRow = 128;
};
template <>
struct TileCfg<FMT_BF16> {
  static constexpr int kWRow = 256;
  static constexpr int kXRow = 256;
};

template <int FMT>
struct Lds {
  static constexpr int kWStride = TileCfg<FMT>::kWRow + 16;
  static constexpr int kXStride = TileCfg<FMT>::kXRow + 16;
  static constexpr int kW = kPBN * kWStride;
  static constexpr int kX = kPBM * kXStride;
  static constexpr int kWS = FMT == FMT_MXFP4 ? kPBN * 4 : 0;  // e8m0 codes, 4 per row per step
  static constexpr int kXS = kPBM * 4;                          // float or e8m0 (one per row)
  static constexpr int kBuf = kW + kX + kWS + kXS;
  static constexpr int kTotal = 2 * kBuf;
};

// Maps a workgroup to (expert or shared, M block, N tile); returns false when idle.
__device__ __forceinline__ bool map_tile(const PrefillGemmArgs& a, int wg, bool& shared, int& expert, int& mblock,
                                         int& ntile) {
  // blocks of the real experts only; ids == num_experts (the sentinel bucket of
  // the align contract) take no part in the GEMMs
  const int routed_wgs = (a.cum[a.num_experts] / kPBM) * a.ntiles;
  if (wg < routed_wgs) {
    // expert owning this workgroup: largest e with cum[e]/BM * ntiles <= wg
    int lo = 0, hi = a.num_experts;  // cum[num_experts] region (sentinel bucket) never has work here
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if ((a.cum[mid] / kPBM) * a.ntiles <= wg) lo = mid; else hi = mid;
    }
    const int b0 = a.cum[lo] / kPBM;
    const int nb = a.cum[lo + 1] / kPBM - b0;
    const int local = wg - b0 * a.ntiles;
    shared = false;
    expert = lo;
    ntile = local / nb;
    mblock = b0 + local % nb;
    return true;
  }
  const int sh0 = a.max_blocks * a.ntiles;
  if (a.shared_blocks > 0 && wg >= sh0 && wg < sh0 + a.shared_blocks * a.ntiles) {
    const int local = wg - sh0;
    shared = true;
    expert = 0;
    ntile = local / a.shared_blocks;
    mblock = local % a.shared_blocks;
    return true;
  }
  return false;
}

template <int FMT, int GATE_UP>
__global__ void __launch_bounds__(kPThreads) prefill_gemm_kernel(PrefillGemmArgs a) {
  using L = Lds<FMT>;
  using C = TileCfg<FMT>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  __shared__ int s_row[kPBM];   // activation row of each tile column (-1: padding)
  __shared__ int s_route[kPBM]; // route (routed) or token (shared) of each column, -1: padding

  bool shared;
  int expert, mblock, ntile;
  if (!map_tile(a, blockIdx.x, shared, expert, mblock, ntile)) return;

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int wn = wave >> 1, wm = wave & 1;
  const int r16 = lane & 15, g = lane >> 4;

  if (tid < kPBM) {
    int row = -1, route = -1;
    if (shared) {
      const int t = mblock * kPBM + tid;
      if (t < a.M) {
        route = t;
        row = a.x_token_rows ? t : a.numel + t;
      }
    } else {
      const int rr = a.sorted[mblock * kPBM + tid];
      if (rr < a.numel) {
        route = rr;
        row = a.x_token_rows ? rr / a.k : rr;
      }
    }
    s_row[tid] = row;
    s_route[tid] = route;
  }
  __syncthreads();

  const BankView bank = shared ? a.ws : a.w;
  const int n0 = GATE_UP ? ntile * (kPBN / 2) : ntile * kPBN;
  const size_t wrow_bytes = FMT == FMT_BF16 ? static_cast<size_t>(a.K) * 2
                            : FMT == FMT_FP8 ? static_cast<size_t>(a.K) : static_cast<size_t>(a.K) / 2;
  const uint8_t* wexp = bank.w + static_cast<size_t>(expert) * a.N * wrow_bytes;
  const size_t xrow_bytes = FMT == FMT_BF16 ? static_cast<size_t>(a.K) * 2 : static_cast<size_t>(a.K);
  const int nkb = a.K / 128;

  auto wrow_of = [&](int r) -> int {  // weight row held in tile row r
    if (GATE_UP) return r < kPBN / 2 ? n0 + r : a.inter + n0 + (r - kPBN / 2);
    return n0 + r;
  };

  // ---- global -> register staging of one K step
  constexpr int kWChunks = kPBN * C::kWRow / 16;
  constexpr int kXChunks = kPBM * C::kXRow / 16;
  constexpr int kWPer = kWChunks / kPThreads;
  constexpr int kXPer = kXChunks / kPThreads;
  u32x4 wreg[kWPer], xreg[kXPer];
  uint32_t wsreg = 0;   // MXFP4: 4 e8m0 codes of one weight row (threads < BN)
  uint32_t xsreg = 0;   // scale of one activation row (threads < BM), float bits or code

  auto load_step = [&](int kb) {
#pragma unroll
    for (int q = 0; q < kWPer; ++q) {
      const int c = tid + q * kPThreads;
      const int r = c / (C::kWRow / 16), col = c % (C::kWRow / 16);
      const uint8_t* p = wexp + static_cast<size_t>(wrow_of(r)) * wrow_bytes + static_cast<size_t>(kb) * C::kWRow + col * 16;
      wreg[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    }
#pragma unroll
    for (int q = 0; q < kXPer; ++q) {
      const int c = tid + q * kPThreads;
      const int r = c / (C::kXRow / 16), col = c % (C::kXRow / 16);
      const int row = s_row[r];
      const int src = row < 0 ? 0 : row;
      const uint8_t* p = a.xq + static_cast<size_t>(src) * xrow_bytes + static_cast<size_t>(kb) * C::kXRow + col * 16;
      xreg[q] = *reinterpret_cast<const u32x4*>(p);
    }
    if constexpr (FMT == FMT_MXFP4) {
      if (tid < kPBN) {
        const uint8_t* sp = static_cast<const uint8_t*>(bank.s) +
                            (static_cast<size_t>(expert) * a.N + wrow_of(tid)) * (a.K / 32) + kb * 4;
        wsreg = *reinterpret_cast<const uint32_t*>(sp);
      }
    }
    if constexpr (FMT != FMT_BF16) {
      if (tid < kPBM) {
        const int row = s_row[tid];
        const int src = row < 0 ? 0 : row;
        if (FMT == FMT_FP8)
          xsreg = __float_as_uint(static_cast<const float*>(a.xs)[static_cast<size_t>(src) * nkb + kb]);
        else
          xsreg = static_cast<const uint8_t*>(a.xs)[static_cast<size_t>(src) * nkb + kb];
      }
    }
  };
  auto store_step = [&](int buf) {
    uint8_t* base = lds + buf * L::kBuf;
#pragma unroll
    for (int q = 0; q < kWPer; ++q) {
      const int c = tid + q * kPThreads;
      const int r = c / (C::kWRow / 16), col = c % (C::kWRow / 16);
      *reinterpret_cast<u32x4*>(base + r * L::kWStride + col * 16) = wreg[q];
    }
#pragma unroll
    for (int q = 0; q < kXPer; ++q) {
      const int c = tid + q * kPThreads;
      const int r = c / (C::kXRow / 16), col = c % (C::kXRow / 16);
      *reinterpret_cast<u32x4*>(base + L::kW + r * L::kXStride + col * 16) = xreg[q];
    }
    if constexpr (FMT == FMT_MXFP4) {
      if (tid < kPBN) *reinterpret_cast<uint32_t*>(base + L::kW + L::kX + tid * 4) = wsreg;
    }
    if constexpr (FMT != FMT_BF16) {
      if (tid < kPBM) *reinterpret_cast<uint32_t*>(base + L::kW + L::kX + L::kWS + tid * 4) = xsreg;
    }
  };

  // wave sub-tiles: weight rows (j) and route columns (i)
  int wrow_base[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (GATE_UP) wrow_base[j] = (j < 2) ? 32 * wn + 16 * j : kPBN / 2 + 32 * wn + 16 * (j - 2);
    else wrow_base[j] = 64 * wn + 16 * j;
  }
  const int xcol_base = 64 * wm;

  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[j][i] = zero;

  load_step(0);
  store_step(0);
  __syncthreads();

  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nkb) load_step(kb + 1);
    const uint8_t* base = lds + cur * L::kBuf;

    if constexpr (FMT == FMT_FP8) {
      float sw[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int wr = wrow_of(wrow_base[j]);
        sw[j] = static_cast<const float*>(bank.s)[(static_cast<size_t>(expert) * (a.N / 128) + wr / 128) * nkb + kb];
      }
      i32x8 xf[4];
      float sx[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint8_t* p = base + L::kW + (xcol_base + 16 * i + r16) * L::kXStride + g * 32;
        const u32x4 lo = *reinterpret_cast<const u32x4*>(p);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(p + 16);
        xf[i] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        sx[i] = *reinterpret_cast<const float*>(base + L::kW + L::kX + L::kWS + (xcol_base + 16 * i + r16) * 4);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint8_t* p = base + (wrow_base[j] + r16) * L::kWStride + g * 32;
        const u32x4 lo = *reinterpret_cast<const u32x4*>(p);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(p + 16);
        const i32x8 wf = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf, xf[i], zero, 0, 0, 0, 0, 0, 0);
          const float f = sx[i] * sw[j];
          acc[j][i] += t * f;
        }
      }
    } else if constexpr (FMT == FMT_MXFP4) {
      // The f8f6f4 MFMA reads an fp8 lane-group g as K = 16g+[0,16) (bytes 0-15)
      // and 64+16g+[0,16) (bytes 16-31), an fp4 lane-group g as the 32-value
      // block [32g, 32g+32), and scale lane-group q as K block q.  The fp4
      // weights are stored K-contiguous, so the fp8 activations are fed in that
      // split order to pair every product with its K.
      i32x8 xf[4];
      int sxc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint8_t* p = base + L::kW + (xcol_base + 16 * i + r16) * L::kXStride;
        const u32x4 lo = *reinterpret_cast<const u32x4*>(p + 16 * g);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(p + 64 + 16 * g);
        xf[i] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        sxc[i] = static_cast<int>(*reinterpret_cast<const uint32_t*>(base + L::kW + L::kX + L::kWS +
                                                                     (xcol_base + 16 * i + r16) * 4));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint8_t* p = base + (wrow_base[j] + r16) * L::kWStride + g * 16;
        const u32x4 v = *reinterpret_cast<const u32x4*>(p);
        const i32x8 wf = {(int)v[0], (int)v[1], (int)v[2], (int)v[3], 0, 0, 0, 0};
        const int swc = base[L::kW + L::kX + (wrow_base[j] + r16) * 4 + g];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          acc[j][i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf, xf[i], acc[j][i], 4, 0, 0, swc, 0, sxc[i]);
      }
    } else {  // FMT_BF16: four K=32 MFMAs per 128 step
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        bf16x8 xf[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint8_t* p = base + L::kW + (xcol_base + 16 * i + r16) * L::kXStride + (g * 32 + s * 8) * 2;
          xf[i] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(p));
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint8_t* p = base + (wrow_base[j] + r16) * L::kWStride + (g * 32 + s * 8) * 2;
          const bf16x8 wf = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(p));
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf, xf[i], acc[j][i], 0, 0, 0);
        }
      }
    }

    if (kb + 1 < nkb) store_step(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds weight rows wrow_base[j] + g*4 + v of route column r16
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int col = xcol_base + 16 * i + r16;
    const int route = s_route[col];
    if (route < 0) continue;
    if (GATE_UP) {
      const int arow = shared ? a.numel + route : route;
      const float lim = shared ? a.sh_act_limit : a.act_limit;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float o[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float gg = bf16_round(acc[s][i][v]);
          float uu = bf16_round(acc[2 + s][i][v]);
          swiglu_clamp(lim, gg, uu);
          o[v] = act_apply(a.act_kind, gg) * uu;
        }
        const int n = n0 + 32 * wn + 16 * s + g * 4;
        uint2 pk;
        pk.x = pack_bf16x2(o[0], o[1]);
        pk.y = pack_bf16x2(o[2], o[3]);
        *reinterpret_cast<uint2*>(a.out + static_cast<size_t>(arow) * a.inter + n) = pk;
      }
    } else {
      const float wt = shared ? 1.0f : a.topk_w[route];
      uint16_t* dst = shared ? a.sh_out + static_cast<size_t>(route) * a.N : a.out + static_cast<size_t>(route) * a.N;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + wrow_base[j] + g * 4;
        uint2 pk;
        pk.x = pack_bf16x2(acc[j][i][0] * wt, acc[j][i][1] * wt);
        pk.y = pack_bf16x2(acc[j][i][2] * wt, acc[j][i][3] * wt);
        *reinterpret_cast<uint2*>(dst + n) = pk;
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Quantised grouped GEMM (FP8, MXFP4) on direct-to-LDS copies
//
// A workgroup of 8 waves computes 256 weight rows x 256 routes (kQBM).  Wave w
// is row group rg = w/2 (64 weight rows: four 16-row MFMA tiles) and column
// half ch = w%2 (128 routes: eight 16-column tiles); two waves share each SIMD,
// so one wave's MFMAs run while the other waits on LDS, folds scales or sits at
// the barrier.  Every operand of a 128-deep K step -- weight rows, activation
// tile, weight scales, activation scales -- is copied global -> LDS by the
// LDS-DMA form of the global loads (no register staging) into a ring of
// kStages stages: the copies of the next kStages-1 steps are in flight while a
// step computes.  Waits are explicit (vmcnt of one step's copies) and the
// barrier is a bare s_barrier, so a barrier never drains copies in flight.
//
// LDS lines (a weight row or an activation column of one K step: 128 bytes,
// 64 for MXFP4 weights) are stored as 16-byte chunks XOR-swizzled by the line
// index (swz_pair, swz_b, swz64: patterns measured free of LDS bank conflicts
// for the way each operand is read).
//
// Gate/up: row group rg owns gate rows n0+32rg+[0,32) and up rows
// I+n0+32rg+[0,32), so SwiGLU pairs registers; a workgroup covers 128
// intermediate features.  Down: rows at or past N (the last tile when
// N % 256 != 0) are read clamped to row N-1 and never stored.  The epilogues
// are VALU work with the matrix cores idle: the gate/up epilogue quantises
// without a division instruction (quant.h) and the down epilogue stores its
// outputs as whole 128-byte rows through LDS.
//
// Schedule (map_tile_q): the active workgroups are laid out XCD-major
// (workgroup b runs on XCD b % 8), so each XCD works through a contiguous range
// of the logical order, in which chunks of q_chunk() M blocks of one expert sweep
// its N tiles: the workgroups an XCD runs at once read several weight tiles and
// share the activations of a few M blocks.
// ----------------------------------------------------------------------------
constexpr int kQBM = 256;     // routes per tile (align block size of the quantised formats)
constexpr int kQRows = 256;   // weight rows per workgroup
constexpr int kQThreads = 512;
constexpr int kXcds = 8;
// M blocks per chunk of the schedule (see map_tile_q): [FP8, MXFP4][gate_up, down].
// Measured on C5 (interleaved A/B, ms): FP8 gate_up 4 -> 2.23-2.24, 8 -> 2.19-2.20,
// 16 -> 2.22, 2 -> 2.32; FP8 down 4 -> 1.25-1.26, 2 -> 1.20, 1 -> 1.22; MXFP4
// gate_up 4 -> 1.79 (2 and 8 slower by 4-7%); MXFP4 down 4 -> 1.04-1.06, 2 ->
// 1.02-1.04, 8 -> 1.09-1.10.
constexpr int kQChunkSel[2][2] = {{8, 2}, {4, 2}};
template <int FMT, int GATE_UP>
constexpr int q_chunk() {
  return kQChunkSel[FMT == FMT_FP8 ? 0 : 1][GATE_UP ? 0 : 1];
}
constexpr int kFoldLag = 3;  // FP8: MFMAs between an MFMA and the fold of its result

template <int FMT>
struct QLds {
  static constexpr int kStages = FMT == FMT_FP8 ? 2 : 3;
  static constexpr int kALine = FMT == FMT_FP8 ? 128 : 64;   // weight bytes per row per K step
  static constexpr int kA = kQRows * kALine;
  static constexpr int kAS = FMT == FMT_FP8 ? 4 * 16 : kQRows * 4;  // fp8: 4 floats per row group; mxfp4: 4 codes per row
  static constexpr int kB = kQBM * 128;
  static constexpr int kBS = kQBM * 4;
  static constexpr int kOffAS = kA, kOffB = kA + kAS, kOffBS = kA + kAS + kB;
  static constexpr int kStage = kA + kAS + kB + kBS;
  static constexpr int kTotal = kStages * kStage;
  static constexpr int kACopies = kA / 1024 / 8;   // 1 KB copies per wave per step
  static constexpr int kBCopies = kB / 1024 / 8;
  // LDS-DMA instructions each wave issues per K step (uniform over waves)
  static constexpr int kDmaPerStep = kACopies + kBCopies + 1;
};

__device__ __forceinline__ int xcd_major(int b, int n) {
  const int per = n / kXcds, rem = n % kXcds;
  const int x = b % kXcds, i = b / kXcds;
  return x * per + min(x, rem) + i;
}

// (M block, N tile) of position `local` in a group of nb M blocks x ntiles:
// chunks of kQChunk M blocks, each chunk sweeping all N tiles.
template <int kQChunk>
__device__ __forceinline__ void chunked(int local, int nb, int ntiles, int& m, int& ntile) {
  const int full = nb / kQChunk, rem = nb - full * kQChunk;
  const int span = kQChunk * ntiles;
  if (local < full * span) {
    const int c = local / span, w = local - c * span;
    ntile = w / kQChunk;
    m = c * kQChunk + (w - ntile * kQChunk);
  } else {
    const int w = local - full * span;
    ntile = w / rem;
    m = full * kQChunk + (w - ntile * rem);
  }
}

// Workgroup b of the grid -> (expert or shared, M block, N tile).  Only the
// active workgroups -- routed blocks of the real experts, then the shared
// expert's blocks -- take part; they are laid out XCD-major over their own
// count, so every XCD gets the same share.  Returns false for idle ones.
template <int kQChunk>
__device__ __forceinline__ bool map_tile_q(const PrefillGemmArgs& a, int b, bool& shared, int& expert, int& mblock,
                                           int& ntile) {
  const int routed = (a.cum[a.num_experts] / kQBM) * a.ntiles;
  const int total = routed + a.shared_blocks * a.ntiles;
  if (b >= total) return false;
  const int wg = xcd_major(b, total);
  if (wg < routed) {
    int lo = 0, hi = a.num_experts;  // largest e with cum[e]/BM * ntiles <= wg
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if ((a.cum[mid] / kQBM) * a.ntiles <= wg) lo = mid; else hi = mid;
    }
    const int b0 = a.cum[lo] / kQBM;
    const int nb = a.cum[lo + 1] / kQBM - b0;
    int m;
    chunked<kQChunk>(wg - b0 * a.ntiles, nb, a.ntiles, m, ntile);
    shared = false;
    expert = lo;
    mblock = b0 + m;
    return true;
  }
  chunked<kQChunk>(wg - routed, a.shared_blocks, a.ntiles, mblock, ntile);
  shared = true;
  expert = 0;
  return true;
}

// Lane index as an asm result: the compiler can neither hoist nor merge it,
// so per-tile set-up code recomputes its lane-derived values instead of keeping
// them live (or spilled) across the K loop.
__device__ __forceinline__ int fresh_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

struct QTile {
  bool shared;  // the shared expert's blocks (tokens in order) instead of a routed expert's
  int expert, mblock, ntile;
};

template <int kQChunk>
__device__ __forceinline__ bool map_tile_q(const PrefillGemmArgs& a, int b, QTile& t) {
  return map_tile_q<kQChunk>(a, b, t.shared, t.expert, t.mblock, t.ntile);
}

// s_barrier without the memory fence of __syncthreads (which would wait for
// every copy in flight); the clobber keeps the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void bare_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// LDS-DMA copies through a buffer descriptor: each lane's 16 (4) bytes at lane
// offset voff plus the wave-uniform soff land at dst + lane * 16 (4), dst
// wave-uniform; a lane offset at or past the descriptor's range reads zeros
// without memory traffic.
__device__ __forceinline__ void lds_buf16(__amdgpu_buffer_rsrc_t r, uint8_t* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void lds_buf4(__amdgpu_buffer_rsrc_t r, uint8_t* dst, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 4, voff, soff, 0, 0);
}

// Chunk swizzles of the LDS lines, chosen by measurement (rocprofv3
// SQ_LDS_BANK_CONFLICT over ds_read_b128 patterns on gfx950): for 128-byte
// lines read as chunk pairs (2g, 2g+1) -- the FP8 operands -- position
// c ^ swz_pair(line) is conflict-free while c ^ (line & 7) is not; for lines
// read as chunks (g, 4+g) -- the MXFP4 activations -- c ^ (line & 7) is
// conflict-free; for 64-byte lines read as chunk g -- the MXFP4 weights --
// c ^ ((line >> 1) & 3) is.
__device__ __forceinline__ int swz_pair(int line) { return ((line & 3) << 1) | ((line >> 2) & 1); }
template <int FMT>
__device__ __forceinline__ int swz_b(int line) { return FMT == FMT_FP8 ? swz_pair(line) : (line & 7); }
__device__ __forceinline__ int swz64(int line) { return (line >> 1) & 3; }

// Empty asm that keeps the value's update at this point of the instruction
// stream (no code is emitted).
__device__ __forceinline__ void pin(f32x4& v) { asm volatile("" : "+v"(v)); }

template <int FMT, int GATE_UP>
__global__ void __launch_bounds__(kQThreads) prefill_qgemm_kernel(PrefillGemmArgs a) {
  using L = QLds<FMT>;
  constexpr int S = L::kStages;
  constexpr int D = S - 1;  // prefetch distance in K steps
  extern __shared__ __attribute__((aligned(16))) uint8_t q_lds[];
  __shared__ int s_row[2][kQBM];    // per tile parity: activation row of each route column (-1: padding)
  __shared__ int s_route[2][kQBM];  // per tile parity: route of each column (-1: padding)
  __shared__ float s_amax[GATE_UP ? 4 * kQBM : 1];  // gate_up epilogue: [row group][column] amax
  __shared__ float s_wt[GATE_UP ? 1 : 2][kQBM];      // down: per tile parity, router weight of each column

  int v = blockIdx.x;
  QTile cur;
  constexpr int kChunk = q_chunk<FMT, GATE_UP>();
  if (!map_tile_q<kChunk>(a, v, cur)) return;

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int rg = wave >> 1, ch = wave & 1;
  const int r16 = lane & 15, g = lane >> 4;
  const int K = a.K, nkb = K / 128;
  const uint32_t rb = FMT == FMT_FP8 ? static_cast<uint32_t>(K) : static_cast<uint32_t>(K) / 2;

  // column tid of tile t from its align entry `raw` (routed tiles) and, for
  // the down GEMM, the route's router weight wraw (loaded with raw, well
  // before this call, so its latency stays off the epilogue)
  auto put_rows = [&](const QTile& t, int raw, float wraw, int b) {
    const int tid = wave * kWave + fresh_lane();
    int row = -1, route = -1;
    if (t.shared) {
      const int tk = t.mblock * kQBM + tid;
      if (tk < a.M) {
        route = tk;
        row = a.x_token_rows ? tk : a.numel + tk;
      }
    } else if (raw < a.numel) {
      route = raw;
      row = a.x_token_rows ? raw / a.k : raw;
    }
    s_row[b][tid] = row;
    s_route[b][tid] = route;
    if constexpr (!GATE_UP) s_wt[b][tid] = t.shared ? 1.0f : wraw;
  };
  auto raw_of = [&](const QTile& t) -> int { return t.shared ? 0 : a.sorted[t.mblock * kQBM + tid]; };
  auto wt_of = [&](const QTile& t, int raw) -> float {
    return (GATE_UP || t.shared || raw >= a.numel) ? 1.0f : a.topk_w[raw];
  };
  auto n0_of = [&](const QTile& t) -> int { return GATE_UP ? t.ntile * (kQRows / 2) : t.ntile * kQRows; };
  // first weight row of tile j of row group q, relative to the tile's first row n0
  auto trow_rel = [&](int q, int j) -> int {
    if (GATE_UP) return (j < 2 ? 0 : a.inter) + 32 * q + 16 * (j & 1);
    return 64 * q + 16 * j;
  };

  // ---- sources of the copies: buffer descriptors + 32-bit lane offsets of K
  // step 0 (step kb adds kb * step bytes as the scalar offset).  Weight rows,
  // weight scales and activation rows past their range (the last down tile's
  // rows past N, padding route columns) read zeros without memory traffic.
  const int xrows = a.x_token_rows ? a.M : a.numel + a.M;
  const __amdgpu_buffer_rsrc_t rsrc_x = make_rsrc(a.xq, static_cast<uint32_t>(xrows) * K);
  __amdgpu_buffer_rsrc_t rsrc_w;
  // scales: the activation scales' descriptor is the kernel's; the weight
  // scales' is set per tile for every wave (waves 4-7 never use it), so that
  // both stay wave-uniform values in scalar registers (a descriptor assigned
  // under a per-wave condition was kept in vector registers and every copy
  // became a loop over its distinct values)
  const __amdgpu_buffer_rsrc_t rsrc_xs = make_rsrc(a.xs, static_cast<uint32_t>(xrows) * nkb * 4);
  __amdgpu_buffer_rsrc_t rsrc_ws = rsrc_xs;
  // weights: copy c of wave w fills LDS rows of 1 KB block i = w*kACopies + c
  uint32_t avoff[L::kACopies];
#pragma unroll
  for (int c = 0; c < L::kACopies; ++c) {
    const int i = wave * L::kACopies + c;
    int R, q;
    if constexpr (FMT == FMT_FP8) {
      R = 8 * i + (lane >> 3);
      q = (lane & 7) ^ swz_pair(R);
    } else {
      R = 16 * i + (lane >> 2);
      q = (lane & 3) ^ swz64(R);
    }
    avoff[c] = static_cast<uint32_t>(trow_rel(R >> 6, (R >> 4) & 3) + (R & 15)) * rb + q * 16;
  }
  // scales: waves 0-3 copy their row group's weight scales (offsets fixed
  // relative to the tile), waves 4-7 64 activation-scale columns each
  uint32_t svoff = 0;
  if (wave < 4) {
    if constexpr (FMT == FMT_FP8) svoff = static_cast<uint32_t>(trow_rel(wave, lane & 3) / 128) * nkb * 4;
    else svoff = static_cast<uint32_t>(trow_rel(wave, lane >> 4) + (lane & 15)) * (K / 32);
  }
  uint8_t* const sdst_base = q_lds + (wave < 4 ? (FMT == FMT_FP8 ? L::kOffAS + wave * 16 : L::kOffAS + wave * 256)
                                               : L::kOffBS + (wave - 4) * 256);
  const bool scopy = wave >= 4 || FMT != FMT_FP8 || lane < 4;
  // activations: copy c of wave w fills LDS columns of 1 KB block i = w*kBCopies + c
  uint32_t xvoff[L::kBCopies];
  auto setup = [&](const QTile& t, int b) {
    const BankView bank = t.shared ? a.ws : a.w;
    const int n0 = n0_of(t);
    rsrc_w = make_rsrc(bank.w + (static_cast<size_t>(t.expert) * a.N + n0) * rb, static_cast<uint32_t>(a.N - n0) * rb);
    if constexpr (FMT == FMT_FP8)
      rsrc_ws = make_rsrc(static_cast<const uint8_t*>(bank.s) +
                              (static_cast<size_t>(t.expert) * (a.N / 128) + n0 / 128) * nkb * 4,
                          static_cast<uint32_t>((a.N - n0) / 128) * nkb * 4);
    else
      rsrc_ws = make_rsrc(static_cast<const uint8_t*>(bank.s) + (static_cast<size_t>(t.expert) * a.N + n0) * (K / 32),
                          static_cast<uint32_t>(a.N - n0) * (K / 32));
    const int ln = fresh_lane();
    if (wave >= 4) {
      const int row = s_row[b][64 * (wave - 4) + ln];
      svoff = row < 0 ? kOutOfRange : static_cast<uint32_t>(row) * nkb * 4;
    }
#pragma unroll
    for (int c = 0; c < L::kBCopies; ++c) {
      const int col = 8 * (wave * L::kBCopies + c) + (ln >> 3);
      const int q = (ln & 7) ^ swz_b<FMT>(col);
      const int row = s_row[b][col];
      xvoff[c] = row < 0 ? kOutOfRange : static_cast<uint32_t>(row) * K + q * 16;
    }
  };

  // piece q of a K step's copies (weight copies, activation copies, scales)
  constexpr int kPieces = L::kACopies + L::kBCopies + 1;
  auto issue_piece = [&](int q, int kb, int stg) {
    uint8_t* st = q_lds + stg * L::kStage;
    if (q < L::kACopies) {
      lds_buf16(rsrc_w, st + (wave * L::kACopies + q) * 1024, avoff[q], static_cast<uint32_t>(kb) * L::kALine);
    } else if (q < L::kACopies + L::kBCopies) {
      const int c = q - L::kACopies;
      lds_buf16(rsrc_x, st + L::kOffB + (wave * L::kBCopies + c) * 1024, xvoff[c], static_cast<uint32_t>(kb) * 128);
    } else if (wave < 4) {
      if (scopy) lds_buf4(rsrc_ws, sdst_base + stg * L::kStage, svoff, static_cast<uint32_t>(kb) * 4);
    } else {
      lds_buf4(rsrc_xs, sdst_base + stg * L::kStage, svoff, static_cast<uint32_t>(kb) * 4);
    }
  };
  auto issue = [&](int kb, int stg) {
    uint8_t* st = q_lds + stg * L::kStage;
#pragma unroll
    for (int c = 0; c < L::kACopies; ++c)
      lds_buf16(rsrc_w, st + (wave * L::kACopies + c) * 1024, avoff[c], static_cast<uint32_t>(kb) * L::kALine);
#pragma unroll
    for (int c = 0; c < L::kBCopies; ++c)
      lds_buf16(rsrc_x, st + L::kOffB + (wave * L::kBCopies + c) * 1024, xvoff[c], static_cast<uint32_t>(kb) * 128);
    if (wave < 4) {
      if (scopy) lds_buf4(rsrc_ws, sdst_base + stg * L::kStage, svoff, static_cast<uint32_t>(kb) * 4);
    } else {
      lds_buf4(rsrc_xs, sdst_base + stg * L::kStage, svoff, static_cast<uint32_t>(kb) * 4);
    }
  };

  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[4][8];

  // One K step from stage stg.  With ikb >= 0 the copies of step ikb into
  // stage istg are issued two per column tile in the first tiles, between the
  // LDS reads and MFMAs, instead of as one burst before the step (a burst
  // stalls the wave's in-order issue until the memory pipeline takes it:
  // measured 3% of the FP8 gate_up GEMM; MXFP4, whose 3-stage ring already
  // spills a few registers, keeps the burst).
  constexpr bool kSpread = FMT == FMT_FP8;
  auto compute = [&](int stg, int ikb, int istg) {
    const uint8_t* st = q_lds + stg * L::kStage;
    i32x8 wf[4];
    int wcode[4];
    float sw[4];
    auto read_w = [&](int j) {
      const int R = 64 * rg + 16 * j + r16;
      if constexpr (FMT == FMT_FP8) {
        const uint8_t* p = st + R * 128;
        const u32x4 lo = *reinterpret_cast<const u32x4*>(p + (((2 * g) ^ swz_pair(R)) * 16));
        const u32x4 hi = *reinterpret_cast<const u32x4*>(p + (((2 * g + 1) ^ swz_pair(R)) * 16));
        wf[j] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
        sw[j] = *reinterpret_cast<const float*>(st + L::kOffAS + rg * 16 + j * 4);
      } else {
        const u32x4 v4 = *reinterpret_cast<const u32x4*>(st + R * 64 + ((g ^ swz64(R)) * 16));
        wf[j] = i32x8{(int)v4[0], (int)v4[1], (int)v4[2], (int)v4[3], 0, 0, 0, 0};
        wcode[j] = st[L::kOffAS + R * 4 + g];
      }
    };
    // Column tile i reads route column 128ch + 16i + r16.  The chunk swizzle
    // depends on the column's low 3 bits (those of r16) only, so every tile's
    // reads are one per-lane base of the step plus a compile-time offset
    // (2048 B per tile for the codes, 64 B for the scales): no address
    // arithmetic per tile.  The f8f6f4 MFMA reads an fp8 lane group g as
    // K = 16g+[0,16) and 64+16g+[0,16), an fp4 lane group as the block
    // [32g, 32g+32).
    const int c0 = 128 * ch + r16;
    const int q_lo = FMT == FMT_FP8 ? (2 * g) ^ swz_b<FMT>(r16) : g ^ swz_b<FMT>(r16);
    const int q_hi = FMT == FMT_FP8 ? (2 * g + 1) ^ swz_b<FMT>(r16) : (4 + g) ^ swz_b<FMT>(r16);
    const uint8_t* const x_lo = st + L::kOffB + c0 * 128 + q_lo * 16;
    const uint8_t* const x_hi = st + L::kOffB + c0 * 128 + q_hi * 16;
    const uint8_t* const x_sc = st + L::kOffBS + c0 * 4;
    auto read_x = [&](int i, i32x8& xf, uint32_t& xs) {
      const u32x4 lo = *reinterpret_cast<const u32x4*>(x_lo + 2048 * i);
      const u32x4 hi = *reinterpret_cast<const u32x4*>(x_hi + 2048 * i);
      xf = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
      xs = *reinterpret_cast<const uint32_t*>(x_sc + 64 * i);
    };
    // The next column tile's LDS reads are issued before this tile's MFMAs.
    // FP8: each scale fold is written kFoldLag MFMAs after its own MFMA (its
    // result register stays live that long), so the compiler can place the
    // fold's VALU work while the matrix core runs later MFMAs instead of
    // waiting out the MFMA result latency; pin() keeps the accumulator updates
    // in that order.
    i32x8 xf[2];
    uint32_t xs[2];
    if constexpr (FMT == FMT_FP8) {
      // The step's first MFMA needs row tile 0 and column tile 0 only: those
      // reads are issued first (LDS returns in order), so after the barrier
      // each wave waits for four reads instead of the whole step's weight
      // tiles (FP8 GEMMs 1.7% faster; MXFP4, whose weight tiles are one read
      // each, 3% slower, so it keeps the weight tiles first)
      read_w(0);
      read_x(0, xf[0], xs[0]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 1; j < 4; ++j) read_w(j);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) read_w(j);
      read_x(0, xf[0], xs[0]);
    }
    // FP8: kFoldLag MFMA results in flight (tq, with their fold factors fq)
    constexpr int P = kFoldLag;
    f32x4 tq[P];
    float fq[P];
#pragma unroll
    for (int q = 0; q < P; ++q) {
      tq[q] = zero;
      fq[q] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (ikb >= 0) {
#pragma unroll
        for (int q = 2 * i; q < 2 * i + 2; ++q)
          if (q < kPieces) issue_piece(q, ikb, istg);
      }
      if (i + 1 < 8) read_x(i + 1, xf[(i + 1) & 1], xs[(i + 1) & 1]);
      // FP8 fold factors of this column tile: a weight scale covers 128 rows,
      // so tiles j = 0, 1 (gate rows) share one and tiles 2, 3 (up rows)
      // another, and the down GEMM's 64 rows of a wave share one
      float fi[2] = {0.f, 0.f};
      if constexpr (FMT == FMT_FP8) fi[0] = __uint_as_float(xs[i & 1]) * sw[0];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (FMT == FMT_FP8) {
          const f32x4 t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[j], xf[i & 1], zero, 0, 0, 0, 0, 0, 0);
          // the step's first MFMA goes out before anything that waits on the
          // later weight-tile reads (the up rows' scale factor among them)
          if (i == 0 && j == 0) {
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (GATE_UP) asm volatile("" : "+v"(sw[2]));
          }
          if (j == 1) fi[1] = GATE_UP ? __uint_as_float(xs[i & 1]) * sw[2] : fi[0];
          const int k = 4 * i + j;
          if (k >= P) {
            const int pi = (k - P) >> 2, pj = (k - P) & 3;
            acc[pj][pi] += tq[k % P] * fq[k % P];
            pin(acc[pj][pi]);
          }
          tq[k % P] = t;
          fq[k % P] = fi[j >> 1];
        } else {
          acc[j][i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wf[j], xf[i & 1], acc[j][i], 4, 0, 0, wcode[j], 0,
                                                                       static_cast<int>(xs[i & 1]));
        }
      }
    }
    if constexpr (FMT == FMT_FP8) {
#pragma unroll
      for (int k = 32 - P; k < 32; ++k) acc[k & 3][k >> 2] += tq[k % P] * fq[k % P];
    }
  };

  // ---- epilogue: lane holds rows trow + g*4 + v of route column 128ch + 16i + r16
  // (stg: an LDS stage that no copy targets before the next tile's K loop)
  auto epilogue = [&](const QTile& t, int b, uint8_t* stg) {
    const int n0 = n0_of(t);
    if constexpr (GATE_UP) {
      // SwiGLU, then the down GEMM's activation quantisation of this 128-feature
      // group (one K group of the down GEMM) per route: amax over the 32 features
      // of the wave (lanes g = 0..3 of a column) and over the 4 row groups (LDS).
      constexpr int QMODE = FMT == FMT_FP8 ? 0 : 2;
      uint32_t pk[8][2][2];  // bf16 pairs (v0,v1), (v2,v3) of each column tile and gate/up tile pair
      float amax[8];
      // SiLU (every configuration here) runs as straight-line code with its
      // kind and the clamp of a clamped SwiGLU fixed at compile time; the other
      // kinds keep the runtime choice
      const float lim = t.shared ? a.sh_act_limit : a.act_limit;
      auto swiglu = [&](auto kind, auto clamp) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float m = 0.f;
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            float o[4];
#pragma unroll
            for (int v4 = 0; v4 < 4; ++v4) {
              // gate and up of one feature rounded to bf16 by one packed conversion
              const uint32_t gu = pack_bf16x2(acc[s2][i][v4], acc[2 + s2][i][v4]);
              float gg = __uint_as_float(gu << 16), uu = __uint_as_float(gu & 0xffff0000u);
              if constexpr (decltype(clamp)::value) {
                gg = fminf(gg, lim);
                uu = fminf(fmaxf(uu, -lim), lim);
              }
              float act;
              if constexpr (decltype(kind)::value == ACT_SILU) act = act_fixed<ACT_SILU>(gg);
              else act = act_apply(a.act_kind, gg);
              o[v4] = act * uu;
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const uint32_t p2 = pack_bf16x2(o[2 * h], o[2 * h + 1]);
              pk[i][s2][h] = p2;
              m = fmaxf(m, fmaxf(fabsf(__uint_as_float(p2 << 16)), fabsf(__uint_as_float(p2 & 0xffff0000u))));
            }
          }
          m = fmaxf(m, __shfl_xor(m, 16));
          m = fmaxf(m, __shfl_xor(m, 32));
          amax[i] = m;
        }
      };
      if (a.act_kind == ACT_SILU) {
        if (lim > 0.f) swiglu(std::integral_constant<int, ACT_SILU>{}, std::true_type{});
        else swiglu(std::integral_constant<int, ACT_SILU>{}, std::false_type{});
      } else {
        swiglu(std::integral_constant<int, -1>{}, std::false_type{});
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (g == 0) s_amax[rg * kQBM + 128 * ch + 16 * i + r16] = amax[i];
      // publish the amax (LDS only: the next tile's copies stay in flight)
      wait_lgkm0();
      bare_barrier();
      const int ng = a.inter / 128;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int col = 128 * ch + 16 * i + r16;
        const int route = s_route[b][col];
        if (route < 0) continue;
        const float m =
            fmaxf(fmaxf(s_amax[col], s_amax[kQBM + col]), fmaxf(s_amax[2 * kQBM + col], s_amax[3 * kQBM + col]));
        float mul;
        const float sc = group_scale<QMODE>(m, mul);
        const int arow = t.shared ? a.numel + route : route;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          float vals[4];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            vals[2 * h] = quant_value<QMODE>(bf16_to_f32(static_cast<uint16_t>(pk[i][s2][h] & 0xffffu)), sc, mul);
            vals[2 * h + 1] = quant_value<QMODE>(bf16_to_f32(static_cast<uint16_t>(pk[i][s2][h] >> 16)), sc, mul);
          }
          uint32_t q4 = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(vals[0], vals[1], 0, false));
          q4 = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(vals[2], vals[3], static_cast<int>(q4), true));
          const int n = n0 + 32 * rg + 16 * s2 + g * 4;
          *reinterpret_cast<uint32_t*>(a.act_q + static_cast<size_t>(arow) * a.inter + n) = q4;
        }
        if (rg == 0 && g == 0) {
          const size_t at = static_cast<size_t>(arow) * ng + t.ntile;
          if (QMODE == 0) static_cast<float*>(a.act_s)[at] = sc;
          else static_cast<uint32_t*>(a.act_s)[at] = static_cast<uint32_t>(sc);
        }
      }
    } else {
      // A lane holds 4 consecutive output rows of a route, so direct stores
      // write 32-byte pieces of 16 routes per instruction.  The outputs are
      // staged in LDS instead (CT column tiles per pass, each wave in its own
      // 128-byte-per-route area, 16-byte chunks swizzled by route so that
      // writes and reads are conflict-free) and stored as whole 128-byte rows
      // of this wave's 64 output rows, 8 routes per instruction: half the
      // store instructions and a quarter of the memory requests.  N is a
      // multiple of 128, so a wave's rows are all inside N or all past it.
      constexpr int CT = FMT == FMT_FP8 ? 4 : 2;
      static_assert(8 * 16 * CT * 128 <= L::kStage, "a pass's staging areas fit one stage");
      uint8_t* const mine = stg + wave * (16 * CT * 128);
      const int nrow0 = n0 + 64 * rg;
      const bool rows_in = nrow0 < a.N;
      uint16_t* const base = t.shared ? a.sh_out : a.out;
#pragma unroll
      for (int p = 0; p < 8 / CT; ++p) {
#pragma unroll
        for (int ii = 0; ii < CT; ++ii) {
          const int i = p * CT + ii;
          const int c = 16 * ii + r16;  // staging row of this lane's route
          const float wt = s_wt[b][128 * ch + 16 * i + r16];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            uint2 pk2;
            pk2.x = pack_bf16x2(acc[j][i][0] * wt, acc[j][i][1] * wt);
            pk2.y = pack_bf16x2(acc[j][i][2] * wt, acc[j][i][3] * wt);
            // rows 16j + 4g .. +3 are bytes 32j + 8g of the route's 128
            const int chunk = (2 * j + (g >> 1)) ^ (c & 7);
            *reinterpret_cast<uint2*>(mine + c * 128 + chunk * 16 + (g & 1) * 8) = pk2;
          }
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
#pragma unroll
        for (int kk = 0; kk < 2 * CT; ++kk) {
          const int c = 8 * kk + (lane >> 3), chunk = lane & 7;
          const u32x4 v = *reinterpret_cast<const u32x4*>(mine + c * 128 + ((chunk ^ (c & 7)) * 16));
          const int route = s_route[b][128 * ch + 16 * (p * CT + (c >> 4)) + (c & 15)];
          if (route >= 0 && rows_in)
            *reinterpret_cast<u32x4*>(base + static_cast<size_t>(route) * a.N + nrow0 + 8 * chunk) = v;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      }
    }
  };

  // ---- persistent loop over this workgroup's tiles (v, v + grid, ...).  The
  // K pipeline runs over a ring of S LDS stages with copies D steps ahead; the
  // ring continues across tiles (global step g0 + kb), so the last D steps of a
  // tile issue the next tile's first D steps, which land while this tile's
  // epilogue runs.  The next tile's align entries are loaded at the start of
  // a tile and published before its last D steps.
  if (tid < kQBM) {
    const int raw0 = raw_of(cur);
    put_rows(cur, raw0, wt_of(cur, raw0), 0);
  }
  __syncthreads();
  setup(cur, 0);
  int buf = 0, g0 = 0;
  bool ahead = false;  // this tile's first D steps were issued during the previous tile
  for (;;) {
    if (!ahead) {
#pragma unroll
      for (int d = 0; d < D; ++d)
        if (d < nkb) issue(d, (g0 + d) % S);
    }
    QTile nxt;
    const bool has_next = map_tile_q<kChunk>(a, v + static_cast<int>(gridDim.x), nxt);
    const bool cross = has_next && nkb > D;  // the next tile's first steps ride in this tile's last D steps
    // (pinned: a known-zero accumulator would let the compiler schedule the
    // first step, which it peels, apart from the others, at a register cost)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        acc[j][i] = zero;
        pin(acc[j][i]);
      }
    wait_vm<0>();
    bare_barrier();
    const int raw = has_next && tid < kQBM ? raw_of(nxt) : 0;
    const float wraw = has_next && tid < kQBM ? wt_of(nxt, raw) : 1.0f;
    // steady steps: step kb + D of this tile is issued; step kb + 1 must have
    // landed at the end (later ones may still fly); every LDS read of the step
    // has returned before its MFMA used it
    int kb = 0;
    for (; kb < nkb - D; ++kb) {
      if constexpr (kSpread) {
        compute((g0 + kb) % S, kb + D, (g0 + kb + D) % S);
      } else {
        issue(kb + D, (g0 + kb + D) % S);
        compute((g0 + kb) % S, -1, 0);
      }
      if (D == 2 && (kb + 2 < nkb || cross)) wait_vm<L::kDmaPerStep>();
      else wait_vm<0>();
      wait_lgkm0();
      bare_barrier();
    }
    // publish the next tile's rows; its first steps ride in this tile's last
    // D steps
    if (has_next) {
      if (tid < kQBM) put_rows(nxt, raw, wraw, buf ^ 1);
      wait_lgkm0();
      bare_barrier();
      if (cross) setup(nxt, buf ^ 1);
    }
    for (; kb < nkb; ++kb) {
      if constexpr (kSpread) {
        compute((g0 + kb) % S, cross ? kb + D - nkb : -1, (g0 + kb + D) % S);
      } else {
        if (cross) issue(kb + D - nkb, (g0 + kb + D) % S);
        compute((g0 + kb) % S, -1, 0);
      }
      if (kb + 1 < nkb) {
        if (D == 2 && cross) wait_vm<L::kDmaPerStep>();
        else wait_vm<0>();
      }
      wait_lgkm0();
      bare_barrier();
    }
    // the stage of this tile's last step: the next tile's first D steps ride
    // in the other stages, and its step D is issued after the barrier that
    // starts its K loop
    epilogue(cur, buf, q_lds + ((g0 + nkb + D) % S) * L::kStage);
    if (!has_next) break;
    ahead = cross;
    cur = nxt;
    buf ^= 1;
    g0 += nkb;
    v += static_cast<int>(gridDim.x);
    if (!ahead) setup(cur, buf);
  }
}

hipError_t launch_act_quant(int mode, const uint16_t* x, int rows, int K, uint8_t* q, void* scales,
                            hipStream_t stream) {
  const dim3 grid((rows + 3) / 4), block(256);
  if (mode == 0)
    hipLaunchKernelGGL(act_quant_kernel<0>, grid, block, 0, stream, x, rows, K, q, scales);
  else if (mode == 1)
    hipLaunchKernelGGL(act_quant_kernel<1>, grid, block, 0, stream, x, rows, K, q, scales);
  else
    hipLaunchKernelGGL(act_quant_kernel<2>, grid, block, 0, stream, x, rows, K, q, scales);
  return hipGetLastError();
}

template <int FMT, int GU>
static hipError_t launch_gemm_t(const PrefillGemmArgs& a, hipStream_t stream) {
  static bool attr = false;
  const void* fn = reinterpret_cast<const void*>(prefill_gemm_kernel<FMT, GU>);
  if (!attr) {
    hipError_t err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, Lds<FMT>::kTotal);
    if (err != hipSuccess) return err;
    attr = true;
  }
  const int wgs = (a.max_blocks + a.shared_blocks) * a.ntiles;
  hipLaunchKernelGGL((prefill_gemm_kernel<FMT, GU>), dim3(wgs), dim3(kPThreads), Lds<FMT>::kTotal, stream, a);
  return hipGetLastError();
}

// CUs of the current device, rounded down to a multiple of the XCD count
static int q_cu_count() {
  static int cached = 0;
  if (cached == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                  hipSuccess || n < kXcds)
      n = 256;
    cached = n / kXcds * kXcds;
  }
  return cached;
}

template <int FMT, int GU>
static hipError_t launch_qgemm_t(PrefillGemmArgs a, hipStream_t stream) {
  static bool attr = false;
  if (!attr) {
    const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(prefill_qgemm_kernel<FMT, GU>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, QLds<FMT>::kTotal);
    if (err != hipSuccess) return err;
    attr = true;
  }
  a.ntiles = GU ? a.inter / (kQRows / 2) : (a.N + kQRows - 1) / kQRows;
  // persistent: one workgroup per CU (the LDS ring admits one), each walking
  // tiles b, b + grid, ...; the grid is a multiple of the XCD count, so a
  // workgroup's tiles all map to its own XCD's range
  const long long tiles = static_cast<long long>(a.max_blocks + a.shared_blocks) * a.ntiles;
  const int wgs = static_cast<int>(std::min<long long>(tiles, q_cu_count()));
  if (wgs <= 0) return hipSuccess;
  hipLaunchKernelGGL((prefill_qgemm_kernel<FMT, GU>), dim3(wgs), dim3(kQThreads), QLds<FMT>::kTotal, stream, a);
  return hipGetLastError();
}

hipError_t launch_prefill_gemm(int fmt, int gate_up, const PrefillGemmArgs& a, hipStream_t stream) {
  if (fmt == FMT_FP8) return gate_up ? launch_qgemm_t<FMT_FP8, 1>(a, stream) : launch_qgemm_t<FMT_FP8, 0>(a, stream);
  if (fmt == FMT_MXFP4)
    return gate_up ? launch_qgemm_t<FMT_MXFP4, 1>(a, stream) : launch_qgemm_t<FMT_MXFP4, 0>(a, stream);
  if (fmt == FMT_BF16) return gate_up ? launch_gemm_t<FMT_BF16, 1>(a, stream) : launch_gemm_t<FMT_BF16, 0>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace ftmoe
