// Decode expert GEMVs: expert-major, each touched expert's weights streamed once.
//
// Work unit: one workgroup = (expert segment, 16-row tile).  A segment is one
// expert with all of its routes (or the shared expert with all tokens); the
// routes of a segment are processed 16 at a time as the N side of a
// v_mfma_f32_16x16x32_bf16, so an expert is read once per 64 routes (4 chunks
// kept in registers) instead of once per route as in the reference's per-route
// decode kernels (kernel/triton/fp8_blockscale_moe.py:23-96).
//
// Weights are the MFMA A operand (rows = output features), activations the B
// operand (columns = routes).  Lane l supplies row/column l%16 and, for each
// 128-wide K block, the 32 K values [kb*128 + (l/16)*32, +32): four MFMAs of
// 8 values each.  A and B use the same K mapping, so the products pair up no
// matter how the hardware orders K inside an MFMA.
//
// The 4 waves of a workgroup split K (wave w takes K blocks w, w+4, ...), and
// their partial sums are reduced through LDS in fixed wave order, so results are
// deterministic.
//
// Formats (A operand dequant, in registers, exact):
//   FMT_BF16   bf16 rows, used as is.
//   FMT_FP8    e4m3 -> bf16 with v_cvt_scalef32_pk_bf16_fp8; the float32 128x128
//              block scale multiplies the K-block partial (W8A16, reference
//              _decode_fp8_moe_kernel: acc += sum(w*a) * s).
//   FMT_MXFP4  e2m1 -> bf16 with v_cvt_scalef32_pk_bf16_fp4 and the e8m0 scale of
//              the lane's 32-value block (power of two, exact in bf16).
//
// Stage 0 (gate_up): rows i0..i0+15 of gate and the same rows of up, then
//   a = bf16(act(bf16(g)) * bf16(u)) stored to the act buffer.
// Stage 1 (down): rows h0..h0+15, routed: ic3[route] = bf16(acc * w[route]),
//   shared: sh_out[token] = bf16(acc).
// A third kernel sums the routes of every token (and the shared expert).
#include "kernels.h"

namespace ftmoe {

constexpr int kTch = 4;       // route chunks (of 16) held in registers per pass
constexpr int kDecWaves = 4;  // waves per workgroup (K split)

template <int FMT>
__device__ __forceinline__ size_t row_bytes(int K) {
  return FMT == FMT_BF16 ? static_cast<size_t>(K) * 2 : FMT == FMT_FP8 ? static_cast<size_t>(K) : static_cast<size_t>(K) / 2;
}

// Loads and dequantises the lane's 32 K values of one weight row for K block kb
// into four bf16x8 MFMA operands.  Returns the block scale for FMT_FP8 (else 1).
template <int FMT>
__device__ __forceinline__ void load_a(const uint8_t* row, const void* sbase, int row_idx, int K, int kb,
                                       int g, bf16x8 (&a)[4]) {
  if constexpr (FMT == FMT_BF16) {
    const u32x4* p = reinterpret_cast<const u32x4*>(row + (static_cast<size_t>(kb) * 128 + g * 32) * 2);
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = __builtin_bit_cast(bf16x8, __builtin_nontemporal_load(p + j));
  } else if constexpr (FMT == FMT_FP8) {
    const u32x4* p = reinterpret_cast<const u32x4*>(row + static_cast<size_t>(kb) * 128 + g * 32);
    const u32x4 v0 = __builtin_nontemporal_load(p);
    const u32x4 v1 = __builtin_nontemporal_load(p + 1);
    const uint32_t wds[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wds[2 * j], 1.0f, false);
      const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wds[2 * j], 1.0f, true);
      const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wds[2 * j + 1], 1.0f, false);
      const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wds[2 * j + 1], 1.0f, true);
      a[j] = bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    }
  } else {  // FMT_MXFP4
    const u32x4 v = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(row + (static_cast<size_t>(kb) * 128 + g * 32) / 2));
    const uint8_t code = static_cast<const uint8_t*>(sbase)[static_cast<size_t>(row_idx) * (K / 32) + kb * 4 + g];
    const float sc = __uint_as_float(static_cast<uint32_t>(code) << 23);
    const uint32_t wds[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wds[j], sc, 0);
      const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wds[j], sc, 1);
      const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wds[j], sc, 2);
      const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wds[j], sc, 3);
      a[j] = bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    }
  }
}

__device__ __forceinline__ void load_b(const uint16_t* row, int kb, int g, bf16x8 (&b)[4]) {
  const u32x4* p = reinterpret_cast<const u32x4*>(row + static_cast<size_t>(kb) * 128 + g * 32);
#pragma unroll
  for (int j = 0; j < 4; ++j) b[j] = __builtin_bit_cast(bf16x8, p[j]);
}

template <int FMT>
__device__ __forceinline__ float fp8_block_scale(const void* sbase, int row0, int N, int K, int kb) {
  if constexpr (FMT == FMT_FP8) {
    return static_cast<const float*>(sbase)[static_cast<size_t>(row0 / 128) * (K / 128) + kb];
  } else {
    return 1.0f;
  }
}

// Accumulates rows [row0, row0+16) of one matrix against up to kTch route chunks.
// NMAT = 2 processes a second matrix (up rows, offset by row_off) in the same pass.
template <int FMT, int NMAT>
__device__ __forceinline__ void gemv_tile(const uint8_t* wbase, const void* sbase, int N, int K, int row0,
                                          int row_off, const uint16_t* const* brow, int nch,
                                          f32x4 (&acc)[NMAT][kTch]) {
  const int lane = lane_id();
  const int r = lane & 15, g = lane >> 4;
  const int wave = threadIdx.x / kWave;
  const int nkb = K / 128;
  const size_t rb = row_bytes<FMT>(K);
  const uint8_t* rows[NMAT];
  int ridx[NMAT];
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    ridx[m] = row0 + r + m * row_off;
    rows[m] = wbase + static_cast<size_t>(ridx[m]) * rb;
  }
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int c = 0; c < kTch; ++c) acc[m][c] = zero;

  for (int kb = wave; kb < nkb; kb += kDecWaves) {
    bf16x8 a[NMAT][4];
#pragma unroll
    for (int m = 0; m < NMAT; ++m) load_a<FMT>(rows[m], sbase, ridx[m], K, kb, g, a[m]);
    bf16x8 b[kTch][4];
#pragma unroll
    for (int c = 0; c < kTch; ++c)
      if (c < nch) load_b(brow[c], kb, g, b[c]);
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
      const float sc = fp8_block_scale<FMT>(sbase, row0 + m * row_off, N, K, kb);
#pragma unroll
      for (int c = 0; c < kTch; ++c) {
        if (c < nch) {
          if constexpr (FMT == FMT_FP8) {
            f32x4 t = zero;
#pragma unroll
            for (int j = 0; j < 4; ++j) t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[m][j], b[c][j], t, 0, 0, 0);
            acc[m][c] += t * sc;
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[m][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[m][j], b[c][j], acc[m][c], 0, 0, 0);
          }
        }
      }
    }
  }
}

template <int FMT_R, int FMT_S, int STAGE>
__global__ void __launch_bounds__(kDecWaves * kWave) decode_stage_kernel(DecodeArgs a) {
  __shared__ f32x4 red[kDecWaves][2][kTch][kWave];
  const int seg = blockIdx.y;
  const bool shared = seg == a.max_seg;
  if (!shared && seg >= a.n_seg[0]) return;
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int r16 = lane & 15, g = lane >> 4;

  const int inter = shared ? a.Is : a.I;
  const int row0 = blockIdx.x * 16;
  if (STAGE == 0 && row0 >= inter) return;
  const int count = shared ? a.M : a.seg_count[seg];
  const int start = shared ? 0 : a.seg_start[seg];
  const int expert = shared ? 0 : a.seg_expert[seg];
  const BankView bank = STAGE == 0 ? (shared ? a.sh_gate_up : a.gate_up) : (shared ? a.sh_down : a.down);
  const int N = STAGE == 0 ? 2 * inter : a.H;
  const int K = STAGE == 0 ? a.H : inter;
  const int fmt = shared ? FMT_S : FMT_R;

  for (int pass = 0; pass * 16 * kTch < count; ++pass) {
    const int base = pass * 16 * kTch;
    const int nch = min(kTch, (count - base + 15) / 16);
    // B operand rows of this lane's route column in each chunk (clamped, masked later)
    const uint16_t* brow[kTch];
#pragma unroll
    for (int c = 0; c < kTch; ++c) {
      const int col = min(base + c * 16 + r16, count - 1);
      if (STAGE == 0) {
        const int tok = shared ? col : a.sorted[start + col] / a.k;
        brow[c] = a.x + static_cast<size_t>(tok) * a.H;
      } else {
        const int arow = shared ? a.M * a.k + col : a.sorted[start + col];
        brow[c] = a.act + static_cast<size_t>(arow) * a.act_stride;
      }
    }
    f32x4 acc[2][kTch];
    if (fmt == FMT_BF16) {
      if constexpr (FMT_R == FMT_BF16 || FMT_S == FMT_BF16) {
        const size_t eb = static_cast<size_t>(N) * row_bytes<FMT_BF16>(K);
        if (STAGE == 0) {
          f32x4 t[2][kTch];
          gemv_tile<FMT_BF16, 2>(bank.w + expert * eb, nullptr, N, K, row0, inter, brow, nch, t);
#pragma unroll
          for (int c = 0; c < kTch; ++c) { acc[0][c] = t[0][c]; acc[1][c] = t[1][c]; }
        } else {
          f32x4 t[1][kTch];
          gemv_tile<FMT_BF16, 1>(bank.w + expert * eb, nullptr, N, K, row0, 0, brow, nch, t);
#pragma unroll
          for (int c = 0; c < kTch; ++c) acc[0][c] = t[0][c];
        }
      }
    } else if (fmt == FMT_FP8) {
      if constexpr (FMT_R == FMT_FP8 || FMT_S == FMT_FP8) {
        const size_t eb = static_cast<size_t>(N) * K;
        const float* sb = static_cast<const float*>(bank.s) + static_cast<size_t>(expert) * (N / 128) * (K / 128);
        if (STAGE == 0) {
          f32x4 t[2][kTch];
          gemv_tile<FMT_FP8, 2>(bank.w + expert * eb, sb, N, K, row0, inter, brow, nch, t);
#pragma unroll
          for (int c = 0; c < kTch; ++c) { acc[0][c] = t[0][c]; acc[1][c] = t[1][c]; }
        } else {
          f32x4 t[1][kTch];
          gemv_tile<FMT_FP8, 1>(bank.w + expert * eb, sb, N, K, row0, 0, brow, nch, t);
#pragma unroll
          for (int c = 0; c < kTch; ++c) acc[0][c] = t[0][c];
        }
      }
    } else {
      if constexpr (FMT_R == FMT_MXFP4 || FMT_S == FMT_MXFP4) {
        const size_t eb = static_cast<size_t>(N) * (K / 2);
        const uint8_t* sb = static_cast<const uint8_t*>(bank.s) + static_cast<size_t>(expert) * N * (K / 32);
        if (STAGE == 0) {
          f32x4 t[2][kTch];
          gemv_tile<FMT_MXFP4, 2>(bank.w + expert * eb, sb, N, K, row0, inter, brow, nch, t);
#pragma unroll
          for (int c = 0; c < kTch; ++c) { acc[0][c] = t[0][c]; acc[1][c] = t[1][c]; }
        } else {
          f32x4 t[1][kTch];
          gemv_tile<FMT_MXFP4, 1>(bank.w + expert * eb, sb, N, K, row0, 0, brow, nch, t);
#pragma unroll
          for (int c = 0; c < kTch; ++c) acc[0][c] = t[0][c];
        }
      }
    }
    // ---- split-K reduction in fixed wave order
    constexpr int NM = STAGE == 0 ? 2 : 1;
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int c = 0; c < kTch; ++c)
        if (c < nch) red[wave][m][c][lane] = acc[m][c];
    __syncthreads();
    if (wave < nch) {
      const int c = wave;
      f32x4 s[NM];
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        s[m] = red[0][m][c][lane];
#pragma unroll
        for (int v = 1; v < kDecWaves; ++v) s[m] += red[v][m][c][lane];
      }
      const int col = base + c * 16 + r16;
      if (col < count) {
        const int rows_at = row0 + g * 4;  // this lane's 4 consecutive output rows
        uint16_t o[4];
        if (STAGE == 0) {
          const int route = shared ? -1 : a.sorted[start + col];
          const float win = (!shared && a.weight_on_input) ? a.topk_w[route] : 1.0f;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float gg = bf16_round(s[0][v] * win);
            const float uu = bf16_round(s[1][v] * win);
            o[v] = f32_to_bf16(act_apply(a.act_kind, gg) * uu);
          }
          const int arow = shared ? a.M * a.k + col : route;
          uint2 pk;
          pk.x = static_cast<uint32_t>(o[0]) | (static_cast<uint32_t>(o[1]) << 16);
          pk.y = static_cast<uint32_t>(o[2]) | (static_cast<uint32_t>(o[3]) << 16);
          *reinterpret_cast<uint2*>(a.act + static_cast<size_t>(arow) * a.act_stride + rows_at) = pk;
        } else {
          uint16_t* dst;
          float wt = 1.0f;
          if (shared) {
            dst = a.sh_out + static_cast<size_t>(col) * a.H + rows_at;
          } else {
            const int route = a.sorted[start + col];
            if (!a.weight_on_input) wt = a.topk_w[route];
            dst = a.ic3 + static_cast<size_t>(route) * a.H + rows_at;
          }
#pragma unroll
          for (int v = 0; v < 4; ++v) o[v] = f32_to_bf16(s[0][v] * wt);
          uint2 pk;
          pk.x = static_cast<uint32_t>(o[0]) | (static_cast<uint32_t>(o[1]) << 16);
          pk.y = static_cast<uint32_t>(o[2]) | (static_cast<uint32_t>(o[3]) << 16);
          *reinterpret_cast<uint2*>(dst) = pk;
        }
      }
    }
    __syncthreads();
  }
}

// y[t] = bf16( bf16(sum_r ic3[t,r]) + sh_out[t] ), routes with ids outside
// [0, num_rows) skipped; sum in route order r = 0..k-1 in float32 (reference
// moe_sum_reduce_kernel, kernel/triton/fused_moe.py:142-153).
__global__ void __launch_bounds__(256) combine_kernel(const uint16_t* __restrict__ ic3,
                                                      const int32_t* __restrict__ ids, int num_rows,
                                                      const uint16_t* __restrict__ sh_out, int M, int k, int H,
                                                      uint16_t* __restrict__ y) {
  const int per_tok = H / 8;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * per_tok) return;
  const int t = idx / per_tok;
  const int h = (idx - t * per_tok) * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int r = 0; r < k; ++r) {
    const int e = ids[t * k + r];
    if (e < 0 || e >= num_rows) continue;
    const uint4 v = *reinterpret_cast<const uint4*>(ic3 + static_cast<size_t>(t * k + r) * H + h);
    const uint32_t wds[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += bf16_to_f32(static_cast<uint16_t>(wds[q] & 0xffffu));
      acc[2 * q + 1] += bf16_to_f32(static_cast<uint16_t>(wds[q] >> 16));
    }
  }
  uint16_t o[8];
  if (sh_out) {
    const uint4 v = *reinterpret_cast<const uint4*>(sh_out + static_cast<size_t>(t) * H + h);
    const uint32_t wds[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      o[2 * q] = f32_to_bf16(bf16_round(acc[2 * q]) + bf16_to_f32(static_cast<uint16_t>(wds[q] & 0xffffu)));
      o[2 * q + 1] = f32_to_bf16(bf16_round(acc[2 * q + 1]) + bf16_to_f32(static_cast<uint16_t>(wds[q] >> 16)));
    }
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q) o[q] = f32_to_bf16(acc[q]);
  }
  uint4 out;
  out.x = o[0] | (static_cast<uint32_t>(o[1]) << 16);
  out.y = o[2] | (static_cast<uint32_t>(o[3]) << 16);
  out.z = o[4] | (static_cast<uint32_t>(o[5]) << 16);
  out.w = o[6] | (static_cast<uint32_t>(o[7]) << 16);
  *reinterpret_cast<uint4*>(y + static_cast<size_t>(t) * H + h) = out;
}

template <int FR, int FS>
static hipError_t launch_stage_t(int stage, const DecodeArgs& a, bool has_shared, hipStream_t stream) {
  const int gy = a.max_seg + (has_shared ? 1 : 0);
  const int imax = has_shared ? max(a.I, a.Is) : a.I;
  if (stage == 0)
    hipLaunchKernelGGL((decode_stage_kernel<FR, FS, 0>), dim3(imax / 16, gy), dim3(kDecWaves * kWave), 0, stream, a);
  else
    hipLaunchKernelGGL((decode_stage_kernel<FR, FS, 1>), dim3(a.H / 16, gy), dim3(kDecWaves * kWave), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_decode_stage(int stage, int fmt_r, int fmt_s, const DecodeArgs& a, hipStream_t stream) {
  const bool sh = fmt_s != FMT_NONE;
  const int fs = sh ? fmt_s : fmt_r;  // FMT_S is unused without a shared expert
#define FTMOE_CASE(R, S) \
  if (fmt_r == R && fs == S) return launch_stage_t<R, S>(stage, a, sh, stream);
  FTMOE_CASE(FMT_BF16, FMT_BF16)
  FTMOE_CASE(FMT_BF16, FMT_FP8)
  FTMOE_CASE(FMT_BF16, FMT_MXFP4)
  FTMOE_CASE(FMT_FP8, FMT_BF16)
  FTMOE_CASE(FMT_FP8, FMT_FP8)
  FTMOE_CASE(FMT_FP8, FMT_MXFP4)
  FTMOE_CASE(FMT_MXFP4, FMT_BF16)
  FTMOE_CASE(FMT_MXFP4, FMT_FP8)
  FTMOE_CASE(FMT_MXFP4, FMT_MXFP4)
#undef FTMOE_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_combine(const uint16_t* ic3, const int32_t* ids, int num_rows, const uint16_t* sh_out, int M,
                          int k, int H, uint16_t* y, hipStream_t stream) {
  const int n = M * (H / 8);
  hipLaunchKernelGGL(combine_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, ic3, ids, num_rows, sh_out, M, k,
                     H, y);
  return hipGetLastError();
}

}  // namespace ftmoe
