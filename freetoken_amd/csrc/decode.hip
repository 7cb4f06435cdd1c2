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
// 128-wide K block, 32 of its K values: four MFMAs of 8 values each, placed by
// k_first() below.  A and B use the same K placement, so the products pair up
// no matter how the hardware orders K inside an MFMA.
//
// The 4 waves of a workgroup split K (wave w takes a contiguous quarter of the
// K blocks), and their partial sums are reduced through LDS in fixed wave
// order, so results are deterministic.  Without a K split (the down stage, and
// gate_up of large FP8 calls) every wave walks the whole K range over its own
// rows, and the waves share the activation chunks through an LDS ring.
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
#include "align_wave.h"
#include "kernels.h"
#include "route_token.h"

namespace ftmoe {

constexpr int kDecWaves = 4;  // waves per workgroup (K split)

template <int FMT>
__device__ __forceinline__ size_t row_bytes(int K) {
  return FMT == FMT_BF16 ? static_cast<size_t>(K) * 2 : FMT == FMT_FP8 ? static_cast<size_t>(K) : static_cast<size_t>(K) / 2;
}

// K placement inside a 128-wide K block: MFMA j (0..3) of lane group g = l/16
// takes the 8 values starting at
//   BF16   32j + 8g                 weights and activations: 16-byte pieces
//                                   at 64j + 16g, one whole 64-byte line of a
//                                   row per load instruction
//   FP8    64(j/2) + 16g + 8(j%2)   weights (from LDS, see dma_compute): the
//                                   16 bytes at 64i + 16g feed MFMAs 2i, 2i+1;
//                                   activations: 128(j/2) + 32g + 16(j%2)
//                                   (measured faster than 32j + 8g here)
//   MXFP4  32g + 8j                 a lane group's 32 values share one e8m0
//                                   scale; weights: 16 bytes at 16g
// The weight side of a lane group starts a_group_bytes * g into the K block's
// row slice; the activation piece of MFMA j sits at
// g * b_group_bytes + b_piece_bytes(j).
template <int FMT>
constexpr uint32_t a_group_bytes() {
  return 16;
}
template <int FMT>
constexpr uint32_t b_group_bytes() {
  return FMT == FMT_BF16 ? 16 : FMT == FMT_FP8 ? 32 : 64;
}
template <int FMT>
constexpr uint32_t b_piece_bytes(int j) {
  return FMT == FMT_BF16 ? 64 * j : FMT == FMT_FP8 ? 128 * (j >> 1) + 16 * (j & 1) : 16 * j;
}

// Raw (still quantised) A-operand bytes of one lane for one 128-wide K block.
template <int FMT>
struct RawA;
template <>
struct RawA<FMT_BF16> {
  bf16x8 v[4];
};
template <>
struct RawA<FMT_FP8> {
  u32x4 v[2];
};
template <>
struct RawA<FMT_MXFP4> {
  u32x4 v[1];
  uint32_t code;
};

// Weights and activations are read through buffer descriptors (make_rsrc,
// buf_x4): base in SGPRs, 32-bit lane offsets, the K-block offset in soffset.

// Weight bytes of one lane for K block kb: the lane's row starts at voff
// (row * row_bytes + a_group_bytes * lane group); the K block adds kb * 128
// values.  MXFP4: the lane's e8m0 code sits at coff + kb * 4 of the
// code rows (sr).  `dead` is 0 or kOutOfRange: a dead K block (past the wave's
// range) is still issued, so every K step issues the same loads and the
// wait counts stay exact, but it reads zeros without touching memory.
template <int FMT>
__device__ __forceinline__ void load_raw(__amdgpu_buffer_rsrc_t wr, __amdgpu_buffer_rsrc_t sr, uint32_t voff,
                                         uint32_t coff, int kb, uint32_t dead, RawA<FMT>& r) {
  if constexpr (FMT == FMT_BF16) {
    const uint32_t so = static_cast<uint32_t>(kb) * 256;
#pragma unroll
    for (int j = 0; j < 4; ++j) r.v[j] = __builtin_bit_cast(bf16x8, buf_x4(wr, (voff | dead) + 64 * j, so));
  } else {
    static_assert(FMT == FMT_MXFP4, "FP8 weights take the LDS path (gemv_tile_dma)");
    r.v[0] = buf_x4(wr, voff | dead, static_cast<uint32_t>(kb) * 64);
    r.code = buf_u8(sr, coff | dead, static_cast<uint32_t>(kb) * 4);
  }
}

// Dequantises raw bytes into four bf16x8 MFMA operands (exact conversions).
template <int FMT>
__device__ __forceinline__ void dequant(const RawA<FMT>& r, bf16x8 (&a)[4]) {
  if constexpr (FMT == FMT_BF16) {
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = r.v[j];
  } else if constexpr (FMT == FMT_FP8) {
    const uint32_t wds[8] = {r.v[0][0], r.v[0][1], r.v[0][2], r.v[0][3], r.v[1][0], r.v[1][1], r.v[1][2], r.v[1][3]};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wds[2 * j], 1.0f, false);
      const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wds[2 * j], 1.0f, true);
      const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wds[2 * j + 1], 1.0f, false);
      const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(wds[2 * j + 1], 1.0f, true);
      a[j] = bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    }
  } else {
    const float sc = __uint_as_float(r.code << 23);  // 2^(code-127), exact for codes >= 1
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = r.v[0][j];
      const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0);
      const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1);
      const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2);
      const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3);
      a[j] = bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    }
  }
}

// Registers of one K block in flight: NMAT weight tiles and NCH activation chunks.
template <int FMT, int NMAT, int NCH>
struct KStage {
  RawA<FMT> w[NMAT];
  u32x4 b[NCH][4];
  float sc[NMAT];  // FP8: the 128x128 block scale of each tile for this K block
};

// Lanes whose route column lies past the segment's end carry kOutOfRange and
// read zeros (MFMA output column c depends on B column c only, and those
// columns are never stored).
// Weight-side addressing of one wave: the expert's matrix (wr), each tile's
// lane offset (wvoff), and the scales: FP8 the expert's scale array sr with
// each tile's scale row at soff (wave-uniform); MXFP4 the expert's e8m0 code
// rows sr with the lane's row and lane group at soff.
template <int NMAT>
struct WTiles {
  __amdgpu_buffer_rsrc_t wr, sr;
  uint32_t wvoff[NMAT];
  uint32_t soff[NMAT];
};

template <int FMT, int NMAT, int NCH>
__device__ __forceinline__ void load_stage(KStage<FMT, NMAT, NCH>& st, const WTiles<NMAT>& wt,
                                           __amdgpu_buffer_rsrc_t br, const uint32_t (&bvoff)[NCH], int kb,
                                           uint32_t dead) {
#pragma unroll
  for (int m = 0; m < NMAT; ++m) load_raw<FMT>(wt.wr, wt.sr, wt.wvoff[m], wt.soff[m], kb, dead, st.w[m]);
  if constexpr (FMT == FMT_FP8) {
    // wave-uniform address: one request per tile, in flight with the weights
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
      st.sc[m] = buf_f32(wt.sr, wt.soff[m] | dead, static_cast<uint32_t>(kb) * 4);
  }
  const uint32_t so = static_cast<uint32_t>(kb) * 256;
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int j = 0; j < 4; ++j) st.b[c][j] = buf_x4(br, (bvoff[c] | dead) + b_piece_bytes<FMT>(j), so);
}

template <int FMT, int NMAT, int NCH>
__device__ __forceinline__ void compute_stage(const KStage<FMT, NMAT, NCH>& st, f32x4 (&acc)[NMAT][NCH]) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    bf16x8 a[4];
    if constexpr (FMT == FMT_BF16) {
#pragma unroll
      for (int j = 0; j < 4; ++j) a[j] = st.w[m].v[j];  // element-wise: no aggregate copy
    } else {
      dequant<FMT>(st.w[m], a);
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if constexpr (FMT == FMT_FP8) {
        f32x4 t = zero;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j], __builtin_bit_cast(bf16x8, st.b[c][j]), t, 0, 0, 0);
        acc[m][c] += t * st.sc[m];
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[m][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j], __builtin_bit_cast(bf16x8, st.b[c][j]), acc[m][c],
                                                              0, 0, 0);
      }
    }
  }
}

// K stages kept in flight: as many as fit next to the accumulators in the
// 256 registers of occupancy 2 (a stage holds NMAT weight tiles, their scales
// and NCH activation chunks), between 2 and 4.
template <int FMT, int NMAT, int NCH>
constexpr int pipeline_depth() {
  constexpr int wregs = FMT == FMT_BF16 ? 16 : FMT == FMT_FP8 ? 8 : 4;
  constexpr int per_stage = NMAT * (wregs + 1) + NCH * 16;
  constexpr int fit = (200 - NMAT * NCH * 4 - 24) / per_stage;
  return fit < 2 ? 2 : fit > 4 ? 4 : fit;
}

// Accumulates NMAT 16-row weight tiles against NCH route chunks of 16 over the
// K blocks [kw*nkb/KS, (kw+1)*nkb/KS) (contiguous per wave) through a ring of
// S register stages: the loads of the next S-1 K blocks are in flight while one
// is computed.  Every step issues its loads (dead ones read zeros), so the
// hardware counters wait for exactly the stage about to be used.
template <int FMT, int NMAT, int NCH, int KS>
__device__ __forceinline__ void gemv_tile(const WTiles<NMAT>& wt, int K, int kw, __amdgpu_buffer_rsrc_t br,
                                          const uint32_t (&bvoff)[NCH], f32x4 (&acc)[NMAT][NCH]) {
  constexpr int S = pipeline_depth<FMT, NMAT, NCH>();
  const int nkb = K / 128;
  const int kb_lo = kw * nkb / KS, kb_hi = (kw + 1) * nkb / KS;
  const int n = kb_hi - kb_lo;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int c = 0; c < NCH; ++c) acc[m][c] = zero;
  KStage<FMT, NMAT, NCH> st[S];
#pragma unroll
  for (int s = 0; s < S - 1; ++s) load_stage(st[s], wt, br, bvoff, kb_lo + s, s < n ? 0u : kOutOfRange);
  // whole groups of S steps: loads and computes unconditional
  int i = 0;
  for (; i + S <= n; i += S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int ahead = i + s + S - 1;
      load_stage(st[(s + S - 1) % S], wt, br, bvoff, kb_lo + ahead, ahead < n ? 0u : kOutOfRange);
      // loads leave in the order the stages are consumed (the counter is
      // in order): keep the scheduler from mixing one step's loads into another's
      __builtin_amdgcn_sched_barrier(0);
      compute_stage(st[s], acc);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // the last n - i < S blocks are already in stages 0.. (loaded above or in
  // the prologue)
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    if (i + s < n) compute_stage(st[s], acc);
}

// Quantised weights (FP8, MXFP4) stream through LDS instead of registers.  A
// register load instruction can cover at most 64 bytes of a row (4 lanes of
// 16 bytes share a row in the MFMA operand layout), so the two halves of each
// 128-byte line are fetched by different instructions and the line has to
// stay in L2 between them.  A DMA instruction (buffer load to LDS) is free to
// give its 64 lanes 8 whole rows: each fetches complete lines, which lets the
// weights use the nontemporal policy (measured on MI355X: 7.1 TB/s against
// 6.2 TB/s for the default policy on a plain stream).  A K step covers 128
// bytes of every row: one K block of FP8, two of MXFP4.  Each wave owns a ring
// of stages in LDS (dma_depth); a stage holds NMAT tiles of 16 rows x 128
// bytes.  Chunk c (16 bytes) of tile row r lands at slot c ^ (r & 7) of the
// row, spreading the operand reads over the LDS banks.  A lane's operands are
// chunks g and 4 + g of its row: FP8 values 16g.. and 64 + 16g.. of the K
// block (MFMAs 0, 1 and 2, 3); MXFP4 values 32g.. of the first and of the
// second K block of the step.
constexpr int kTileBytes = 16 * 128;
constexpr int kNtPolicy = 2;  // cache policy bits of a nontemporal load

template <int FMT>
constexpr int dma_kstep() {  // K values per step
  return FMT == FMT_FP8 ? 128 : 256;
}
template <int FMT>
constexpr int dma_pieces() {  // activation loads (16 bytes) per chunk and step
  return FMT == FMT_FP8 ? 4 : 8;
}
template <int FMT, int NMAT, int NCH, bool CT = false>
constexpr int dma_per_step() {  // vector memory instructions of one dma_issue (CT: codes from the LDS table)
  return (CT ? 2 : 3) * NMAT + dma_pieces<FMT>() * NCH;
}

// Per-step side data of a tile: FP8 the 128x128 block scale (wave-uniform);
// MXFP4 the lane's row of e8m0 codes for the step's two K blocks (byte g of
// each word is the lane group's code).
template <int FMT>
struct DmaSide;
template <>
struct DmaSide<FMT_FP8> {
  float s;
};
template <>
struct DmaSide<FMT_MXFP4> {
  uint2 codes;
};

template <int NMAT>
struct DmaTiles {
  __amdgpu_buffer_rsrc_t wr, sr;
  uint32_t voff[NMAT][2];  // lane's DMA source in instruction h (rows 8h..8h+7) of tile m
  uint32_t soff[NMAT];     // FP8: tile's scale row (wave-uniform); MXFP4: lane's code row
};

// CW: the weights are read more than once by nearby workgroups (the shared
// expert's token pieces): the default policy instead of the nontemporal one,
// so that the later readers find the lines in L2.
template <bool CW = false>
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0,
                                           CW ? 0 : kNtPolicy);
}

__device__ __forceinline__ void lds_dma16_cached(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

template <int FMT, int NMAT, int NCH, bool CT = false, bool CW = false>
__device__ __forceinline__ void dma_issue(const DmaTiles<NMAT>& dt, __amdgpu_buffer_rsrc_t br,
                                          const uint32_t (&bvoff)[NCH], uint8_t* stage, int step, uint32_t dead,
                                          u32x4 (&b)[NCH][dma_pieces<FMT>()], DmaSide<FMT> (&side)[NMAT]) {
  const uint32_t so = static_cast<uint32_t>(step) * 128;
#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int h = 0; h < 2; ++h) lds_dma16<CW>(dt.wr, stage + m * kTileBytes + h * 1024, dt.voff[m][h] | dead, so);
  if constexpr (!CT) {
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
      if constexpr (FMT == FMT_FP8)
        side[m].s = buf_f32(dt.sr, dt.soff[m] | dead, static_cast<uint32_t>(step) * 4);
      else
        side[m].codes = buf_x2(dt.sr, dt.soff[m] | dead, static_cast<uint32_t>(step) * 8);
    }
  }
  const uint32_t sb = static_cast<uint32_t>(step) * dma_kstep<FMT>() * 2;
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int j = 0; j < dma_pieces<FMT>(); ++j) {
      const uint32_t piece = FMT == FMT_FP8 ? b_piece_bytes<FMT_FP8>(j) : 256 * (j >> 2) + b_piece_bytes<FMT_MXFP4>(j & 3);
      b[c][j] = buf_x4(br, (bvoff[c] | dead) + piece, sb);
    }
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// s_barrier without the release fence of __syncthreads (which would wait for
// every copy in flight); the clobber keeps LDS accesses on their side of it.
__device__ __forceinline__ void bare_barrier_dec() { asm volatile("s_barrier" ::: "memory"); }

// One step of one stage: operands from LDS at rd0, rd1 (chunks g and 4 + g of
// row r16), dequantised exactly to bf16, then the MFMAs (FP8: the block scale
// folds each K block's partial into acc; MXFP4: the e8m0 scale is exact in the
// dequant, acc chains through both K blocks in order).
template <int FMT, int NMAT, int NCH>
__device__ __forceinline__ void dma_compute(const uint8_t* stage, uint32_t rd0, uint32_t rd1, int gsh,
                                            const u32x4 (&b)[NCH][dma_pieces<FMT>()],
                                            const DmaSide<FMT> (&side)[NMAT], f32x4 (&acc)[NMAT][NCH]) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  u32x4 w0[NMAT], w1[NMAT];
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    w0[m] = *reinterpret_cast<const u32x4*>(stage + m * kTileBytes + rd0);
    w1[m] = *reinterpret_cast<const u32x4*>(stage + m * kTileBytes + rd1);
  }
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    if constexpr (FMT == FMT_FP8) {
      RawA<FMT_FP8> r;
      r.v[0] = w0[m];
      r.v[1] = w1[m];
      bf16x8 a[4];
      dequant<FMT_FP8>(r, a);
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        f32x4 t = zero;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[j], __builtin_bit_cast(bf16x8, b[c][j]), t, 0, 0, 0);
        acc[m][c] += t * side[m].s;
      }
    } else {
#pragma unroll
      for (int blk = 0; blk < 2; ++blk) {
        RawA<FMT_MXFP4> r;
        r.v[0] = blk == 0 ? w0[m] : w1[m];
        r.code = ((blk == 0 ? side[m].codes.x : side[m].codes.y) >> gsh) & 0xffu;
        bf16x8 a[4];
        dequant<FMT_MXFP4>(r, a);
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[m][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                a[j], __builtin_bit_cast(bf16x8, b[c][4 * blk + j]), acc[m][c], 0, 0, 0);
      }
    }
  }
}

// MXFP4 with a K split (the gate_up stage): the e8m0 codes of the workgroup's
// NMAT tiles (16 rows each, K/32 bytes per row) are copied into LDS once per
// pass, a few 1 KB DMA instructions per wave, instead of one 8-byte load per
// tile and step whose 64 lanes gather from 16 rows.  Measured on C3 and C4
// shapes: those per-step loads cost 18% of the MXFP4 gate_up stage.  Each
// wave reads its codes for step st from LDS: row r of tile m at
// (16 m + r) * K/32 + 8 st, the same two words the per-step load returned.
constexpr int kCodeTableBytes = 16384;
template <int NMAT>
__device__ __forceinline__ bool code_table_fits(int K) {
  return K % 512 == 0 && NMAT * 16 * (K / 32) <= kCodeTableBytes;
}

// Copies the table (NMAT * 16 rows of K/32 bytes) into ctab.  The tiles are
// the gate_up stage's: table rows [0, 16 RT) are weight rows wrow0.. (gate),
// the next 16 RT rows are inter + wrow0.. (up).  Instruction q of the
// workgroup covers table bytes [1024 q, 1024 q + 1024) and is issued by wave
// q % kDecWaves; lanes past the table read zeros (the region is
// kCodeTableBytes long).  The row is computed, not looked up, so that no
// per-lane index reaches memory.
template <int RT>
__device__ __forceinline__ void code_table_fill(__amdgpu_buffer_rsrc_t sr, int K, int wrow0, int inter, int wave,
                                                uint8_t* ctab) {
  const int rb = K / 32, bytes = 2 * RT * 16 * rb, lane = lane_id();
  for (int q = wave; q * 1024 < bytes; q += kDecWaves) {
    const int b = q * 1024 + lane * 16;
    uint32_t src = kOutOfRange;
    if (b < bytes) {
      const int row = b / rb, off = b - row * rb;
      const int grow = row < 16 * RT ? wrow0 + row : inter + wrow0 + row - 16 * RT;
      src = static_cast<uint32_t>(grow) * rb + off;
    }
    lds_dma16_cached(sr, ctab + q * 1024, src, 0);
  }
}

// The codes of step st for the lane's row of each tile (ctl: the lane's row
// r16 of tile 0; ctile: bytes per tile, 16 * K/32).  ctl is __restrict__: with
// that alias information the compiler does not make these reads wait for the
// weight copies (LDS DMA) in flight, which without it it must assume may
// write the same LDS.
template <int NMAT>
__device__ __forceinline__ void code_table_side(const uint8_t* __restrict__ ctl, uint32_t ctile, int st,
                                                DmaSide<FMT_MXFP4> (&sd)[NMAT]) {
#pragma unroll
  for (int m = 0; m < NMAT; ++m) sd[m].codes = *reinterpret_cast<const uint2*>(ctl + m * ctile + 8 * st);
}

// Computes the stages T.. of the last `left` steps of a ring of S stages,
// waiting for each stage alone (the S-2-T stages behind it stay in flight).
template <int FMT, int S, int T, int NMAT, int NCH, bool CT = false>
__device__ __forceinline__ void dma_tail(int left, const uint8_t* ring, uint32_t rd0, uint32_t rd1, int gsh,
                                         const u32x4 (&b)[S][NCH][dma_pieces<FMT>()],
                                         const DmaSide<FMT> (&side)[S][NMAT], f32x4 (&acc)[NMAT][NCH],
                                         const uint8_t* ctl = nullptr, uint32_t ctile = 0, int st0 = 0) {
  if constexpr (T < S - 1) {
    if (left > T) {
      wait_vmcnt<(S - 2 - T) * dma_per_step<FMT, NMAT, NCH, CT>()>();
      if constexpr (CT) {
        DmaSide<FMT> sd[NMAT];
        code_table_side<NMAT>(ctl, ctile, st0 + T, sd);
        dma_compute<FMT, NMAT, NCH>(ring + T * NMAT * kTileBytes, rd0, rd1, gsh, b[T], sd, acc);
      } else {
        dma_compute<FMT, NMAT, NCH>(ring + T * NMAT * kTileBytes, rd0, rd1, gsh, b[T], side[T], acc);
      }
      dma_tail<FMT, S, T + 1, NMAT, NCH, CT>(left, ring, rd0, rd1, gsh, b, side, acc, ctl, ctile, st0);
    }
  }
}

// Ring depth of the LDS path: 2 stages of 4 tiles (64 KiB of LDS per
// workgroup, two resident per CU) or 3 stages of 2 (FP8 measured against 2
// and 4: 3 is the fastest at b = 1 and no slower at b = 8 and 64; MXFP4 keeps
// 2 when two route chunks make a stage's registers large).
// The wide kernels of large FP8 calls (passes of up to four route chunks)
// keep 2 stages for every pass, so that their LDS stays at 80 KB.
template <int FMT, int NMAT, int NCH, int WIDE = 0>
constexpr int dma_depth() {
  return (WIDE || NMAT >= 4 || NCH >= 4) ? 2 : (FMT == FMT_MXFP4 && NCH > 1) ? 2 : 3;
}
template <int FMT, int NMAT, int WIDE = 0>
constexpr int dma_ring_bytes() {  // per wave, the larger of the NCH variants (WIDE: 2 stages for all)
  if constexpr (WIDE) return dma_depth<FMT, NMAT, 4, 1>() * NMAT * kTileBytes;
  return (dma_depth<FMT, NMAT, 1>() > dma_depth<FMT, NMAT, 2>() ? dma_depth<FMT, NMAT, 1>()
                                                                  : dma_depth<FMT, NMAT, 2>()) *
         NMAT * kTileBytes;
}

// Counterpart of gemv_tile for FP8 and MXFP4: the same K range and
// accumulation order, the weights through the wave's LDS ring of S stages (the
// DMA of the next S-1 steps is in flight while one is computed; a dead step
// still issues, reading zeros, so every step's wait count is exact).
template <int FMT, int NMAT, int NCH, int KS, bool CT = false, bool CW = false>
__device__ __forceinline__ void gemv_tile_dma(const DmaTiles<NMAT>& dt, int K, int kw, __amdgpu_buffer_rsrc_t br,
                                              const uint32_t (&bvoff)[NCH], uint8_t* ring,
                                              f32x4 (&acc)[NMAT][NCH], uint8_t* ctab = nullptr, int wrow0 = 0,
                                              int inter = 0) {
  static_assert(!CT || (FMT == FMT_MXFP4 && KS == kDecWaves && NMAT % 2 == 0),
                "the code table serves the MXFP4 gate_up stage with one row group");
  constexpr int S = dma_depth<FMT, NMAT, NCH>();
  constexpr int P = dma_pieces<FMT>();
  constexpr int kStage = NMAT * kTileBytes;
  const int lane = lane_id(), r16 = lane & 15, g = lane >> 4;
  const uint32_t rd0 = r16 * 128 + ((g ^ (r16 & 7)) << 4);
  const uint32_t rd1 = r16 * 128 + (((4 + g) ^ (r16 & 7)) << 4);
  const int gsh = 8 * g;
  const int nst = K / dma_kstep<FMT>();
  const int st_lo = kw * nst / KS, st_hi = (kw + 1) * nst / KS;
  const int n = st_hi - st_lo;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int c = 0; c < NCH; ++c) acc[m][c] = zero;
  u32x4 b[S][NCH][P];
  DmaSide<FMT> side[S][NMAT];  // unused with the code table
  const uint32_t ctile = 16 * static_cast<uint32_t>(K / 32);
  const uint8_t* ctl = ctab + r16 * (K / 32);
  if constexpr (CT) code_table_fill<NMAT / 2>(dt.sr, K, wrow0, inter, kw, ctab);
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    dma_issue<FMT, NMAT, NCH, CT, CW>(dt, br, bvoff, ring + s * kStage, st_lo + s, s < n ? 0u : kOutOfRange, b[s],
                                  side[s]);
  DmaSide<FMT> nx[NMAT];  // the code table: codes of the next step
  if constexpr (CT) {
    // the table copies were issued first: wait for them alone, then make
    // every wave's copies visible
    wait_vmcnt<(S - 1) * dma_per_step<FMT, NMAT, NCH, CT>()>();
    bare_barrier_dec();
    code_table_side<NMAT>(ctl, ctile, st_lo, nx);
  }
  int i = 0;
  for (; i + S <= n; i += S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int ahead = i + s + S - 1;
      dma_issue<FMT, NMAT, NCH, CT, CW>(dt, br, bvoff, ring + ((s + S - 1) % S) * kStage, st_lo + ahead,
                                    ahead < n ? 0u : kOutOfRange, b[(s + S - 1) % S], side[(s + S - 1) % S]);
      wait_vmcnt<(S - 1) * dma_per_step<FMT, NMAT, NCH, CT>()>();
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (CT) {
        // this step's codes were read during the previous one; read the next
        // step's now (the scheduling barriers keep them in this step)
        DmaSide<FMT> sd[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m) sd[m] = nx[m];
        code_table_side<NMAT>(ctl, ctile, min(st_lo + i + s + 1, st_hi - 1), nx);
        dma_compute<FMT, NMAT, NCH>(ring + s * kStage, rd0, rd1, gsh, b[s], sd, acc);
      } else {
        dma_compute<FMT, NMAT, NCH>(ring + s * kStage, rd0, rd1, gsh, b[s], side[s], acc);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // the last n - i < S steps sit in stages 0.. (loaded above)
  dma_tail<FMT, S, 0, NMAT, NCH, CT>(n - i, ring, rd0, rd1, gsh, b, side, acc, ctl, ctile, st_lo + i);
}

// ---- Down stage: activations shared through LDS ----------------------------
// In the down stage (KS = 1) the 4 waves of a workgroup walk the same K range
// with the same route columns, so the activation chunks of a step are copied
// once per workgroup (each wave DMAs a quarter of the columns) into a shared
// ring of S + 1 slots instead of being loaded by every wave (measured: the
// per-wave activation loads cost ~12% of the b = 64 down kernel).  A slot
// holds NCH chunks of 16 columns x CB bytes (the step's K values in bf16);
// 16-byte piece p of column c sits at slot position p ^ c, so the 16 columns
// of one MFMA operand read hit distinct banks.  One barrier per step makes
// every wave's copies visible; the extra slot means a refill never lands on a
// slot another wave may still be reading (it was last read two steps before).
template <int FMT>
constexpr int act_col_bytes() {
  return dma_kstep<FMT>() * 2;
}
template <int FMT>
constexpr int act_copies() {  // 1 KB copies per wave per chunk and step
  return 16 * act_col_bytes<FMT>() / 1024 / kDecWaves;
}
template <int FMT, int NCH>
constexpr int act_slot_bytes() {
  return NCH * 16 * act_col_bytes<FMT>();
}
template <int FMT, int NMAT, int NCH, bool CR = false>
constexpr int sh_per_step() {  // vector memory instructions of one sh_issue (CR: codes in registers)
  return (CR ? 2 : 3) * NMAT + NCH * act_copies<FMT>();
}
template <int FMT, int NMAT, int CMAX>
constexpr int sh_act_ring_bytes() {  // the larger of the NCH variants up to CMAX chunks per pass (4: wide kernels)
  if constexpr (CMAX == 4) return (dma_depth<FMT, NMAT, 4, 1>() + 1) * act_slot_bytes<FMT, 4>();
  constexpr int one = (dma_depth<FMT, NMAT, 1>() + 1) * act_slot_bytes<FMT, 1>();
  constexpr int two = (dma_depth<FMT, NMAT, 2>() + 1) * act_slot_bytes<FMT, 2>();
  return CMAX == 1 || one > two ? one : two;
}


template <int FMT, int NMAT, int NCH, bool CR = false, bool CW = false>
__device__ __forceinline__ void sh_issue(const DmaTiles<NMAT>& dt, __amdgpu_buffer_rsrc_t br,
                                         const uint32_t (&avoff)[NCH][act_copies<FMT>()], uint8_t* wstage,
                                         uint8_t* aslot, int wave, int step, uint32_t dead,
                                         DmaSide<FMT> (&side)[NMAT]) {
  constexpr int CB = act_col_bytes<FMT>();
  const uint32_t so = static_cast<uint32_t>(step) * 128;
#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int h = 0; h < 2; ++h) lds_dma16<CW>(dt.wr, wstage + m * kTileBytes + h * 1024, dt.voff[m][h] | dead, so);
  if constexpr (!CR) {
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
      if constexpr (FMT == FMT_FP8)
        side[m].s = buf_f32(dt.sr, dt.soff[m] | dead, static_cast<uint32_t>(step) * 4);
      else
        side[m].codes = buf_x2(dt.sr, dt.soff[m] | dead, static_cast<uint32_t>(step) * 8);
    }
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int v = 0; v < act_copies<FMT>(); ++v)
      lds_dma16_cached(br, aslot + c * 16 * CB + (wave * act_copies<FMT>() + v) * 1024, avoff[c][v] | dead,
                       static_cast<uint32_t>(step) * CB);
}

template <int FMT, int NMAT, int NCH>
__device__ __forceinline__ void sh_compute(const uint8_t* wstage, const uint8_t* aslot, uint32_t rd0, uint32_t rd1,
                                           int r16, int g, const DmaSide<FMT> (&side)[NMAT],
                                           f32x4 (&acc)[NMAT][NCH]) {
  constexpr int CB = act_col_bytes<FMT>();
  constexpr int P = dma_pieces<FMT>();
  u32x4 b[NCH][P];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int j = 0; j < P; ++j) {
      // piece (16 bytes) of the lane's MFMA operand j, then its swizzled position
      const int pp = FMT == FMT_FP8 ? 8 * (j >> 1) + 2 * g + (j & 1) : 16 * (j >> 2) + 4 * g + (j & 3);
      b[c][j] = *reinterpret_cast<const u32x4*>(aslot + c * 16 * CB + r16 * CB + ((pp ^ r16) << 4));
    }
  dma_compute<FMT, NMAT, NCH>(wstage, rd0, rd1, 8 * g, b, side, acc);
}

// MXFP4 down stage (no K split) of at most 8 K steps: the lane's row of e8m0
// codes lives in registers, 16 bytes per lane group (those of steps 2g and
// 2g + 1), loaded once per pass instead of one gathered 8-byte load per tile
// and step; step st takes its two words from lane group st / 2 by a lane
// permutation (no memory access).
constexpr int kCodeRegSteps = 8;
template <int NMAT>
__device__ __forceinline__ void code_regs_side(const u32x4 (&cr)[NMAT], int r16, int st,
                                               DmaSide<FMT_MXFP4> (&sd)[NMAT]) {
  const int src = (r16 + 16 * (st >> 1)) * 4;
  const bool hi = (st & 1) != 0;
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    sd[m].codes.x = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(hi ? cr[m][2] : cr[m][0])));
    sd[m].codes.y = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(hi ? cr[m][3] : cr[m][1])));
  }
}

template <int FMT, int S, int SA, int T, int NMAT, int NCH, bool CR = false>
__device__ __forceinline__ void sh_tail(int left, int i, const uint8_t* ring, const uint8_t* aring, uint32_t rd0,
                                        uint32_t rd1, int r16, int g, const DmaSide<FMT> (&side)[S][NMAT],
                                        f32x4 (&acc)[NMAT][NCH], const u32x4 (&cr)[NMAT]) {
  if constexpr (T < S - 1) {
    if (left > T) {
      wait_vmcnt<(S - 2 - T) * sh_per_step<FMT, NMAT, NCH, CR>()>();
      bare_barrier_dec();
      if constexpr (CR) {
        DmaSide<FMT> sd[NMAT];
        code_regs_side<NMAT>(cr, r16, i + T, sd);
        sh_compute<FMT, NMAT, NCH>(ring + T * NMAT * kTileBytes, aring + ((i + T) % SA) * act_slot_bytes<FMT, NCH>(),
                                   rd0, rd1, r16, g, sd, acc);
      } else {
        sh_compute<FMT, NMAT, NCH>(ring + T * NMAT * kTileBytes, aring + ((i + T) % SA) * act_slot_bytes<FMT, NCH>(),
                                   rd0, rd1, r16, g, side[T], acc);
      }
      sh_tail<FMT, S, SA, T + 1, NMAT, NCH, CR>(left, i, ring, aring, rd0, rd1, r16, g, side, acc, cr);
    }
  }
}

// gemv_tile_dma for the down stage with the activations in the shared ring
// (aring); route column col of chunk c reads activation row arow[c][...]
// through the per-lane copy offsets avoff (kOutOfRange past the segment).
template <int FMT, int NMAT, int NCH, int WIDE = 0, bool CR = false, bool CW = false>
__device__ __forceinline__ void gemv_tile_dma_sh(const DmaTiles<NMAT>& dt, int K, int wave,
                                                 __amdgpu_buffer_rsrc_t br,
                                                 const uint32_t (&avoff)[NCH][act_copies<FMT>()], uint8_t* ring,
                                                 uint8_t* aring, f32x4 (&acc)[NMAT][NCH]) {
  static_assert(!CR || FMT == FMT_MXFP4, "codes in registers: MXFP4 only");
  constexpr int S = dma_depth<FMT, NMAT, NCH, WIDE>();
  constexpr int SA = S + 1;
  constexpr int kStage = NMAT * kTileBytes;
  constexpr int kSlot = act_slot_bytes<FMT, NCH>();
  const int lane = lane_id(), r16 = lane & 15, g = lane >> 4;
  const uint32_t rd0 = r16 * 128 + ((g ^ (r16 & 7)) << 4);
  const uint32_t rd1 = r16 * 128 + (((4 + g) ^ (r16 & 7)) << 4);
  const int n = K / dma_kstep<FMT>();
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < NMAT; ++m)
#pragma unroll
    for (int c = 0; c < NCH; ++c) acc[m][c] = zero;
  DmaSide<FMT> side[S][NMAT];  // unused with the codes in registers
  u32x4 cr[NMAT];
  DmaSide<FMT> nx[NMAT];  // codes in registers: those of the next step
  if constexpr (CR) {
    // issued before the first step's copies: its wait covers them
#pragma unroll
    for (int m = 0; m < NMAT; ++m) cr[m] = buf_x4(dt.sr, dt.soff[m] + 16 * g, 0);
  }
  bare_barrier_dec();  // the previous pass's last slots have been read by every wave
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    sh_issue<FMT, NMAT, NCH, CR, CW>(dt, br, avoff, ring + s * kStage, aring + s * kSlot, wave, s,
                                 s < n ? 0u : kOutOfRange, side[s]);
  int i = 0;
  for (; i + S <= n; i += S) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int t = i + s, ahead = t + S - 1;
      sh_issue<FMT, NMAT, NCH, CR, CW>(dt, br, avoff, ring + ((s + S - 1) % S) * kStage, aring + (ahead % SA) * kSlot,
                                   wave, ahead, ahead < n ? 0u : kOutOfRange, side[(s + S - 1) % S]);
      wait_vmcnt<(S - 1) * sh_per_step<FMT, NMAT, NCH, CR>()>();
      bare_barrier_dec();  // every wave's copies of step t have landed
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (CR) {
        DmaSide<FMT> sd[NMAT];
        if (t == 0) {
          code_regs_side<NMAT>(cr, r16, 0, sd);
        } else {
#pragma unroll
          for (int m = 0; m < NMAT; ++m) sd[m] = nx[m];
        }
        // the next step's codes, permuted while this step computes
        code_regs_side<NMAT>(cr, r16, t + 1, nx);
        sh_compute<FMT, NMAT, NCH>(ring + s * kStage, aring + (t % SA) * kSlot, rd0, rd1, r16, g, sd, acc);
      } else {
        sh_compute<FMT, NMAT, NCH>(ring + s * kStage, aring + (t % SA) * kSlot, rd0, rd1, r16, g, side[s], acc);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  sh_tail<FMT, S, SA, 0, NMAT, NCH, CR>(n - i, i, ring, aring, rd0, rd1, r16, g, side, acc, cr);
}

// Where a segment's column lives.  Routed segments: column col is route
// sorted[start + col]; shared pieces: column col is token start + col.
struct SegView {
  bool shared;
  int expert, start, count;
};

// Where a lane's column goes, read before the K loop so that the epilogue
// issues no dependent loads.  Stage 0: the act row and the router weight
// applied to the input (1 unless weight_on_input); stage 1: the ic3 row (the
// route) or the sh_out row (the token) and the router weight applied to the
// output.
struct ColDst {
  int row;
  float w;
};

template <int STAGE>
__device__ __forceinline__ ColDst col_dst(const DecodeArgs& a, const SegView& sv, int col, int route) {
  ColDst d;
  if constexpr (STAGE == 0) {
    d.row = sv.shared ? a.M * a.k + sv.start + col : route;
    d.w = (!sv.shared && a.weight_on_input) ? a.topk_w[route] : 1.0f;
  } else {
    d.row = sv.shared ? sv.start + col : route;
    d.w = (!sv.shared && !a.weight_on_input) ? a.topk_w[route] : 1.0f;
  }
  return d;
}

template <int N>
__device__ __forceinline__ ColDst pick(const ColDst (&d)[N], int c) {
  ColDst r = d[0];
#pragma unroll
  for (int i = 1; i < N; ++i)
    if (c == i) r = d[i];
  return r;
}

// Epilogue of one 16-row output tile for one lane (4 consecutive rows
// rows_at..rows_at+3 of its column).  Stage 0: g, u are the gate and up sums;
// stage 1: g is the down sum (u unused).
template <int STAGE>
__device__ __forceinline__ void tile_epilogue(const DecodeArgs& a, const SegView& sv, ColDst d, int rows_at, f32x4 g,
                                              f32x4 u) {
  float o[4];
  uint16_t* dst;
  if constexpr (STAGE == 0) {
    const float lim = sv.shared ? a.sh_act_limit : a.act_limit;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      // gate and up rounded to bf16 by one packed conversion
      const uint32_t gu = pack_bf16x2(g[v] * d.w, u[v] * d.w);
      float gg = __uint_as_float(gu << 16), uu = __uint_as_float(gu & 0xffff0000u);
      swiglu_clamp(lim, gg, uu);
      o[v] = act_apply(a.act_kind, gg) * uu;
    }
    dst = a.act + static_cast<size_t>(d.row) * a.act_stride + rows_at;
  } else {
    dst = (sv.shared ? a.sh_out : a.ic3) + static_cast<size_t>(d.row) * a.H + rows_at;
#pragma unroll
    for (int v = 0; v < 4; ++v) o[v] = g[v] * d.w;
  }
  uint2 pk;
  pk.x = pack_bf16x2(o[0], o[1]);
  pk.y = pack_bf16x2(o[2], o[3]);
  *reinterpret_cast<uint2*>(dst) = pk;
}

// One pass over up to NCH chunks (16 columns each) of a segment.  The 4 waves
// of the workgroup form 4/KS row groups of KS waves; a row group covers RT
// 16-row tiles per matrix (gate and up tiles in stage 0) and its KS waves split
// K.  With KS > 1 the partial sums meet in LDS (red[4][NMAT][NCH][64] float4)
// and are added in fixed wave order, so results do not depend on timing.
template <int FMT, int STAGE, int RT, int KS, int NCH, int WIDE = 0, bool CW = false>
__device__ __forceinline__ void decode_pass(const DecodeArgs& a, const BankView& bank, const SegView& sv, int base,
                                            int row0, int inter, uint8_t* smem, uint8_t* aring) {
  f32x4* red = reinterpret_cast<f32x4*>(smem);
  constexpr int NMAT = STAGE == 0 ? 2 * RT : RT;
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform (SGPR)
  const int kw = wave % KS, rg = wave / KS;
  const int r16 = lane & 15, g = lane >> 4;
  const int N = STAGE == 0 ? 2 * inter : a.H;
  const int K = STAGE == 0 ? a.H : inter;
  const int nch = min(NCH, (sv.count - base + 15) / 16);
  const int wrow0 = row0 + rg * 16 * RT;

  // activation rows: x (stage 0) or the act buffer (stage 1)
  const uint16_t* bbase = STAGE == 0 ? a.x : a.act;
  const uint32_t brows = STAGE == 0 ? static_cast<uint32_t>(a.M)
                                    : static_cast<uint32_t>(a.M * a.k + (a.sh_out ? a.M : 0));
  const uint32_t bstride = STAGE == 0 ? static_cast<uint32_t>(a.H) : static_cast<uint32_t>(a.act_stride);
  const __amdgpu_buffer_rsrc_t br = make_rsrc(bbase, brows * bstride * 2);
  uint32_t bvoff[NCH];
  ColDst cd[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col = base + c * 16 + r16;
    if (col < sv.count) {
      const int route = sv.shared ? -1 : a.sorted[sv.start + col];
      int row;
      if (STAGE == 0) row = sv.shared ? sv.start + col : route / a.k;
      else row = sv.shared ? a.M * a.k + sv.start + col : route;
      bvoff[c] = static_cast<uint32_t>(row) * bstride * 2 + g * b_group_bytes<FMT>();
      cd[c] = col_dst<STAGE>(a, sv, col, route);
    } else {
      bvoff[c] = kOutOfRange;
      cd[c] = ColDst{0, 0.0f};
    }
  }
  const uint32_t rb = static_cast<uint32_t>(row_bytes<FMT>(K));
  WTiles<NMAT> wt;
  wt.wr = make_rsrc(bank.w + static_cast<size_t>(sv.expert) * N * rb, static_cast<uint32_t>(N) * rb);
  if constexpr (FMT == FMT_FP8) {
    const uint32_t sbytes = static_cast<uint32_t>(N / 128) * (K / 128) * 4;
    wt.sr = make_rsrc(static_cast<const uint8_t*>(bank.s) + static_cast<size_t>(sv.expert) * sbytes, sbytes);
  } else if constexpr (FMT == FMT_MXFP4) {
    const uint32_t cbytes = static_cast<uint32_t>(N) * (K / 32);
    wt.sr = make_rsrc(static_cast<const uint8_t*>(bank.s) + static_cast<size_t>(sv.expert) * cbytes, cbytes);
  } else {
    wt.sr = wt.wr;
  }
#pragma unroll
  for (int m = 0; m < NMAT; ++m) {
    // matrix m: gate tiles then up tiles (stage 0); down tiles (stage 1)
    const int tile_row = (STAGE == 0 && m >= RT) ? inter + wrow0 + 16 * (m - RT) : wrow0 + 16 * m;
    const int ridx = tile_row + r16;
    wt.wvoff[m] = static_cast<uint32_t>(ridx) * rb + g * a_group_bytes<FMT>();
    if constexpr (FMT == FMT_MXFP4)
      wt.soff[m] = static_cast<uint32_t>(ridx) * (K / 32) + g;
    else  // a 16-row tile lies inside one 128-row scale block
      wt.soff[m] = static_cast<uint32_t>(tile_row / 128) * (K / 128) * 4;
  }
  f32x4 acc[NMAT][NCH];
  // FP8 always, MXFP4 when a K step (two K blocks) divides K: the LDS path
  constexpr bool kDma = FMT == FMT_FP8 || FMT == FMT_MXFP4;
  if (kDma && K % dma_kstep<FMT>() == 0) {
    if constexpr (kDma) {
      DmaTiles<NMAT> dt;
      dt.wr = wt.wr;
      dt.sr = wt.sr;
      const int dr = lane >> 3, dc = (lane & 7) ^ dr;  // DMA lane: row dr of 8, stored at slot lane & 7
#pragma unroll
      for (int m = 0; m < NMAT; ++m) {
        const int tile_row = (STAGE == 0 && m >= RT) ? inter + wrow0 + 16 * (m - RT) : wrow0 + 16 * m;
#pragma unroll
        for (int h = 0; h < 2; ++h) dt.voff[m][h] = static_cast<uint32_t>(tile_row + 8 * h + dr) * rb + dc * 16;
        dt.soff[m] = FMT == FMT_FP8 ? wt.soff[m] : static_cast<uint32_t>(tile_row + r16) * (K / 32);
      }
      uint8_t* ring = smem + wave * dma_ring_bytes<FMT, NMAT, WIDE>();
      if constexpr (KS == 1) {
        // activation copies: copy v of chunk c of this wave covers columns
        // q * (1024 / CB) + lane / (CB / 16), q = wave * act_copies + v
        constexpr int CB = act_col_bytes<FMT>();
        uint32_t avoff[NCH][act_copies<FMT>()];
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
          for (int v = 0; v < act_copies<FMT>(); ++v) {
            const int colc = (wave * act_copies<FMT>() + v) * (1024 / CB) + lane / (CB / 16);
            const int piece = (lane % (CB / 16)) ^ colc;
            const int col = base + c * 16 + colc;
            if (col < sv.count) {
              int row;
              if (STAGE == 0) row = sv.shared ? sv.start + col : a.sorted[sv.start + col] / a.k;
              else row = sv.shared ? a.M * a.k + sv.start + col : a.sorted[sv.start + col];
              avoff[c][v] = static_cast<uint32_t>(row) * bstride * 2 + piece * 16;
            } else {
              avoff[c][v] = kOutOfRange;
            }
          }
        if constexpr (FMT == FMT_MXFP4) {
          if (K <= kCodeRegSteps * dma_kstep<FMT>())
            gemv_tile_dma_sh<FMT, NMAT, NCH, WIDE, true>(dt, K, wave, br, avoff, ring, aring, acc);
          else
            gemv_tile_dma_sh<FMT, NMAT, NCH, WIDE>(dt, K, wave, br, avoff, ring, aring, acc);
        } else {
          gemv_tile_dma_sh<FMT, NMAT, NCH, WIDE, false, CW>(dt, K, wave, br, avoff, ring, aring, acc);
        }
      } else {
        if constexpr (FMT == FMT_MXFP4 && KS == kDecWaves && STAGE == 0) {
          // aring: the code table's LDS, behind the waves' rings
          if (code_table_fits<NMAT>(K)) gemv_tile_dma<FMT, NMAT, NCH, KS, true>(dt, K, kw, br, bvoff, ring, acc, aring, wrow0, inter);
          else gemv_tile_dma<FMT, NMAT, NCH, KS>(dt, K, kw, br, bvoff, ring, acc);
        } else {
          gemv_tile_dma<FMT, NMAT, NCH, KS, false, CW>(dt, K, kw, br, bvoff, ring, acc);
        }
      }
    }
  } else {
    if constexpr (FMT != FMT_FP8)  // FP8 K is a multiple of 128: never here
      gemv_tile<FMT, NMAT, NCH, KS>(wt, K, kw, br, bvoff, acc);
  }

  if constexpr (KS == 1) {
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const int col = base + c * 16 + r16;
        if (c < nch && col < sv.count)
          tile_epilogue<STAGE>(a, sv, cd[c], wrow0 + 16 * t + g * 4, acc[t][c], acc[STAGE == 0 ? RT + t : t][c]);
      }
  } else {
    if constexpr (kDma) __syncthreads();  // red overlays the waves' LDS rings
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        if (c < nch) red[((wave * NMAT + m) * NCH + c) * kWave + lane] = acc[m][c];
    __syncthreads();
    // the KS waves of a row group finish its (tile, chunk) items round robin
    for (int item = kw; item < RT * nch; item += KS) {
      const int t = item / nch, c = item % nch;
      const int col = base + c * 16 + r16;
      const int mg = t, mu = STAGE == 0 ? RT + t : t;
      const int w0 = rg * KS;
      f32x4 sg = red[((w0 * NMAT + mg) * NCH + c) * kWave + lane];
      f32x4 su = red[((w0 * NMAT + mu) * NCH + c) * kWave + lane];
#pragma unroll
      for (int v = 1; v < KS; ++v) {
        sg += red[(((w0 + v) * NMAT + mg) * NCH + c) * kWave + lane];
        if (STAGE == 0) su += red[(((w0 + v) * NMAT + mu) * NCH + c) * kWave + lane];
      }
      if (col < sv.count) tile_epilogue<STAGE>(a, sv, pick(cd, c), wrow0 + 16 * t + g * 4, sg, su);
    }
    __syncthreads();
  }
}

// Route chunks (of 16) per pass, sized so that two K stages of weights and
// activations plus the accumulators fit 256 registers per lane (occupancy 2).
// With the activations shared through LDS (KS = 1) MXFP4 takes one chunk per
// pass, which keeps LDS at 80 KB (two workgroups per CU).  WIDE kernels (FP8
// calls of at least kWideMinTokens tokens, segments of up to 64 routes) run
// FP8 passes of up to four chunks, as many as the segment's routes need, so
// an expert's weights are read once for its 64 routes.
template <int FMT, int STAGE, int RT, int KS, int WIDE = 0>
constexpr int chunks_per_pass() {
  if constexpr (WIDE && KS == 1 && FMT == FMT_FP8) return 4;
  if constexpr (KS == 1 && FMT == FMT_MXFP4) return 1;
  if constexpr (STAGE == 0) return RT == 1 ? 2 : (FMT == FMT_BF16 ? 1 : 2);
  return 2;
}

template <int FMT, int STAGE, int RT, int KS, int WIDE = 0, bool CW = false>
__device__ __forceinline__ void decode_segment(const DecodeArgs& a, const BankView& bank, const SegView& sv, int row0,
                                               int inter, uint8_t* smem, uint8_t* aring) {
  constexpr int CMAX = chunks_per_pass<FMT, STAGE, RT, KS, WIDE>();
  for (int base = 0; base < sv.count; base += 16 * CMAX) {
    if constexpr (CMAX == 4) {
      // as many chunks as the segment has routes left (all on the 2-stage ring)
      const int left = sv.count - base;
      if (left <= 16) decode_pass<FMT, STAGE, RT, KS, 1, WIDE, CW>(a, bank, sv, base, row0, inter, smem, aring);
      else if (left <= 32) decode_pass<FMT, STAGE, RT, KS, 2, WIDE, CW>(a, bank, sv, base, row0, inter, smem, aring);
      else decode_pass<FMT, STAGE, RT, KS, 4, WIDE, CW>(a, bank, sv, base, row0, inter, smem, aring);
    } else if constexpr (CMAX == 1) {
      decode_pass<FMT, STAGE, RT, KS, 1>(a, bank, sv, base, row0, inter, smem, aring);
    } else {
      if (sv.count - base <= 16) decode_pass<FMT, STAGE, RT, KS, 1, 0, CW>(a, bank, sv, base, row0, inter, smem, aring);
      else decode_pass<FMT, STAGE, RT, KS, 2, 0, CW>(a, bank, sv, base, row0, inter, smem, aring);
    }
  }
}

constexpr int kRedFloats4 = kDecWaves * 8 * kWave;  // NMAT * chunks_per_pass <= 8 (K-split kernels)

// Grid: x = row blocks of (4/KS) * RT * 16 rows, y = the shared expert's token
// pieces of seg_cap tokens, then the routed segments (max_seg, the tail beyond
// n_seg exits).  The shared pieces come first: their workgroups can be several
// times heavier than the routed ones (a bf16 shared expert beside MXFP4 routed
// experts reads 4x the bytes per row) and would otherwise start last and trail.
template <int FMT_R, int FMT_S, int STAGE, int RT, int KS, int WIDE = 0>
struct StageSmem {
  static constexpr int kNmat = STAGE == 0 ? 2 * RT : RT;
  static constexpr int kRingF8 =
      (FMT_R == FMT_FP8 || FMT_S == FMT_FP8) ? dma_ring_bytes<FMT_FP8, kNmat, WIDE && KS == 1>() : 0;
  static constexpr int kRingF4 =
      (FMT_R == FMT_MXFP4 || FMT_S == FMT_MXFP4) ? dma_ring_bytes<FMT_MXFP4, kNmat>() : 0;
  static constexpr int kRing = kDecWaves * (kRingF8 > kRingF4 ? kRingF8 : kRingF4);
  // without a K split the activation ring shared by the waves follows the waves' weight rings
  static constexpr bool kShAct = KS == 1;
  static constexpr int kActF8 = kShAct && (FMT_R == FMT_FP8 || FMT_S == FMT_FP8)
                                    ? sh_act_ring_bytes<FMT_FP8, kNmat, chunks_per_pass<FMT_FP8, STAGE, RT, KS, WIDE>()>()
                                    : 0;
  static constexpr int kActF4 =
      kShAct && (FMT_R == FMT_MXFP4 || FMT_S == FMT_MXFP4)
          ? sh_act_ring_bytes<FMT_MXFP4, kNmat, chunks_per_pass<FMT_MXFP4, STAGE, RT, KS>()>()
          : 0;
  static constexpr int kAct = kActF8 > kActF4 ? kActF8 : kActF4;
  // MXFP4 with a K split: the e8m0 code table of the workgroup's tiles
  static constexpr int kCodes = (KS == kDecWaves && (FMT_R == FMT_MXFP4 || FMT_S == FMT_MXFP4)) ? kCodeTableBytes : 0;
  static constexpr int kRed = KS > 1 ? kRedFloats4 * 16 : 0;
  static constexpr int kSmem =
      kRing + kAct + kCodes > kRed ? kRing + kAct + kCodes : kRed > 16 ? kRed : 16;
};

// One workgroup of the stage grid: row block bx of segment seg, the first n_sh
// segments being the shared expert's token pieces.
template <int FMT_R, int FMT_S, int STAGE, int RT, int KS, int WIDE = 0>
__device__ __forceinline__ void decode_stage_block(const DecodeArgs& a, int bx, int seg, int n_sh, uint8_t* smem) {
  constexpr int kRing = StageSmem<FMT_R, FMT_S, STAGE, RT, KS, WIDE>::kRing;
  SegView sv;
  sv.shared = seg < n_sh;
  if (sv.shared) {
    sv.expert = 0;
    sv.start = seg * a.seg_cap;
    sv.count = min(a.seg_cap, a.M - sv.start);
  } else {
    seg -= n_sh;
    if (seg >= a.n_seg[0]) return;
    sv.expert = a.seg_expert[seg];
    sv.start = a.seg_start[seg];
    sv.count = a.seg_count[seg];
  }
  // both fields read, then chosen: a select between the two (adjacent)
  // argument fields was compiled into a load from a private copy of the
  // arguments, i.e. scratch memory, in some instantiations
  const int ia = a.I, is = a.Is;
  const int inter = sv.shared ? is : ia;
  const int row0 = bx * (kDecWaves / KS) * RT * 16;
  if (STAGE == 0 && row0 >= inter) return;
  // field-wise selects keep the kernel argument block out of private memory
  BankView bank;
  if constexpr (STAGE == 0) {
    bank.w = sv.shared ? a.sh_gate_up.w : a.gate_up.w;
    bank.s = sv.shared ? a.sh_gate_up.s : a.gate_up.s;
  } else {
    bank.w = sv.shared ? a.sh_down.w : a.down.w;
    bank.s = sv.shared ? a.sh_down.s : a.down.s;
  }
  const int fmt = sv.shared ? FMT_S : FMT_R;
  if (fmt == FMT_BF16) {
    if constexpr (FMT_R == FMT_BF16 || FMT_S == FMT_BF16)
      decode_segment<FMT_BF16, STAGE, RT, KS>(a, bank, sv, row0, inter, smem, smem + kRing);
  } else if (fmt == FMT_FP8) {
    if constexpr (FMT_R == FMT_FP8 || FMT_S == FMT_FP8)
    {
      // the shared expert's token pieces read the same weights at about the
      // same time (the grid's first rows: each row block's pieces are
      // gridDim.x apart, a multiple of 8, so on the same XCD)
      if (sv.shared && a.M > a.seg_cap)
        decode_segment<FMT_FP8, STAGE, RT, KS, WIDE, true>(a, bank, sv, row0, inter, smem, smem + kRing);
      else
        decode_segment<FMT_FP8, STAGE, RT, KS, WIDE>(a, bank, sv, row0, inter, smem, smem + kRing);
    }
  } else {
    if constexpr (FMT_R == FMT_MXFP4 || FMT_S == FMT_MXFP4)
      decode_segment<FMT_MXFP4, STAGE, RT, KS>(a, bank, sv, row0, inter, smem, smem + kRing);
  }
}

template <int FMT_R, int FMT_S, int STAGE, int RT, int KS, int WIDE = 0>
__global__ void __launch_bounds__(kDecWaves * kWave) __attribute__((amdgpu_waves_per_eu(2))) decode_stage_kernel(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[StageSmem<FMT_R, FMT_S, STAGE, RT, KS, WIDE>::kSmem];
  // shared pieces (0 without a shared expert, or when the router's launch ran them)
  const int n_sh = static_cast<int>(gridDim.y) - a.max_seg;
  decode_stage_block<FMT_R, FMT_S, STAGE, RT, KS, WIDE>(a, blockIdx.x, blockIdx.y, n_sh, smem);
}

// ---- Router + permutation beside the shared expert's gate_up --------------
// For decode calls of at most kRouteSharedTokens tokens with a grouped-sigmoid
// router and a shared expert: workgroup 0 routes (wave t takes token t, then
// wave 0 aligns, as route_align_kernel does) while workgroups 1.. run the
// shared expert's gate_up piece -- the same K split, code and arithmetic as
// the shared piece of the stage-0 grid, which then leaves it out.  The shared
// expert does not depend on the routing, so its weights stream while the
// router's dependent chains keep one CU busy.  One 16-row tile per wave gives
// the piece enough workgroups to finish under the router (two tiles per wave
// outlasted it).  Measured: C3 (bf16 shared beside MXFP4) b=1 60.6 -> 53.8 us,
// b=2 69.3 -> 67.3 us; C4 b=1 -1%.  Up to 4 tokens (one per wave of the
// routing workgroup), against the separate launches with the current
// kernels: C4 b=3 144.6 -> 142.9 us, b=4 163.8 -> 160.2 us, C3 b=4 equal.
constexpr int kSharedRT = 1, kSharedKS = 4;
constexpr int kRouteSharedTokens = 4;
static_assert(kRouteSharedTokens <= kDecWaves, "the routing workgroup routes one token per wave");

template <int PER, int FS>
__global__ void __launch_bounds__(kDecWaves * kWave) __attribute__((amdgpu_waves_per_eu(2)))
route_shared_kernel(RouteArgs r, AlignArgs al, DecodeArgs a) {
  using SM = StageSmem<FS, FS, 0, kSharedRT, kSharedKS>;
  static_assert(SM::kSmem >= (kDecWaves * PER + 1) * kWave * 4, "router scratch must fit the stage's LDS");
  __shared__ __attribute__((aligned(16))) uint8_t smem[SM::kSmem];
  if (blockIdx.x == 0) {
    float* s_c = reinterpret_cast<float*>(smem);
    int* s_ids = reinterpret_cast<int*>(smem + kDecWaves * PER * kWave * 4);
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    if (wave < r.M) {
      const int id = grouped_token<PER>(static_cast<const float*>(r.logits) + static_cast<size_t>(wave) * r.E, r.bias,
                                        r.E, r.n_group, r.topk_group, r.k, r.renorm, r.scale, s_c + wave * PER * kWave,
                                        r.out_w + static_cast<size_t>(wave) * r.k,
                                        r.out_ids + static_cast<size_t>(wave) * r.k);
      if (lane < r.k) s_ids[wave * r.k + lane] = id;
    }
    __syncthreads();
    if (wave == 0) align_small(al, s_ids);
    return;
  }
  decode_stage_block<FS, FS, 0, kSharedRT, kSharedKS>(a, blockIdx.x - 1, 0, 1, smem);
}

template <int PER>
static hipError_t launch_route_shared_per(int fmt_s, const RouteArgs& r, const AlignArgs& al, const DecodeArgs& a,
                                          hipStream_t stream) {
  const dim3 grid(1 + (a.Is + kSharedRT * 16 * (kDecWaves / kSharedKS) - 1) / (kSharedRT * 16 * (kDecWaves / kSharedKS)));
  if (fmt_s == FMT_BF16)
    hipLaunchKernelGGL((route_shared_kernel<PER, FMT_BF16>), grid, dim3(kDecWaves * kWave), 0, stream, r, al, a);
  else if (fmt_s == FMT_FP8)
    hipLaunchKernelGGL((route_shared_kernel<PER, FMT_FP8>), grid, dim3(kDecWaves * kWave), 0, stream, r, al, a);
  else
    hipLaunchKernelGGL((route_shared_kernel<PER, FMT_MXFP4>), grid, dim3(kDecWaves * kWave), 0, stream, r, al, a);
  return hipGetLastError();
}

bool route_shared_fits(const RouteArgs& r, const AlignArgs& al, int fmt_s, const DecodeArgs& a) {
  const int per = (r.E + kWave - 1) / kWave;
  return r.grouped && fmt_s != FMT_NONE && a.Is > 0 && r.M <= kRouteSharedTokens && r.M * r.k <= kWave &&
         align_fits_wave(al) && per <= 4 && al.ids == r.out_ids;
}

hipError_t launch_route_shared(const RouteArgs& r, const AlignArgs& al, int fmt_s, const DecodeArgs& a,
                               hipStream_t stream) {
  if (!route_shared_fits(r, al, fmt_s, a)) return hipErrorNotSupported;
  const int per = (r.E + kWave - 1) / kWave;
  if (per <= 1) return launch_route_shared_per<1>(fmt_s, r, al, a, stream);
  if (per <= 2) return launch_route_shared_per<2>(fmt_s, r, al, a, stream);
  return launch_route_shared_per<4>(fmt_s, r, al, a, stream);
}

// y[t] = bf16( bf16(sum_r ic3[t,r]) + sh_out[t] ), routes with ids outside
// [0, num_rows) skipped; sum in route order r = 0..k-1 in float32 (reference
// moe_sum_reduce_kernel, kernel/triton/fused_moe.py:142-153).  STREAM: ic3 is
// read once and is far larger than L2 (prefill), so its loads are nontemporal;
// decode's ic3 was just written and is still in L2.
template <bool STREAM>
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
  // routes in groups of 8: the group's ids are read, then the ic3 rows of its
  // valid routes, all before the adds (the ic3 row of route r is t*k + r
  // whatever its id; rows of skipped routes hold stale data and are not read,
  // which matters where most routes are skipped: an expert-parallel share, the
  // misses of an offload cache)
  for (int r0 = 0; r0 < k; r0 += 8) {
    u32x4 v[8];
    bool ok[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int r = r0 + q;
      const int e = r < k ? ids[t * k + r] : -1;
      ok[q] = e >= 0 && e < num_rows;
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const u32x4* src = reinterpret_cast<const u32x4*>(ic3 + static_cast<size_t>(t * k + r0 + q) * H + h);
      v[q] = !ok[q] ? u32x4{0, 0, 0, 0} : STREAM ? __builtin_nontemporal_load(src) : *src;
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if (!ok[q]) continue;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        acc[2 * w] += bf16_to_f32(static_cast<uint16_t>(v[q][w] & 0xffffu));
        acc[2 * w + 1] += bf16_to_f32(static_cast<uint16_t>(v[q][w] >> 16));
      }
    }
  }
  uint32_t o[4];
  if (sh_out) {
    const uint4 v = *reinterpret_cast<const uint4*>(sh_out + static_cast<size_t>(t) * H + h);
    const uint32_t wds[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t r = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);  // bf16(sum) of both features
      o[q] = pack_bf16x2(__uint_as_float(r << 16) + __uint_as_float(wds[q] << 16),
                         __uint_as_float(r & 0xffff0000u) + __uint_as_float(wds[q] & 0xffff0000u));
    }
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
  }
  uint4 out;
  out.x = o[0];
  out.y = o[1];
  out.z = o[2];
  out.w = o[3];
  *reinterpret_cast<uint4*>(y + static_cast<size_t>(t) * H + h) = out;
}

// Launch shapes.  Stage 0 (K = hidden, long rows): the 4 waves split K and a
// workgroup covers RT tiles of gate and of up.  Stage 1 (K = intermediate,
// short rows): each wave owns RT whole tiles.  RT = 2 halves the activation
// loads per weight byte and is faster at every measured batch except when its
// grid leaves the resident slots much emptier than RT = 1's (b = 1 gate_up:
// 1.1 rounds against 2.25), so RT = 1 is used only when it fills the slots at
// least 15 points better.  (RT = 4 down tiles measured no faster than RT = 2
// once the weights come through LDS.)

// Resident workgroups per CU of a kernel (runtime occupancy query, cached).
template <auto KERNEL>
static int resident_per_cu() {
  static int cached = 0;
  if (cached == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(KERNEL), kDecWaves * kWave, 0) !=
            hipSuccess ||
        n < 1)
      n = 1;
    cached = n;
  }
  return cached;
}

static int cu_count() {
  static int cached = 0;
  if (cached == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                  hipSuccess || n < 1)
      n = 256;
    cached = n;
  }
  return cached;
}

// Fraction of the resident slots kept busy over the rounds of a grid.
static double fill(long long wgs, long long slots) {
  const long long rounds = (wgs + slots - 1) / slots;
  return static_cast<double>(wgs) / static_cast<double>(rounds * slots);
}

template <auto KERNEL>
static double fill_of(dim3 g) {
  return fill(static_cast<long long>(g.x) * g.y, static_cast<long long>(cu_count()) * resident_per_cu<KERNEL>());
}

template <auto KERNEL>
static hipError_t launch_one(dim3 g, const DecodeArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL(KERNEL, g, dim3(kDecWaves * kWave), 0, stream, a);
  return hipGetLastError();
}

constexpr int kGateUpSharedMinM = 80;

// Bytes per weight times two (bf16 4, FP8 2, MXFP4 1).
static int bytes_per_weight_x2(int fmt) { return fmt == FMT_BF16 ? 4 : fmt == FMT_FP8 ? 2 : 1; }

template <int FR, int FS>
static hipError_t launch_stage_t(int stage, const DecodeArgs& a, bool has_shared, hipStream_t stream) {
  const int gy = a.max_seg + (has_shared ? (a.M + a.seg_cap - 1) / a.seg_cap : 0);
  const int imax = has_shared ? max(a.I, a.Is) : a.I;
  constexpr double kSlack = 0.15;
  if constexpr (FR == FMT_FP8) {
    if (a.seg_cap > kDecodeSegCap) {
      // wide segments (FP8 calls from kWideMinTokens tokens): no K split (as
      // below) and four-chunk passes, so an expert with up to 64 routes is
      // read once (with 32-route segments about half of C4 b=256's experts
      // were read twice): C4 b=256 637 -> 594-597 us.  From 144 tokens:
      // against the 32-route kernels, interleaved A/B, C4 b=144 515 -> 507 us,
      // b=160 521 -> 508, b=192 560 -> 531, b=224 595 -> 545, b=255 624 ->
      // 565; b=96-128 equal
      if (stage == 0) {
        constexpr auto kw = decode_stage_kernel<FR, FS, 0, 1, 1, 1>;
        return launch_one<kw>(dim3((imax + 63) / 64, gy), a, stream);
      }
      constexpr auto kw = decode_stage_kernel<FR, FS, 1, 2, 1, 1>;
      return launch_one<kw>(dim3(a.H / 128, gy), a, stream);
    }
  }
  if (stage == 0) {
    constexpr auto k1 = decode_stage_kernel<FR, FS, 0, 1, 4>;
    constexpr auto k2 = decode_stage_kernel<FR, FS, 0, 2, 4>;
    if (FR == FMT_FP8 && a.M >= kGateUpSharedMinM) {
      // large FP8 calls: no K split, the 4 waves own 16 + 16 rows each and
      // share the activation chunks through LDS (half the activation reads
      // per weight byte of the RT = 2 K-split grid); measured C4 b=128 326 ->
      // 302 us, b=16-64 unchanged, b=8 slower (its grid no longer fills the
      // GPU); MXFP4 (one chunk per pass) slower at b=8-64.  From 80 tokens
      // (interleaved A/B against the K split): C4 b=80 471 -> 464 us, b=96
      // 480 -> 470, b=112 498 -> 478; b=32-64 equal within 2 us
      constexpr auto ks = decode_stage_kernel<FR, FS, 0, 1, 1>;
      return launch_one<ks>(dim3((imax + 63) / 64, gy), a, stream);
    }
    const dim3 g1((imax + 15) / 16, gy), g2((imax + 31) / 32, gy);
    // FP8 calls of up to four tokens, or whose RT = 2 grid is a single round
    // of resident workgroups: few experts, many of the grid's segments empty
    // (routes to experts outside the slot bank), and the RT = 1 grid's twice
    // as many, half as long workgroups end together more evenly (C4 b=1
    // 72.5-72.8 -> 69.6-70.6 us, b=2 115.4-116.1 -> 109.7-109.8 us; b=4
    // 160.1 -> 156.7 and 176.9 -> 175.7 us on two boxes, b=3 equal; up to 8
    // tokens C2 b=8 was 5% slower; MXFP4 at C3 b=1 0.8 us slower, so it
    // keeps RT = 2)
    if (FR == FMT_FP8 &&
        (a.M <= 4 ||
         static_cast<long long>(g2.x) * g2.y <= static_cast<long long>(cu_count()) * resident_per_cu<k2>()))
      return launch_one<k1>(g1, a, stream);
    // MXFP4 up to 8 tokens keeps two row tiles per wave (C3 b=2 66.0-66.5 ->
    // 65.1 us; one tile per wave 0.6-10 us slower at b=1-8)
    if (FR == FMT_MXFP4 && a.M <= 8) return launch_one<k2>(g2, a, stream);
    if (fill_of<k2>(g2) >= fill_of<k1>(g1) - kSlack) return launch_one<k2>(g2, a, stream);
    return launch_one<k1>(g1, a, stream);
  }
  constexpr auto k1 = decode_stage_kernel<FR, FS, 1, 1, 1>;
  constexpr auto k2 = decode_stage_kernel<FR, FS, 1, 2, 1>;
  const dim3 g1(a.H / 64, gy), g2(a.H / 128, gy);
  // a shared expert whose rows are several times heavier than the routed ones
  // (bf16 beside MXFP4) trails the small grid of a one- or two-token call:
  // halve its tiles (C3 down at b=1 22.8 -> 16.5 us, b=2 unchanged; from b=4
  // on the routed segments fill the GPU and one tile per wave is slower)
  const bool heavy_shared = has_shared && bytes_per_weight_x2(FS) >= 4 * bytes_per_weight_x2(FR);
  if (heavy_shared && a.M <= 2) return launch_one<k1>(g1, a, stream);
  // one FP8 token: K split two ways (half the rows per workgroup's row group
  // walk, twice the workgroups); interleaved A/B: C4 b=1 69.6 -> 68.9 us, C2
  // b=1 30.2 -> 29.3 us; from two tokens equal or slower
  if (FR == FMT_FP8 && a.M == 1) {
    constexpr auto kh = decode_stage_kernel<FR, FS, 1, 2, 2>;
    return launch_one<kh>(dim3(a.H / 64, gy), a, stream);
  }
  if (fill_of<k2>(g2) >= fill_of<k1>(g1) - kSlack) return launch_one<k2>(g2, a, stream);
  return launch_one<k1>(g1, a, stream);
}

hipError_t launch_decode_stage(int stage, int fmt_r, int fmt_s, const DecodeArgs& a, hipStream_t stream,
                               bool shared_pieces) {
  const bool sh = fmt_s != FMT_NONE && shared_pieces;
  const int fs = fmt_s != FMT_NONE ? fmt_s : fmt_r;  // FMT_S is unused without a shared expert
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
  // ic3 well beyond the 32 MB of L2 (prefill): stream it
  if (static_cast<size_t>(M) * k * H * 2 > (size_t{64} << 20))
    hipLaunchKernelGGL(combine_kernel<true>, dim3((n + 255) / 256), dim3(256), 0, stream, ic3, ids, num_rows, sh_out,
                       M, k, H, y);
  else
    hipLaunchKernelGGL(combine_kernel<false>, dim3((n + 255) / 256), dim3(256), 0, stream, ic3, ids, num_rows, sh_out,
                       M, k, H, y);
  return hipGetLastError();
}

}  // namespace ftmoe
