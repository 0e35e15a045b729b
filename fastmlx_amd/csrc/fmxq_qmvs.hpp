// fmxq_qmvs.hpp -- the K walk of one wave of the int4 (group 64) skinny MFMA
// product, shared by the dense GEMV (qmvs_kernel, fmxq_skinny.hip) and the
// grouped MoE product (fmxq_moe_gemm.hip).
//
// A wave owns 16 NTT output columns (rows of W) starting at nb, up to 16 MT rows
// of x (lane (m = l % 16, q = l / 16) holds the pointer to its x row, advanced by
// 16 q elements), NMAT weight matrices sharing those x rows (gate and up of a
// SwitchGLU), and the steps [s0, s1) of SU 64-value units each.
//
// Per step, for each matrix:
//   - the 16 NTT rows x 32 SU bytes of packed weights are read with whole-segment
//     loads (instruction i, lane L -> row i * (64 / LPR) + L / LPR, 16-byte chunk
//     L % LPR) two steps ahead into registers and written to the wave's LDS stage
//     at XOR-swizzled chunk positions;
//   - the stage is read back in the v_mfma_f32_16x16x32_bf16 B layout: lane
//     (c = l % 16, q) takes words 2q, 2q+1 of its row's unit, MFMA i word 2q+i,
//     as bf16(128 + q) pairs (exponent trick, fmxq_mfma_frag.hpp);
//   - scales and biases of the step come as one load per lane and reach the
//     lanes that use them through ds_bpermute.
// A = x in the same k order (xfrag4 of two 16-byte pieces per unit), XD units
// ahead.  Per group: P = sum x (128 + q), xs = sum x (MFMA against ones),
// acc += s P + (b - 128 s) xs.  With FOLD the bias term of four groups goes in
// as one fp32 MFMA (qmvs_bias4) instead of per-group FMAs: fewer VALU
// operations, one more MFMA dependency on the accumulators.  The MoE walks (two
// matrices per wave, VALU-bound) take it; the dense walks measured slower
// with it and do not.
//
// The stage needs no barrier: a wave reads only what it wrote, and the LDS
// operations of one wave complete in order.  Rows past N re-read row N-1 and
// steps past s1 re-read step s1-1; neither reaches an output.
#pragma once
#include <type_traits>

#include "fmxq_common.hpp"
#include "fmxq_mfma_frag.hpp"

namespace fmxq {

constexpr int kQmvsXD = 4;  // x units in flight per wave

// Stage position of 16-byte chunk c of row r: 128-byte rows (SU = 4) use the
// 8-chunk XOR pattern, 256-byte rows (SU = 8) XOR with the row's low 4 bits, so
// the 16 rows a B-fragment read touches at one chunk land on distinct banks.
template <int SU>
__device__ __forceinline__ int qmvs_pos(int c, int r) {
  if constexpr (SU == 4) return c ^ ((r & 7) ^ ((r >> 3) & 1));
  else return c ^ (r & 15);
}

// The bias term of four consecutive units u = 0..3 (K order):
// acc[m][c] += sum_u xs_m(u) bo_c(u), with xs_m(u) the sum of x row m over unit
// u and bo_c(u) = b - 128 s of output column c in unit u, as one
// v_mfma_f32_16x16x4_f32 whose A operand (lane l: row l % 16, k = l / 16) is the
// x sum and B operand (lane l: k = l / 16, column l % 16) the column offset.
// Each unit's values are computed in every lane and kept (qmvs_pick) by the
// lanes whose l / 16 is the unit's position in its group of four.
//
// Sum of x row l % 16 over a unit (A fragment a): the x fragment as the B operand
// of an MFMA against ones, so the result's column (l % 16) is the x row.
__device__ __forceinline__ float qmvs_xsum(const bf16x8 (&a)[2]) {
  const bf16x8 ones = as_bf16x8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
  f32x4 s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, a[0], f32x4{}, 0, 0, 0);
  s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, a[1], s, 0, 0, 0);
  return s[0];
}
// Without the fold: the sums of x rows 4 (l / 16) + r (the accumulator's rows)
// over a unit, x as the A operand against ones.
__device__ __forceinline__ f32x4 qmvs_xsum_rows(const bf16x8 (&a)[2]) {
  const bf16x8 ones = as_bf16x8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
  f32x4 s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], ones, f32x4{}, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], ones, s, 0, 0, 0);
}
__device__ __forceinline__ float qmvs_pick(int j, float v, float held) {
  return ((threadIdx.x & 63) >> 4) == (j & 3) ? v : held;
}
__device__ __forceinline__ f32x4 qmvs_bias4(float xs, float bo, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(xs, bo, acc, 0, 0, 0);
}

template <int NTT, int SU, int BITS = 4>
struct QmvsGeom {
  static constexpr int ROWS = 16 * NTT;
  static constexpr int RB = SU * 8 * BITS;     // bytes of one row per step
  static constexpr int LPR = RB / 16;          // lanes per row in one load instruction
  static constexpr int NI = ROWS * RB / 1024;  // load instructions per step
  static constexpr int SPL = (64 / ROWS == 2) ? SU : SU / 2;  // groups per scale load
  static constexpr int STAGE = ROWS * RB;      // LDS bytes per matrix
};

// w, sc, bi: the NMAT matrices ([N, K/8] u32, [N, K/64] bf16 x2).  stage: this
// wave's NMAT * STAGE bytes of LDS.  xrow: per-lane x row pointers (see above).
template <int MT, int NTT, int SU, int NMAT, bool FOLD>
__device__ __forceinline__ void qmvs_slice(uint8_t* stage, const uint32_t* const (&w)[NMAT],
                                           const uint16_t* const (&sc)[NMAT],
                                           const uint16_t* const (&bi)[NMAT], int64_t nb,
                                           int64_t N, int64_t K, const uint16_t* const (&xrow)[MT],
                                           int64_t s0, int64_t s1,
                                           f32x4 (&acc)[NMAT][MT][NTT]) {
  using G = QmvsGeom<NTT, SU>;
  constexpr int XD = kQmvsXD, U = 64, NI = G::NI, LPR = G::LPR, RB = G::RB, ROWS = G::ROWS;
  constexpr int SPL = G::SPL;
  typedef uint32_t sbv_t __attribute__((ext_vector_type(SPL / 2)));
  const int lane = threadIdx.x & 63;
  const int c16 = lane & 15, q = lane >> 4;
  const int64_t wpr = K / 8, gpr = K / 64;

  // Weights through buffer resources (byte offsets below 2^31, checked by the
  // callers): a step past the slice loads from an offset past the matrix, which
  // returns zeros without a memory access, so the pipeline's last loads fetch
  // nothing yet still issue (the instruction stream stays the same).
  uint32_t wq[NI];
  int wo[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int r = i * (64 / LPR) + lane / LPR;
    int64_t n = nb + r;
    n = n < N ? n : N - 1;
    wq[i] = (uint32_t)((n * wpr + (lane % LPR) * 4) * 4);
    wo[i] = r * RB + (qmvs_pos<RB / 32>(lane % LPR, r) << 4);
  }
  __amdgpu_buffer_rsrc_t wres[NMAT];
#pragma unroll
  for (int p = 0; p < NMAT; ++p)
    wres[p] = __builtin_amdgcn_make_buffer_rsrc((void*)w[p], (short)0, (int)(N * wpr * 4), 0x00020000);
  int wr[NTT][SU];
#pragma unroll
  for (int t = 0; t < NTT; ++t)
#pragma unroll
    for (int j = 0; j < SU; ++j) {
      const int r = 16 * t + c16;
      wr[t][j] = r * RB + (qmvs_pos<SU>(2 * j + (q >> 1), r) << 4) + (q & 1) * 8;
    }
  // Scale loads: lane -> row l % ROWS, kind (l / ROWS) & 1 (0 scales, 1 biases)
  // and, for 16-row tiles, which half of the step's groups (l / ROWS / 2).
  const int sh = lane / ROWS;
  int64_t nrow = nb + lane % ROWS;
  nrow = nrow < N ? nrow : N - 1;
  const int64_t soff = nrow * gpr + ((64 / ROWS == 2) ? 0 : (sh >> 1) * SPL);
  const uint16_t* sbrow[NMAT];
#pragma unroll
  for (int p = 0; p < NMAT; ++p) sbrow[p] = ((sh & 1) ? bi[p] : sc[p]) + soff;

  u32x4 wbuf[2][NMAT][NI];
  sbv_t sbuf[2][NMAT];
  u32x4 xv[XD][MT][2];
  auto load_w = [&](int d, int64_t st) {
    const bool past = st >= s1;
    st = past ? s1 - 1 : st;
#pragma unroll
    for (int p = 0; p < NMAT; ++p) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
        wbuf[d][p][i] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       wres[p], past ? (int)0x80000000u : (int)(wq[i] + (uint32_t)st * SU * 32), 0,
                       2 /* nt */));
      sbuf[d][p] = *reinterpret_cast<const sbv_t*>(sbrow[p] + st * SU);
    }
  };
  const int64_t u_end = s1 * SU;
  auto load_x = [&](int d, int64_t u) {
    u = u < u_end ? u : u_end - 1;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const u32x4* xs = reinterpret_cast<const u32x4*>(xrow[mt] + u * U);
      xv[d][mt][0] = xs[0];
      xv[d][mt][1] = xs[1];
    }
  };

  if (s1 <= s0) return;
  load_w(0, s0);
  load_w(1, s0 + 1);
#pragma unroll
  for (int d = 0; d < XD; ++d) load_x(d, s0 * SU + d);
  for (int64_t st = s0; st < s1; st += 2) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int64_t stp = st + e;
      if (stp < s1) {
#pragma unroll
        for (int p = 0; p < NMAT; ++p)
#pragma unroll
          for (int i = 0; i < NI; ++i)
            *reinterpret_cast<u32x4*>(stage + p * G::STAGE + wo[i]) = wbuf[e][p][i];
        sbv_t mine[NMAT];
#pragma unroll
        for (int p = 0; p < NMAT; ++p) mine[p] = sbuf[e][p];
        load_w(e, stp + 2);
        // Scale and bias pairs (groups 2k, 2k+1 of the step) of the wave's rows.
        uint32_t sv[NMAT][NTT][SU / 2], bv[NMAT][NTT][SU / 2];
#pragma unroll
        for (int p = 0; p < NMAT; ++p)
#pragma unroll
          for (int t = 0; t < NTT; ++t)
#pragma unroll
            for (int k = 0; k < SU / 2; ++k) {
              const int row = 16 * t + c16;
              const int hi = (64 / ROWS == 2) ? 0 : k / (SPL / 2);
              const int idx = (64 / ROWS == 2) ? k : k % (SPL / 2);
              sv[p][t][k] = (uint32_t)__shfl((int)mine[p][idx], (2 * hi) * ROWS + row, 64);
              bv[p][t][k] = (uint32_t)__shfl((int)mine[p][idx], (2 * hi + 1) * ROWS + row, 64);
            }
        static_assert(!FOLD || SU % 4 == 0, "bias term per four units");
        float xsel[MT] = {}, bsel[NMAT][NTT] = {};
        f32x4 xr[MT];
#pragma unroll
        for (int j = 0; j < SU; ++j) {
          const int xd = (e * SU + j) % XD;
          bf16x8 A[MT][2];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            A[mt][0] = xfrag4(xv[xd][mt][0]);
            A[mt][1] = xfrag4(xv[xd][mt][1]);
          }
          load_x(xd, stp * SU + j + XD);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            if constexpr (FOLD) xsel[mt] = qmvs_pick(j, qmvs_xsum(A[mt]), xsel[mt]);
            else xr[mt] = qmvs_xsum_rows(A[mt]);
          }
#pragma unroll
          for (int p = 0; p < NMAT; ++p) {
            u32x2 wv[NTT];
#pragma unroll
            for (int t = 0; t < NTT; ++t)
              wv[t] = *reinterpret_cast<const u32x2*>(stage + p * G::STAGE + wr[t][j]);
            f32x4 P[MT][NTT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
              for (int t = 0; t < NTT; ++t) {
                P[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][0], wfrag<4>(wv[t][0]),
                                                                   f32x4{}, 0, 0, 0);
                P[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][1], wfrag<4>(wv[t][1]),
                                                                   P[mt][t], 0, 0, 0);
              }
#pragma unroll
            for (int t = 0; t < NTT; ++t) {
              const float s = (j & 1) ? bf16_hi(sv[p][t][j >> 1]) : bf16_lo(sv[p][t][j >> 1]);
              const float b = (j & 1) ? bf16_hi(bv[p][t][j >> 1]) : bf16_lo(bv[p][t][j >> 1]);
              const float bo = __builtin_fmaf(-128.f, s, b);
              if constexpr (FOLD) bsel[p][t] = qmvs_pick(j, bo, bsel[p][t]);
#pragma unroll
              for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                  acc[p][mt][t][r] = __builtin_fmaf(
                      s, P[mt][t][r],
                      FOLD ? acc[p][mt][t][r] : __builtin_fmaf(bo, xr[mt][r], acc[p][mt][t][r]));
            }
          }
          if (FOLD && (j & 3) == 3) {
#pragma unroll
            for (int p = 0; p < NMAT; ++p)
#pragma unroll
              for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int t = 0; t < NTT; ++t)
                  acc[p][mt][t] = qmvs_bias4(xsel[mt], bsel[p][t], acc[p][mt][t]);
          }
        }
      }
    }
  }
}

typedef __attribute__((address_space(3))) void qmvs_lds_t;

// s_waitcnt vmcnt(N) lgkmcnt(0) (gfx9 encoding, expcnt left alone).
template <int N>
__device__ __forceinline__ void qmvs_wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// Bytes of one row of the block-shared x stage: one 4-unit step, 256 bf16 values.
constexpr int kXStageRow = 512;

// The walk of qmvs_slice for a block of WV (4 or 8) waves that all walk the same
// steps [s0, s1) of 256 K values (each wave its own 16 NTT columns from nb), with
// the segment's x rows shared through LDS instead of loaded by every wave.
//
// x stage (xs0 / xs1, one step each, alternating): 16 MTW rows of kXStageRow
// bytes; 16-byte chunk c of row r sits at position c ^ (r & 15), so the 16 rows
// an A-fragment read touches at one chunk fall on distinct banks.  The block
// fills a stage with buffer_load ... lds (no VGPR staging): with AX = 8 MTW / WV
// instructions per wave, instruction j of wave `wave` covers rows 2 (AX wave + j)
// and the next, lane L landing at row + L / 32,
// position L % 32; xo[j] is that lane's byte offset (its x row and swizzled
// chunk) in xres, and a step adds kXStageRow bytes.  An instruction whose two
// rows are both at or past the segment's length `len` is not issued (its stage
// rows keep stale bytes, which reach only accumulator rows that are never stored).
//
// Step st waits for its x stage (vmcnt then s_barrier: each wave's DMA has
// landed and every wave has left step st - 1, whose stage the next DMA
// overwrites), DMAs the x of step st + 1, stages its weights (loaded two steps
// ahead, as in qmvs_slice) and runs the MFMAs.  Skipped DMA instructions change
// no wait: the explicit wait counts only the weight loads issued after a step's
// x.  Only acc[.][0, MTW) is touched.
//
// DEQ (not with FOLD): the weights are dequantized instead, w = bf16(fma(s, q, b))
// in natural order (deq_frag4), and the MFMAs accumulate x . w straight into acc
// with x read in natural order: no Σx MFMAs, no per-group corrections and no x
// permutation, for 22 VALU per packed word instead of 7.  The word's VALU is
// shared by the MTW x tiles, so it pays from 2 tiles (17 to 64 x rows).
//
// BITS = 8 (with DEQ only): 256-byte row slices per step (16-chunk stage rows), and
// lane (c, q) reads chunk 4 j + q of its row's unit j, the 16 values that its two
// MFMAs of the unit take (words 0-1 and 2-3, deq_frag8); the x fragments are those
// of the int4 walk.
template <int MTW, int MT, int NTT, int NMAT, int WV, bool FOLD, bool DEQ = false, int BITS = 4>
__device__ __forceinline__ void qmvs_walk_xlds(uint8_t* xs0, uint8_t* xs1, uint8_t* stage,
                                               __amdgpu_buffer_rsrc_t xres,
                                               const uint32_t (&xo)[8 * MTW / WV], int wave,
                                               int64_t len,
                                               const uint32_t* const (&w)[NMAT],
                                               const uint16_t* const (&sc)[NMAT],
                                               const uint16_t* const (&bi)[NMAT], int64_t nb,
                                               int64_t N, int64_t K, int64_t s0, int64_t s1,
                                               f32x4 (&acc)[NMAT][MT][NTT]) {
  constexpr int SU = 4;
  using G = QmvsGeom<NTT, SU, BITS>;
  constexpr int NI = G::NI, LPR = G::LPR, RB = G::RB, ROWS = G::ROWS, SPL = G::SPL;
  constexpr int AX = 8 * MTW / WV;
  static_assert(MTW <= MT, "walked tiles");
  static_assert(AX >= 1 && AX * WV == 8 * MTW, "x DMA split over the block's waves");
  static_assert(BITS == 4 || (BITS == 8 && DEQ), "int8 weights are dequantized");
  using wv_t = std::conditional_t<BITS == 8, u32x4, u32x2>;
  typedef uint32_t sbv_t __attribute__((ext_vector_type(SPL / 2)));
  const int lane = threadIdx.x & 63;
  const int c16 = lane & 15, q = lane >> 4;
  const int64_t wpr = K * BITS / 32, gpr = K / 64;

  // Weights through buffer resources as in qmvs_slice: steps past s1 load zeros
  // without a memory access.
  uint32_t wq[NI];
  int wo[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int r = i * (64 / LPR) + lane / LPR;
    int64_t n = nb + r;
    n = n < N ? n : N - 1;
    wq[i] = (uint32_t)((n * wpr + (lane % LPR) * 4) * 4);
    wo[i] = r * RB + (qmvs_pos<RB / 32>(lane % LPR, r) << 4);
  }
  __amdgpu_buffer_rsrc_t wres[NMAT];
#pragma unroll
  for (int p = 0; p < NMAT; ++p)
    wres[p] = __builtin_amdgcn_make_buffer_rsrc((void*)w[p], (short)0, (int)(N * wpr * 4), 0x00020000);
  int wr[NTT][SU];
#pragma unroll
  for (int t = 0; t < NTT; ++t)
#pragma unroll
    for (int j = 0; j < SU; ++j) {
      const int r = 16 * t + c16;
      wr[t][j] = BITS == 8 ? r * RB + (qmvs_pos<RB / 32>(4 * j + q, r) << 4)
                           : r * RB + (qmvs_pos<RB / 32>(2 * j + (q >> 1), r) << 4) + (q & 1) * 8;
    }
  // Scale/bias loads.  16-row tiles (NTT = 1): one 8-byte load per lane covers two
  // steps (lane -> row l % 16, kind (l / 16) & 1 (scales, biases), step l / 32 of
  // the pair: that step's 4 groups), issued in even steps (counted from s0) for
  // the next pair; a lane's step is clamped to s1 - 1, so an odd step count reads
  // no further.
  // 32-row tiles: one load per lane and step as in qmvs_slice.
  constexpr bool PAIR = ROWS == 16;
  typedef uint32_t spv_t __attribute__((ext_vector_type(2)));
  const int sh = lane / ROWS;
  int64_t nrow = nb + lane % ROWS;
  nrow = nrow < N ? nrow : N - 1;
  const int64_t soff =
      nrow * gpr + ((PAIR || 64 / ROWS == 2) ? 0 : (sh >> 1) * SPL);
  const uint16_t* sbrow[NMAT];
#pragma unroll
  for (int p = 0; p < NMAT; ++p) sbrow[p] = ((sh & 1) ? bi[p] : sc[p]) + soff;
  const int ph = lane >> 5;  // step of the pair (PAIR)
  // A-fragment byte offsets in a stage: row 16 mt + c16, chunk 8 j + 2 q (+1).
  int xa[SU][2];
#pragma unroll
  for (int j = 0; j < SU; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) xa[j][h] = c16 * kXStageRow + (((8 * j + 2 * q + h) ^ c16) << 4);

  u32x4 wbuf[2][NMAT][NI];
  sbv_t sbuf[2][NMAT];
  spv_t sp[NMAT], held[NMAT];
  // Weights (and, without PAIR, the step's scales) of step st into set d; with PAIR
  // and pair set, the scales of steps st and st + 1 after the weights.
  auto load_w = [&](int d, int64_t st, bool pair) {
    const bool past = st >= s1;
    st = past ? s1 - 1 : st;
#pragma unroll
    for (int p = 0; p < NMAT; ++p) {
#pragma unroll
      for (int i = 0; i < NI; ++i)
        wbuf[d][p][i] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       wres[p], past ? (int)0x80000000u : (int)(wq[i] + (uint32_t)st * RB), 0,
                       2 /* nt */));
      if constexpr (!PAIR) sbuf[d][p] = *reinterpret_cast<const sbv_t*>(sbrow[p] + st * SU);
    }
    if constexpr (PAIR) {
      if (pair) {
        int64_t sl = st + ph;
        sl = sl < s1 ? sl : s1 - 1;
#pragma unroll
        for (int p = 0; p < NMAT; ++p) sp[p] = *reinterpret_cast<const spv_t*>(sbrow[p] + sl * SU);
      }
    }
  };
  auto issue_x = [&](int64_t st, uint8_t* xs) {
#pragma unroll
    for (int j = 0; j < AX; ++j)
      if (2 * (wave * AX + j) < len)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (qmvs_lds_t*)(xs + (wave * AX + j) * 1024),
                                                 16, (int)xo[j], (int)(st * kXStageRow), 0, 0);
  };

  if (s1 <= s0) return;
  issue_x(s0, xs0);
  __builtin_amdgcn_sched_barrier(0);
  load_w(0, s0, true);
  load_w(1, s0 + 1, false);
  __builtin_amdgcn_sched_barrier(0);
  // One step; e (0 or 1) picks the stage and register set.  Pairs of steps run
  // unconditionally inside the loop and an odd last step after it, so every path
  // into a step has issued the same loads (the compiler then waits for no more
  // than the explicit wait does).
  auto step = [&](auto ec, int64_t stp) {
    constexpr int e = decltype(ec)::value;
    uint8_t* xc = e ? xs1 : xs0;
    uint8_t* xn = e ? xs0 : xs1;
    // Issued after this step's x: the loads of step stp + 1's weights, and with
    // PAIR the scales of the pair that follows (loaded in even steps only).
    if constexpr (PAIR && e == 0) qmvs_wait_vm_lgkm0<NMAT * NI>();
    else qmvs_wait_vm_lgkm0<NMAT * (NI + 1)>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // The weight stage is written and read back (B words of all SU units), and
    // the scale and bias pairs shuffled, before the next x DMA goes out: LDS
    // accesses after it that the compiler cannot tell apart from its target
    // would wait for it.
#pragma unroll
    for (int p = 0; p < NMAT; ++p)
#pragma unroll
      for (int i = 0; i < NI; ++i)
        *reinterpret_cast<u32x4*>(stage + p * G::STAGE + wo[i]) = wbuf[e][p][i];
    wv_t wv[SU][NMAT][NTT];
#pragma unroll
    for (int j = 0; j < SU; ++j)
#pragma unroll
      for (int p = 0; p < NMAT; ++p)
#pragma unroll
        for (int t = 0; t < NTT; ++t)
          wv[j][p][t] = *reinterpret_cast<const wv_t*>(stage + p * G::STAGE + wr[t][j]);
    uint32_t sv[NMAT][NTT][SU / 2], bv[NMAT][NTT][SU / 2];
    if constexpr (PAIR) {
      if constexpr (e == 0) {
#pragma unroll
        for (int p = 0; p < NMAT; ++p) held[p] = sp[p];
      }
#pragma unroll
      for (int p = 0; p < NMAT; ++p)
#pragma unroll
        for (int k = 0; k < SU / 2; ++k) {
          sv[p][0][k] = (uint32_t)__shfl((int)held[p][k], 32 * e + c16, 64);
          bv[p][0][k] = (uint32_t)__shfl((int)held[p][k], 32 * e + 16 + c16, 64);
        }
    } else {
      sbv_t mine[NMAT];
#pragma unroll
      for (int p = 0; p < NMAT; ++p) mine[p] = sbuf[e][p];
#pragma unroll
      for (int p = 0; p < NMAT; ++p)
#pragma unroll
        for (int t = 0; t < NTT; ++t)
#pragma unroll
          for (int k = 0; k < SU / 2; ++k) {
            const int row = 16 * t + c16;
            const int hi = (64 / ROWS == 2) ? 0 : k / (SPL / 2);
            const int idx = (64 / ROWS == 2) ? k : k % (SPL / 2);
            sv[p][t][k] = (uint32_t)__shfl((int)mine[p][idx], (2 * hi) * ROWS + row, 64);
            bv[p][t][k] = (uint32_t)__shfl((int)mine[p][idx], (2 * hi + 1) * ROWS + row, 64);
          }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (stp + 1 < s1) issue_x(stp + 1, xn);
    __builtin_amdgcn_sched_barrier(0);
    load_w(e, stp + 2, e == 0);
    __builtin_amdgcn_sched_barrier(0);
    float xsel[MTW] = {}, bsel[NMAT][NTT] = {};
    f32x4 xr[MTW];
#pragma unroll
    for (int j = 0; j < SU; ++j) {
      if constexpr (DEQ) {
        static_assert(!FOLD, "DEQ accumulates the dequantized product directly");
        bf16x8 A[MTW][2];
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            A[mt][h] = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(xc + mt * 16 * kXStageRow + xa[j][h]));
#pragma unroll
        for (int p = 0; p < NMAT; ++p)
#pragma unroll
          for (int t = 0; t < NTT; ++t) {
            const float s = (j & 1) ? bf16_hi(sv[p][t][j >> 1]) : bf16_lo(sv[p][t][j >> 1]);
            const float b = (j & 1) ? bf16_hi(bv[p][t][j >> 1]) : bf16_lo(bv[p][t][j >> 1]);
            bf16x8 B0, B1;
            if constexpr (BITS == 8) {
              B0 = deq_frag8(wv[j][p][t][0], wv[j][p][t][1], s, b);
              B1 = deq_frag8(wv[j][p][t][2], wv[j][p][t][3], s, b);
            } else {
              B0 = deq_frag4(wv[j][p][t][0], s, s * 0.0625f, b);
              B1 = deq_frag4(wv[j][p][t][1], s, s * 0.0625f, b);
            }
#pragma unroll
            for (int mt = 0; mt < MTW; ++mt) {
              acc[p][mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][0], B0, acc[p][mt][t], 0, 0, 0);
              acc[p][mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][1], B1, acc[p][mt][t], 0, 0, 0);
            }
          }
        continue;
      }
      bf16x8 A[MTW][2];
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) {
        A[mt][0] = xfrag4(*reinterpret_cast<const u32x4*>(xc + mt * 16 * kXStageRow + xa[j][0]));
        A[mt][1] = xfrag4(*reinterpret_cast<const u32x4*>(xc + mt * 16 * kXStageRow + xa[j][1]));
      }
#pragma unroll
      for (int mt = 0; mt < MTW; ++mt) {
        if constexpr (FOLD) xsel[mt] = qmvs_pick(j, qmvs_xsum(A[mt]), xsel[mt]);
        else xr[mt] = qmvs_xsum_rows(A[mt]);
      }
#pragma unroll
      for (int p = 0; p < NMAT; ++p) {
        f32x4 P[MTW][NTT];
#pragma unroll
        for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
          for (int t = 0; t < NTT; ++t) {
            P[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                A[mt][0], wfrag<4>(wv[j][p][t][0]), f32x4{}, 0, 0, 0);
            P[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                A[mt][1], wfrag<4>(wv[j][p][t][1]), P[mt][t], 0, 0, 0);
          }
#pragma unroll
        for (int t = 0; t < NTT; ++t) {
          const float s = (j & 1) ? bf16_hi(sv[p][t][j >> 1]) : bf16_lo(sv[p][t][j >> 1]);
          const float b = (j & 1) ? bf16_hi(bv[p][t][j >> 1]) : bf16_lo(bv[p][t][j >> 1]);
          const float bo = __builtin_fmaf(-128.f, s, b);
          if constexpr (FOLD) bsel[p][t] = qmvs_pick(j, bo, bsel[p][t]);
#pragma unroll
          for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              acc[p][mt][t][r] = __builtin_fmaf(
                  s, P[mt][t][r],
                  FOLD ? acc[p][mt][t][r] : __builtin_fmaf(bo, xr[mt][r], acc[p][mt][t][r]));
        }
      }
      if (FOLD && (j & 3) == 3) {
#pragma unroll
        for (int p = 0; p < NMAT; ++p)
#pragma unroll
          for (int mt = 0; mt < MTW; ++mt)
#pragma unroll
            for (int t = 0; t < NTT; ++t)
              acc[p][mt][t] = qmvs_bias4(xsel[mt], bsel[p][t], acc[p][mt][t]);
      }
    }
  };
  int64_t st = s0;
#pragma clang loop unroll(disable)
  for (; st + 1 < s1; st += 2) {
    step(std::integral_constant<int, 0>{}, st);
    step(std::integral_constant<int, 1>{}, st + 1);
  }
  if (st < s1) step(std::integral_constant<int, 0>{}, st);
  qmvs_wait_vm_lgkm0<0>();
}

// The dense form of qmvs_walk_xlds for walks of at most D steps, with every load
// of the walk issued before the first step: each wave loads the scale/bias words
// of its D steps, the block DMAs the x rows of all D steps into D stage slots
// (xs + d * 16 MT kXStageRow; slot layout as above, every DMA instruction issued,
// rows past the x rows re-reading a valid one), then each wave loads the weights
// of its D steps into registers.  One wait (vmcnt: the weight loads issued after the last x DMA) and
// one s_barrier make all x slots visible to all waves; step d then waits only for
// its own weights.  So the walk pays one memory round trip rather than one per
// step.  Steps d with s0 + d >= s1 load from clamped
// addresses (weights from an offset past the buffer, which reads zeros without
// a memory access) and are not computed.
// DEQ: the weights dequantized and x in natural order, as in qmvs_walk_xlds, and
// BITS = 8 with it as there.
template <int MT, int NTT, int WV, int D, bool DEQ = false, int BITS = 4>
__device__ __forceinline__ void qmvs_walk_xall(uint8_t* xs, uint8_t* stage, __amdgpu_buffer_rsrc_t xres,
                                               const uint32_t (&xo)[8 * MT / WV], int wave,
                                               const uint32_t* w, const uint16_t* sc,
                                               const uint16_t* bi, int64_t nb, int64_t N, int64_t K,
                                               int64_t s0, int64_t s1, f32x4 (&acc)[MT][NTT]) {
  constexpr int SU = 4;
  using G = QmvsGeom<NTT, SU, BITS>;
  constexpr int NI = G::NI, LPR = G::LPR, RB = G::RB, ROWS = G::ROWS, SPL = G::SPL;
  constexpr int AX = 8 * MT / WV;
  constexpr int XSLOT = 16 * MT * kXStageRow;
  static_assert(AX >= 1 && AX * WV == 8 * MT, "x DMA split over the block's waves");
  static_assert(D >= 1 && D * NI < 64, "vmcnt range");
  static_assert(BITS == 4 || (BITS == 8 && DEQ), "int8 weights are dequantized");
  using wv_t = std::conditional_t<BITS == 8, u32x4, u32x2>;
  typedef uint32_t sbv_t __attribute__((ext_vector_type(SPL / 2)));
  const int lane = threadIdx.x & 63;
  const int c16 = lane & 15, q = lane >> 4;
  const int64_t wpr = K * BITS / 32, gpr = K / 64;
  if (s1 <= s0) return;

  uint32_t wq[NI];
  int wo[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int r = i * (64 / LPR) + lane / LPR;
    int64_t n = nb + r;
    n = n < N ? n : N - 1;
    wq[i] = (uint32_t)((n * wpr + (lane % LPR) * 4) * 4);
    wo[i] = r * RB + (qmvs_pos<RB / 32>(lane % LPR, r) << 4);
  }
  const __amdgpu_buffer_rsrc_t wres =
      __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, (int)(N * wpr * 4), 0x00020000);
  int wr[NTT][SU];
#pragma unroll
  for (int t = 0; t < NTT; ++t)
#pragma unroll
    for (int j = 0; j < SU; ++j) {
      const int r = 16 * t + c16;
      wr[t][j] = BITS == 8 ? r * RB + (qmvs_pos<RB / 32>(4 * j + q, r) << 4)
                           : r * RB + (qmvs_pos<RB / 32>(2 * j + (q >> 1), r) << 4) + (q & 1) * 8;
    }
  // Scale/bias words as in qmvs_slice: lane -> row l % ROWS, kind (l / ROWS) & 1,
  // and for 16-row tiles which half of the step's groups (l / ROWS / 2).
  const int sh = lane / ROWS;
  int64_t nrow = nb + lane % ROWS;
  nrow = nrow < N ? nrow : N - 1;
  const uint16_t* sbrow = ((sh & 1) ? bi : sc) + nrow * gpr + ((64 / ROWS == 2) ? 0 : (sh >> 1) * SPL);
  int xa[SU][2];
#pragma unroll
  for (int j = 0; j < SU; ++j)
#pragma unroll
    for (int h = 0; h < 2; ++h) xa[j][h] = c16 * kXStageRow + (((8 * j + 2 * q + h) ^ c16) << 4);

  // Issue order: scale/bias words, x DMAs, weights.  The wait for x then counts
  // only the weight loads (16-byte loads, which the compiler cannot merge), however
  // the scale loads were combined.
  u32x4 wbuf[D][NI];
  sbv_t sbuf[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int64_t st = s0 + d < s1 ? s0 + d : s1 - 1;
    sbuf[d] = *reinterpret_cast<const sbv_t*>(sbrow + st * SU);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int64_t st = s0 + d < s1 ? s0 + d : s1 - 1;
#pragma unroll
    for (int j = 0; j < AX; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xres, (qmvs_lds_t*)(xs + d * XSLOT + (wave * AX + j) * 1024), 16, (int)xo[j],
          (int)(st * kXStageRow), 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const bool past = s0 + d >= s1;
    const int64_t st = past ? s1 - 1 : s0 + d;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      wbuf[d][i] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                     wres, past ? (int)0x80000000u : (int)(wq[i] + (uint32_t)st * RB), 0,
                     2 /* nt */));
  }
  __builtin_amdgcn_sched_barrier(0);
  qmvs_wait_vm_lgkm0<D * NI>();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  const bf16x8 ones = as_bf16x8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);

#pragma unroll
  for (int d = 0; d < D; ++d) {
    if (s0 + d >= s1) break;
    const uint8_t* xc = xs + d * XSLOT;
#pragma unroll
    for (int i = 0; i < NI; ++i)
      *reinterpret_cast<u32x4*>(stage + wo[i]) = wbuf[d][i];
    wv_t wv[SU][NTT];
#pragma unroll
    for (int j = 0; j < SU; ++j)
#pragma unroll
      for (int t = 0; t < NTT; ++t)
        wv[j][t] = *reinterpret_cast<const wv_t*>(stage + wr[t][j]);
    uint32_t sv[NTT][SU / 2], bv[NTT][SU / 2];
#pragma unroll
    for (int t = 0; t < NTT; ++t)
#pragma unroll
      for (int k = 0; k < SU / 2; ++k) {
        const int row = 16 * t + c16;
        const int hi = (64 / ROWS == 2) ? 0 : k / (SPL / 2);
        const int idx = (64 / ROWS == 2) ? k : k % (SPL / 2);
        sv[t][k] = (uint32_t)__shfl((int)sbuf[d][idx], (2 * hi) * ROWS + row, 64);
        bv[t][k] = (uint32_t)__shfl((int)sbuf[d][idx], (2 * hi + 1) * ROWS + row, 64);
      }
#pragma unroll
    for (int j = 0; j < SU; ++j) {
      if constexpr (DEQ) {
        bf16x8 A[MT][2];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            A[mt][h] = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(xc + mt * 16 * kXStageRow + xa[j][h]));
#pragma unroll
        for (int t = 0; t < NTT; ++t) {
          const float sf = (j & 1) ? bf16_hi(sv[t][j >> 1]) : bf16_lo(sv[t][j >> 1]);
          const float bf = (j & 1) ? bf16_hi(bv[t][j >> 1]) : bf16_lo(bv[t][j >> 1]);
          bf16x8 B0, B1;
          if constexpr (BITS == 8) {
            B0 = deq_frag8(wv[j][t][0], wv[j][t][1], sf, bf);
            B1 = deq_frag8(wv[j][t][2], wv[j][t][3], sf, bf);
          } else {
            B0 = deq_frag4(wv[j][t][0], sf, sf * 0.0625f, bf);
            B1 = deq_frag4(wv[j][t][1], sf, sf * 0.0625f, bf);
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][0], B0, acc[mt][t], 0, 0, 0);
            acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][1], B1, acc[mt][t], 0, 0, 0);
          }
        }
        continue;
      }
      bf16x8 A[MT][2];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        A[mt][0] = xfrag4(*reinterpret_cast<const u32x4*>(xc + mt * 16 * kXStageRow + xa[j][0]));
        A[mt][1] = xfrag4(*reinterpret_cast<const u32x4*>(xc + mt * 16 * kXStageRow + xa[j][1]));
      }
      f32x4 xsum[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        xsum[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][0], ones, f32x4{}, 0, 0, 0);
        xsum[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][1], ones, xsum[mt], 0, 0, 0);
      }
      f32x4 P[MT][NTT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < NTT; ++t) {
          P[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][0], wfrag<4>(wv[j][t][0]),
                                                             f32x4{}, 0, 0, 0);
          P[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[mt][1], wfrag<4>(wv[j][t][1]),
                                                             P[mt][t], 0, 0, 0);
        }
#pragma unroll
      for (int t = 0; t < NTT; ++t) {
        const float sf = (j & 1) ? bf16_hi(sv[t][j >> 1]) : bf16_lo(sv[t][j >> 1]);
        const float bf = (j & 1) ? bf16_hi(bv[t][j >> 1]) : bf16_lo(bv[t][j >> 1]);
        const float bo = __builtin_fmaf(-128.f, sf, bf);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[mt][t][r] = __builtin_fmaf(sf, P[mt][t][r], __builtin_fmaf(bo, xsum[mt][r], acc[mt][t][r]));
      }
    }
  }
}

}  // namespace fmxq
