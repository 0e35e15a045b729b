// fmxq_skinny.hip -- MFMA GEMV for 5 <= M <= 32 (speculative verify, small
// decode batches): quantized_matmul rows that are too many for the dot2 GEMV
// and too few to amortise an LDS-dequantised GEMM tile.
//
// Replaces mlx_quantized_matmul (mlxgo/binding_cgo.go:636-643) for
// x [M, K] with M = batch * (k+1) draft positions (the verify step of
// pipeline/pipeline.go:56-65) or small decode batches (llama.go:403).
//
// Both kernels take the weights as the MFMA B operand in the exponent-trick
// form bf16(offset + q) and fold the scale in per group:
//   P = sum_k x (offset + q), xs = sum_k x (an MFMA against ones),
//   acc += s * P + (b - offset * s) * xs.
//
// qmvs_kernel (int4, group 64; the decode-batch and verify shapes):
//   - v_mfma_f32_16x16x32_bf16; a wave owns 16 NTT output columns and MT
//     16-row tiles of x, and one K slice of the block's row range;
//   - the packed weights are read coalesced (each load instruction covers whole
//     128- or 256-byte row segments of 4 or 8 rows) into a per-wave LDS stage
//     and read back in the B-operand layout: lane (c = l % 16, q = l / 16)
//     holds words 2q, 2q+1 of its row's 64-value unit, MFMA i takes word 2q+i;
//   - scales and biases of a step arrive as one 8-byte load per lane and are
//     passed to the lanes that need them with ds_bpermute;
//   - A = x: lane (m = l % 16, q) loads x[m][64u + 16q .. +16] (two 16-byte
//     pieces) XD units ahead.
//   Reading the weights in the B-operand layout straight from memory (one
//   instruction spanning 32 rows at 32 bytes each) runs at under half the HBM
//   rate of these whole-segment loads.
//
// qmv_mfma_kernel (every other int4/int8 case):
//   v_mfma_f32_32x32x16_bf16 with the weights straight from registers, no LDS:
//   - lane l holds output column n = l % 32 and, for each 16-byte load, 32 int4
//     (16 int8) values of row n; lane halves g = l / 32 cover the two halves of a
//     64-value (32-value for int8) unit, so every MFMA step sums over one
//     quantization group only (group_size >= 64 for int4, >= 32 for int8);
//   - B values are bf16(128 + q) from the exponent trick (0x4300 | q); int8
//     values are split into two nibbles, the high one as bf16(2048 + 16 q_hi)
//     (0x4500 | q_hi), so each int8 element occupies two MFMA k slots;
//   - A = x in the matching pair order, loaded per unit from global memory
//     (rows >= M read a valid row; their outputs are discarded).
// In both the K axis is split over the KS waves of a block, which meet in LDS.
//
// qmvw_kernel (int4, group 64, 9 <= M <= 64 where it wins: M > 16, or wide
// outputs / long rows at M <= 16):
//   - the same 16x16x32 tile walk, but the WV waves of a block (4; 8 for 64-row
//     x tiles on the pipelined walk) own WV W tiles side by side over one K part
//     and share the block's x rows, which the block
//     DMAs into LDS (buffer_load ... lds) once per step: qmvs reads x once per
//     wave, and at M = 16 that is twice the weight bytes through the texture
//     units (isolating the two streams on MI355X: x, not the weights, set the
//     qmvs time);
//   - the K parts of a row block are separate blocks (grid y) writing fp32
//     partials; qmvw_fixup_kernel sums them in part order and rounds;
//   - walks of at most 4 steps issue every load first (qmvs_walk_xall), longer
//     ones double-buffer x one step ahead (qmvs_walk_xlds).
#include <algorithm>

#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"
#include "fmxq_mfma_frag.hpp"
#include "fmxq_qmvs.hpp"

namespace fmxq {

template <int NT>
struct SkStage {
  u32x4 w[NT];
  uint32_t sb[NT];
  u32x4 x[4];  // int4: four 16-byte x pieces; int8: two (x[0], x[1]) used
};

// NT: 32-row tiles per wave.  RL: accumulator registers carrying rows < M
// (4 per 8 rows).  KS: waves of a block splitting K; WAVES: waves per block.
template <int BITS, int NT, int RL, int KS, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void qmv_mfma_kernel(QmmArgs a) {
  constexpr int RG = WAVES / KS;
  constexpr int U = BITS == 4 ? 64 : 32;            // values per unit (two 16-byte halves)
  constexpr float OFF = BITS == 4 ? 128.f : 2176.f;  // exponent-trick offset per value
  constexpr float XSCALE = BITS == 4 ? 1.f : 0.5f;   // int8 A duplicates each x value
  __shared__ float red[KS > 1 ? RG : 1][KS > 1 ? KS - 1 : 1][NT][RL][64];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = wave / KS, ks = wave % KS;
  const int ml = lane & 31, half = lane >> 5;
  const int64_t nb = ((int64_t)blockIdx.x * RG + rg) * 32 * NT;
  const int64_t nu = a.K / U;
  const int64_t u0 = ks * nu / KS, u1 = (ks + 1) * nu / KS;
  const int gshift = __builtin_ctz((unsigned)a.group_size);  // a power of two
  const int64_t wpr = a.K * BITS / 32, gpr = a.K >> gshift;
  const int mrow = ml < a.M ? ml : (int)a.M - 1;
  const uint16_t* xrow = a.x + (int64_t)mrow * a.ldx + half * (U / 2);

  const uint32_t* wrow[NT];
  const uint16_t* srow[NT];
  const uint16_t* brow[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int64_t n = nb + t * 32 + ml;
    n = n < a.N ? n : a.N - 1;
    wrow[t] = a.w + n * wpr + half * 4;
    srow[t] = a.scales + n * gpr;
    brow[t] = a.biases + n * gpr;
  }

  auto load = [&](SkStage<NT>& st, int64_t u) {
    u = u < u1 ? u : u1 - 1;  // tail loads re-read the last unit; never computed
    const int64_t g = (u * U + half * (U / 2)) >> gshift;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      st.w[t] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow[t] + u * 8));
      st.sb[t] = (uint32_t)srow[t][g] | ((uint32_t)brow[t][g] << 16);
    }
    const u32x4* xs = reinterpret_cast<const u32x4*>(xrow + u * U);
    if constexpr (BITS == 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) st.x[j] = xs[j];
    } else {
      st.x[0] = xs[0];
      st.x[1] = xs[1];
    }
  };

  f32x16 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x16{};
  const bf16x8 ones = as_bf16x8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);

  auto compute = [&](const SkStage<NT>& st) {
    bf16x8 A[4];
    if constexpr (BITS == 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) A[j] = xfrag4(st.x[j]);
    } else {
      A[0] = xfrag8(st.x[0][0], st.x[0][1]);
      A[1] = xfrag8(st.x[0][2], st.x[0][3]);
      A[2] = xfrag8(st.x[1][0], st.x[1][1]);
      A[3] = xfrag8(st.x[1][2], st.x[1][3]);
    }
    f32x16 xs = {};
    f32x16 P[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) P[t] = f32x16{};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      xs = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[j], ones, xs, 0, 0, 0);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        P[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[j], wfrag<BITS>(st.w[t][j]), P[t], 0, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float s = bf16_lo(st.sb[t]);
      const float bo = __builtin_fmaf(-OFF, s, bf16_hi(st.sb[t])) * XSCALE;
#pragma unroll
      for (int r = 0; r < RL; ++r) acc[t][r] = __builtin_fmaf(s, P[t][r], __builtin_fmaf(bo, xs[r], acc[t][r]));
    }
  };

  if (u1 > u0) {
    SkStage<NT> s0, s1;
    load(s0, u0);
    load(s1, u0 + 1);
    for (int64_t u = u0; u < u1; u += 2) {
      compute(s0);
      load(s0, u + 2);
      if (u + 1 < u1) compute(s1);
      load(s1, u + 3);
    }
  }

  if constexpr (KS > 1) {
    if (ks > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < RL; ++r) red[rg][ks - 1][t][r][lane] = acc[t][r];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int r = 0; r < RL; ++r)
#pragma unroll
        for (int v = 0; v < KS - 1; ++v) acc[t][r] += red[rg][v][t][r][lane];
  }
  // C layout of a 32x32 tile: register r of lane l is row 8*(r/4) + 4*(l/32) + r%4,
  // column l%32.
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t n = nb + t * 32 + ml;
#pragma unroll
    for (int r = 0; r < RL; ++r) {
      const int64_t m = (r / 4) * 8 + half * 4 + (r % 4);
      if (m < a.M && n < a.N) a.y[m * a.ldy + n] = finish_out(acc[t][r], a.bias, n);
    }
  }
}

bool qmv_mfma_supported(const QmmArgs& a) {
  if (a.M < 1 || a.M > 32) return false;
  if (a.bits == 4) return a.group_size >= 64 && a.K % 64 == 0;
  return a.group_size >= 32 && a.K % 32 == 0;
}

template <int BITS, int NT, int RL, int KS, int WAVES>
static hipError_t launch_sk(const QmmArgs& a, hipStream_t stream) {
  constexpr int rows_per_block = (WAVES / KS) * 32 * NT;
  const unsigned blocks = (unsigned)((a.N + rows_per_block - 1) / rows_per_block);
  qmv_mfma_kernel<BITS, NT, RL, KS, WAVES><<<blocks, WAVES * 64, 0, stream>>>(a);
  return hipGetLastError();
}

template <int BITS, int RL>
static hipError_t launch_sk_rl(const QmmArgs& a, hipStream_t stream) {
  // Split K over the waves of a block until the launch has about 2048 waves
  // (eight per CU), keeping at least eight units per wave: a 32-row tile per
  // wave is too few waves for narrow outputs (4096 rows: 128 tiles).
  const int64_t tiles = (a.N + 31) / 32;
  const int64_t units = a.K / (BITS == 4 ? 64 : 32);
  int ks = 1;
  while (ks < 16 && tiles * ks < 2048 && units / (2 * ks) >= 8) ks *= 2;
  switch (ks) {
    case 1: return launch_sk<BITS, 1, RL, 1, 4>(a, stream);
    case 2: return launch_sk<BITS, 1, RL, 2, 4>(a, stream);
    case 4: return launch_sk<BITS, 1, RL, 4, 4>(a, stream);
    case 8: return launch_sk<BITS, 1, RL, 8, 8>(a, stream);
    default: return launch_sk<BITS, 1, RL, 16, 16>(a, stream);
  }
}

hipError_t launch_qmv_mfma(const QmmArgs& a, hipStream_t stream) {
  const int rl = (int)((a.M + 7) / 8) * 4;
  if (a.bits == 4) {
    switch (rl) {
      case 4: return launch_sk_rl<4, 4>(a, stream);
      case 8: return launch_sk_rl<4, 8>(a, stream);
      case 12: return launch_sk_rl<4, 12>(a, stream);
      default: return launch_sk_rl<4, 16>(a, stream);
    }
  }
  switch (rl) {
    case 4: return launch_sk_rl<8, 4>(a, stream);
    case 8: return launch_sk_rl<8, 8>(a, stream);
    case 12: return launch_sk_rl<8, 12>(a, stream);
    default: return launch_sk_rl<8, 16>(a, stream);
  }
}

// ---------------------------------------------------------------------------
// qmvs_kernel.  Block: KS waves over the same 16 NTT rows, each wave a
// contiguous run of SU-unit steps walked by qmvs_slice (fmxq_qmvs.hpp); the
// slices meet in LDS.

namespace {

constexpr int kQmvsKS = 4;  // waves (K slices) per block

template <int MT, int NTT, int SU>
__global__ __launch_bounds__(kQmvsKS * 64) void qmvs_kernel(QmmArgs a) {
  constexpr int KS = kQmvsKS;
  using G = QmvsGeom<NTT, SU>;
  __shared__ __attribute__((aligned(16))) uint8_t stage[KS][G::STAGE];
  __shared__ float red[KS - 1][MT][NTT][4][64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, q = lane >> 4;
  const int64_t nb = (int64_t)blockIdx.x * G::ROWS;
  const int64_t nst = a.K / (SU * 64);
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + c16;
    xrow[mt] = a.x + (int64_t)(m < a.M ? m : (int)a.M - 1) * a.ldx + q * 16;
  }
  f32x4 acc[1][MT][NTT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NTT; ++t) acc[0][mt][t] = f32x4{};
  const uint32_t* const w[1] = {a.w};
  const uint16_t* const sc[1] = {a.scales};
  const uint16_t* const bi[1] = {a.biases};
  qmvs_slice<MT, NTT, SU, 1, false>(stage[wave], w, sc, bi, nb, a.N, a.K, xrow, wave * nst / KS,
                             (wave + 1) * nst / KS, acc);

  if (wave > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < NTT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave - 1][mt][t][r][lane] = acc[0][mt][t][r];
  }
  __syncthreads();
  if (wave > 0) return;
  // C layout of a 16x16 tile: register r of lane l is row 4 (l / 16) + r,
  // column l % 16.
#pragma unroll
  for (int t = 0; t < NTT; ++t) {
    const int64_t n = nb + 16 * t + c16;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = acc[0][mt][t][r];
#pragma unroll
        for (int k = 0; k < KS - 1; ++k) v += red[k][mt][t][r][lane];
        const int64_t m = 16 * mt + 4 * q + r;
        if (m < a.M && n < a.N) a.y[m * a.ldy + n] = finish_out(v, a.bias, n);
      }
  }
}

struct QmvsShape {
  int ntt, su;
};
// 32-row blocks while that still leaves >= 256 blocks; 256-byte steps for long
// rows in 16-row blocks.
static QmvsShape qmvs_shape(const QmmArgs& a) {
  if (a.N >= 8192) return {2, 4};
  if (a.K % 512 == 0 && a.K >= 8192) return {1, 8};
  return {1, 4};
}

template <int MT, int NTT, int SU>
static hipError_t launch_qmvs_cfg(const QmmArgs& a, hipStream_t stream) {
  const unsigned blocks = (unsigned)((a.N + 16 * NTT - 1) / (16 * NTT));
  qmvs_kernel<MT, NTT, SU><<<blocks, kQmvsKS * 64, 0, stream>>>(a);
  return hipGetLastError();
}

template <int MT>
static hipError_t launch_qmvs_mt(const QmmArgs& a, hipStream_t stream) {
  const QmvsShape sh = qmvs_shape(a);
  if (sh.ntt == 2) return launch_qmvs_cfg<MT, 2, 4>(a, stream);
  if (sh.su == 8) return launch_qmvs_cfg<MT, 1, 8>(a, stream);
  return launch_qmvs_cfg<MT, 1, 4>(a, stream);
}

}  // namespace

bool qmvs_supported(const QmmArgs& a) {
  auto al = [](const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; };
  // 8-byte scale loads: K a multiple of 256 keeps every scale row 8-byte aligned.
  // Weights go through a buffer resource: their byte size must stay below 2^31.
  return a.bits == 4 && a.group_size == 64 && a.M >= 1 && a.M <= 32 && a.K % 256 == 0 &&
         a.N * (a.K / 2) < (int64_t(1) << 31) &&
         a.ldx % 8 == 0 && al(a.x, 16) && al(a.w, 16) && al(a.scales, 8) && al(a.biases, 8);
}

hipError_t launch_qmvs(const QmmArgs& a, hipStream_t stream) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (!qmvs_supported(a)) return hipErrorInvalidValue;
  return a.M <= 16 ? launch_qmvs_mt<1>(a, stream) : launch_qmvs_mt<2>(a, stream);
}

// ---------------------------------------------------------------------------
// qmvw_kernel.  Block: WV waves side by side over WV * 16 NTT rows of W and one
// K part (steps [s0, s1) of 256 values); the block's x rows (16 MT of them) go to
// LDS once per step for all its waves (qmvs_walk_xlds), so x costs the texture
// units a 1 / WV share of what it costs qmvs, where every wave loads its own.
// Grid: (row blocks, K parts).  One part stores bf16 outputs; several write fp32
// partials [part][M][N] to a.ws and qmvw_fixup_kernel sums them in part order.

namespace {

// The pipelined walk dequantizes the weights (qmvs_walk_xlds DEQ) from this many
// 16-row x tiles: at M = 64, 30.3 -> 24.2 us on 14336x4096 and 29.3 -> 23.6 us on
// 4096x14336; at M = 32 on 4096x14336 19.5 -> 17.9 us.
#ifndef FMXQ_QMVW_DEQ_MIN_MT
#define FMXQ_QMVW_DEQ_MIN_MT 2
#endif
constexpr int kQmvwDeqMinMT = FMXQ_QMVW_DEQ_MIN_MT;
// The up-front walk likewise from 2 tiles (C1 stack at M = 24 / 32: 3.03 -> 2.99 ms,
// 3.09 -> 3.01 ms); at one tile the exponent-trick form is quicker (M = 16 on
// 14336x4096: 16.0 against 17.7 us dequantized).
#ifndef FMXQ_QMVW_XALL_DEQ_MIN_MT
#define FMXQ_QMVW_XALL_DEQ_MIN_MT 2
#endif
constexpr int kQmvwXallDeqMinMT = FMXQ_QMVW_XALL_DEQ_MIN_MT;

// int8 weights (BITS = 8) always take the dequantizing walks (there is no
// exponent-trick form for 8-bit values).
template <int MT, int NTT, int WV, int D, int BITS = 4>
__global__ __launch_bounds__(WV * 64) __attribute__((amdgpu_waves_per_eu(MT == 1 && NTT == 1 ? 3 : 2)))
void qmvw_kernel(QmmArgs a) {
  using G = QmvsGeom<NTT, 4, BITS>;
  constexpr bool kDeqXlds = BITS == 8 || MT >= kQmvwDeqMinMT;
  constexpr bool kDeqXall = BITS == 8 || MT >= kQmvwXallDeqMinMT;
  constexpr int AX = 8 * MT / WV;
  constexpr int XSLOTS = D > 0 ? D : 2;
  __shared__ __attribute__((aligned(1024))) uint8_t xs[XSLOTS][16 * MT * kXStageRow];
  __shared__ __attribute__((aligned(16))) uint8_t stage[WV][G::STAGE];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c16 = lane & 15, q = lane >> 4;
  const int64_t nb = (int64_t)blockIdx.x * (16 * NTT * WV) + wave * (16 * NTT);
  const int parts = a.splits > 1 ? a.splits : 1;
  const int part = (int)blockIdx.y;
  const int64_t nst = a.K / 256;
  const int64_t s0 = part * nst / parts, s1 = (part + 1) * nst / parts;

  // x through a buffer resource (qmvw_supported keeps its byte size below 2^31).
  // DMA instruction j of this wave fills stage rows 2 (AX wave + j) and the next
  // (qmvs_walk_xlds); a row past M reads row M - 1 and reaches no stored output.
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.x, (short)0, (int)(((a.M - 1) * a.ldx + a.K) * 2), 0x00020000);
  uint32_t xo[AX];
#pragma unroll
  for (int j = 0; j < AX; ++j) {
    const int r = 2 * (wave * AX + j) + (lane >> 5);
    const int c = (lane & 31) ^ (r & 15);
    const int64_t xr = r < a.M ? r : a.M - 1;
    xo[j] = (uint32_t)(xr * a.ldx * 2 + c * 16);
  }
  f32x4 acc[1][MT][NTT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NTT; ++t) acc[0][mt][t] = f32x4{};
  if constexpr (D > 0) {
    qmvs_walk_xall<MT, NTT, WV, D, kDeqXall, BITS>(&xs[0][0], stage[wave], xres, xo, wave,
                                                              a.w, a.scales, a.biases,
                                   nb, a.N, a.K, s0, s1, acc[0]);
  } else {
    const uint32_t* const w[1] = {a.w};
    const uint16_t* const sc[1] = {a.scales};
    const uint16_t* const bi[1] = {a.biases};
    qmvs_walk_xlds<MT, MT, NTT, 1, WV, false, kDeqXlds, BITS>(xs[0], xs[1], stage[wave], xres, xo,
                                                                     wave, a.M, w, sc, bi,
                                       nb, a.N, a.K, s0, s1, acc);
  }

  // C layout of a 16x16 tile: register r of lane l is row 4 (l / 16) + r, column
  // l % 16.
#pragma unroll
  for (int t = 0; t < NTT; ++t) {
    const int64_t n = nb + 16 * t + c16;
    if (n >= a.N) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = 16 * mt + 4 * q + r;
        if (m >= a.M) continue;
        if (parts == 1) a.y[m * a.ldy + n] = finish_out(acc[0][mt][t][r], a.bias, n);
        else a.ws[((int64_t)part * a.M + m) * a.N + n] = acc[0][mt][t][r];
      }
  }
}

// Grid (ceil(N / 1024), M): thread t of block x sums the parts of outputs
// 4 (256 x + t) .. +4 of row blockIdx.y (N % 4 == 0, so 16-byte pieces), or of
// output 256 x + t alone when N % 4 != 0 (grid x then ceil(N / 256)).  All parts
// are loaded before the first add (at most kQmvwMaxParts), so a thread waits for
// one round trip instead of one per part; the sum runs in part order.
constexpr int kQmvwMaxParts = 16;

__global__ __launch_bounds__(256) void qmvw_fixup_kernel(QmmArgs a) {
  const int64_t m = blockIdx.y;
  const int64_t mn = a.M * a.N;
  const float* src = a.ws + m * a.N;
  uint16_t* dst = a.y + m * a.ldy;
  const int parts = a.splits;
  if ((a.N & 3) == 0) {
    const int64_t n = 4 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
    if (n >= a.N) return;
    f32x4 v[kQmvwMaxParts];
#pragma unroll
    for (int p = 0; p < kQmvwMaxParts; ++p)
      if (p < parts) v[p] = *reinterpret_cast<const f32x4*>(src + p * mn + n);
    f32x4 t = v[0];
#pragma unroll
    for (int p = 1; p < kQmvwMaxParts; ++p)
      if (p < parts) t += v[p];
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[n + i] = finish_out(t[i], a.bias, n + i);
  } else {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (n >= a.N) return;
    float v[kQmvwMaxParts];
#pragma unroll
    for (int p = 0; p < kQmvwMaxParts; ++p)
      if (p < parts) v[p] = src[p * mn + n];
    float t = v[0];
#pragma unroll
    for (int p = 1; p < kQmvwMaxParts; ++p)
      if (p < parts) t += v[p];
    dst[n] = finish_out(t, a.bias, n);
  }
}

template <int MT, int NTT, int WV, int D>
hipError_t launch_qmvw_cfg(const QmmArgs& a, hipStream_t stream) {
  const int parts = a.splits > 1 ? a.splits : 1;
  const dim3 grid((unsigned)((a.N + 16 * NTT * WV - 1) / (16 * NTT * WV)), (unsigned)parts);
  if (a.bits == 8) {
    // int8: 16-row W tiles, pipelined walk only (qmvw_plan)
    if constexpr (NTT == 1 && D == 0) qmvw_kernel<MT, 1, WV, 0, 8><<<grid, WV * 64, 0, stream>>>(a);
    else return hipErrorInvalidValue;
  } else {
    qmvw_kernel<MT, NTT, WV, D><<<grid, WV * 64, 0, stream>>>(a);
  }
  if (parts > 1) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t per = (a.N & 3) == 0 ? 1024 : 256;
    qmvw_fixup_kernel<<<dim3((unsigned)((a.N + per - 1) / per), (unsigned)a.M), 256, 0, stream>>>(a);
  }
  return hipGetLastError();
}

template <int MT, int NTT, int WV>
hipError_t launch_qmvw_d(const QmmArgs& a, int d, hipStream_t stream) {
  if (d == 2) return launch_qmvw_cfg<MT, NTT, WV, 2>(a, stream);
  if constexpr (MT <= 2) {
    if (d == 4) return launch_qmvw_cfg<MT, NTT, WV, 4>(a, stream);
  }
  return launch_qmvw_cfg<MT, NTT, WV, 0>(a, stream);
}

template <int MT>
hipError_t launch_qmvw_mt(const QmmArgs& a, int ntt, int d, hipStream_t stream) {
  if constexpr (MT <= 2) {
    if (ntt == 2) return launch_qmvw_d<MT, 2, 4>(a, d, stream);
  }
  return launch_qmvw_d<MT, 1, 4>(a, d, stream);
}

}  // namespace

bool qmvw_supported(const QmmArgs& a) {
  auto al = [](const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; };
  // K a multiple of 256 (whole steps; 8-byte scale loads stay aligned).  Weights
  // and x go through buffer resources: their byte sizes must stay below 2^31.
  return (a.bits == 4 || a.bits == 8) && a.group_size == 64 && a.M >= 1 && a.M <= kQmvwMaxM &&
         a.K % 256 == 0 && a.N * (a.K * a.bits / 8) < (int64_t(1) << 31) &&
         ((a.M - 1) * a.ldx + a.K) * 2 < (int64_t(1) << 31) && a.ldx % 8 == 0 &&
         al(a.x, 16) && al(a.w, 16) && al(a.scales, 8) && al(a.biases, 8);
}

// Shapes measured on MI355X (4-bit group 64, M = 16 / 32 / 64; the Llama-3-8B
// projections): long rows (K >= 8192) split K into 8 pipelined parts; wide
// outputs (N >= 8192) take 32-row W tiles and 4 up-front parts for x tiles of up
// to 32 rows, 2 pipelined parts for 64; N >= 4096 takes 4 parts; narrower outputs
// 8 up-front parts of two steps.  No more parts than give about two blocks per CU
// (a 128256-row head needs none), and the up-front walk only where its parts
// hold at most d steps.
QmvwPlan qmvw_plan(const QmmArgs& a, int cus) {
  QmvwPlan p;
  p.mt = a.M <= 16 ? 1 : a.M <= 32 ? 2 : 4;
  p.ntt = 1;
  p.wv = 4;
  const int64_t nst = a.K / 256;
  int64_t parts;
  if (a.K >= 8192) {
    parts = 8;
    p.d = 0;
  } else if (a.N >= 8192) {
    if (p.mt <= 2) {
      p.ntt = 2;
      parts = 4;
      p.d = 4;
    } else {
      parts = 2;
      p.d = 0;
    }
  } else if (a.N >= 4096) {
    parts = 4;
    p.d = p.mt <= 2 ? 4 : 0;
  } else {
    parts = 8;
    p.d = 2;
  }
  if (a.bits == 8) {
    // int8: 16-row W tiles and the pipelined walk (the up-front one would hold
    // twice the weight registers).
    p.ntt = 1;
    p.d = 0;
  }
  // 64-row x tiles on the pipelined walk: 8-wave blocks of 128 weight rows, so
  // each x step DMA'd into LDS serves twice the weights (33-64 rows, against 4
  // waves: 14336x4096 M = 33 / 48 / 64 22.3 / 23.3 / 24.0 -> 20.6 / 22.3 / 24.4
  // us, 4096x14336 21.5 / 22.2 / 23.5 -> 19.9 / 21.8 / 23.0 us; int8 M = 64
  // 26.5 / 26.2 -> 25.8 / 25.4 us).  16- and 32-row tiles stay at 4 waves (int8
  // at M = 17-24 on 14336x4096 lost 12% with 8).
  if (p.mt == 4 && p.ntt == 1 && p.d == 0) p.wv = 8;
  const int64_t rows = 16 * p.ntt * p.wv;
  const int64_t rblocks = (a.N + rows - 1) / rows;
  const int64_t enough = (2 * (int64_t)cus + rblocks - 1) / rblocks;
  parts = std::min(parts, std::max<int64_t>(enough, 1));
  parts = std::max<int64_t>(1, std::min({parts, nst, (int64_t)kQmvwMaxParts}));
  if (p.d > 0 && parts * p.d < nst) p.d = 0;
  p.parts = (int)parts;
  p.ws_floats = parts > 1 ? parts * a.M * a.N : 0;
  return p;
}

hipError_t launch_qmvw(const QmmArgs& a, const QmvwPlan& p, hipStream_t stream) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (!qmvw_supported(a) || p.parts > kQmvwMaxParts ||
      (p.parts > 1 && (!a.ws || a.splits != p.parts)))
    return hipErrorInvalidValue;
  // The upfront walk holds at most d steps: every part must fit.
  if ((p.wv != 4 && !(p.wv == 8 && p.mt == 4 && p.d == 0)) || (p.mt == 4 && p.ntt != 1) ||
      (p.d > 0 && ((a.K / 256 + p.parts - 1) / p.parts > p.d || (p.mt == 4 && p.d > 2))) ||
      (a.bits == 8 && (p.ntt != 1 || p.d != 0)))
    return hipErrorInvalidValue;
  if (p.mt == 1) return launch_qmvw_mt<1>(a, p.ntt, p.d, stream);
  if (p.mt == 2) return launch_qmvw_mt<2>(a, p.ntt, p.d, stream);
  // 64-row x tiles use 16-row W tiles only (32-row ones would spill), and at most
  // two up-front steps (LDS); the pipelined walk runs 8-wave blocks.
  if (p.wv == 8) return launch_qmvw_cfg<4, 1, 8, 0>(a, stream);
  return launch_qmvw_mt<4>(a, 1, p.d, stream);
}

}  // namespace fmxq
