// fmxq_skinny.hip -- MFMA GEMV for 5 <= M <= 32 (speculative verify, small
// decode batches): quantized_matmul rows that are too many for the dot2 GEMV
// and too few to amortise an LDS-dequantised GEMM tile.
//
// Replaces mlx_quantized_matmul (mlxgo/binding_cgo.go:636-643) for
// x [M, K] with M = batch * (k+1) draft positions (the verify step of
// pipeline/pipeline.go:56-65) or small decode batches (llama.go:403).
//
// v_mfma_f32_32x32x16_bf16 with the weights as the B operand straight from
// registers, no LDS:
//   - lane l holds output column n = l % 32 and, for each 16-byte load, 32 int4
//     (16 int8) values of row n; lane halves g = l / 32 cover the two halves of a
//     64-value (32-value for int8) unit, so every MFMA step sums over one
//     quantization group only (group_size >= 64 for int4, >= 32 for int8);
//   - B values are bf16(128 + q) from the exponent trick (0x4300 | q); int8
//     values are split into two nibbles, the high one as bf16(2048 + 16 q_hi)
//     (0x4500 | q_hi), so each int8 element occupies two MFMA k slots;
//   - A = x in the matching pair order, loaded per unit from global memory
//     (rows >= M read a valid row; their outputs are discarded);
//   - per group: P = sum_k x (offset + q), xs = sum_k x (an MFMA against ones),
//     acc += s * P + (b - offset * s) * xs.
// The K axis is split over the KS waves of a block, which meet in LDS.
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"
#include "fmxq_mfma_frag.hpp"

namespace fmxq {

template <int NT>
struct SkStage {
  u32x4 w[NT];
  uint32_t sb[NT];
  u32x4 x[4];  // int4: four 16-byte x pieces; int8: two (x[0], x[1]) used
};

// NT: 32-row tiles per wave.  RL: accumulator registers carrying rows < M
// (4 per 8 rows).  KS: waves of a block splitting K.
template <int BITS, int NT, int RL, int KS>
__global__ __launch_bounds__(256) void qmv_mfma_kernel(QmmArgs a) {
  constexpr int RG = 4 / KS;
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

template <int BITS, int NT, int RL, int KS>
static hipError_t launch_sk(const QmmArgs& a, hipStream_t stream) {
  constexpr int rows_per_block = (4 / KS) * 32 * NT;
  const unsigned blocks = (unsigned)((a.N + rows_per_block - 1) / rows_per_block);
  qmv_mfma_kernel<BITS, NT, RL, KS><<<blocks, 256, 0, stream>>>(a);
  return hipGetLastError();
}

template <int BITS, int RL>
static hipError_t launch_sk_rl(const QmmArgs& a, hipStream_t stream) {
  // Split K over the 4 waves of a block unless there are rows enough to give each
  // wave its own 32-row tile across at least ~1024 waves.
  if (a.N >= 32 * 4 * 1024 / 4) return launch_sk<BITS, 1, RL, 1>(a, stream);
  return launch_sk<BITS, 1, RL, 4>(a, stream);
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

}  // namespace fmxq
