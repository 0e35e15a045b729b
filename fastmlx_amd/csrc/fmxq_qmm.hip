// fmxq_qmm.hip -- MFMA GEMM for quantized_matmul at M > 4 (verify and prefill).
//
// Replaces the GEMM side of mlx_quantized_matmul (mlxgo/binding_cgo.go:636-643)
// for x [M, K] with M = batch * seq rows (compute/models/llama.go:403 on
// [batch, L, D], prefill at batch_generator.go:258).
//
// Block tile BM x BN over a 64-deep K step; 4 waves in a WM x WN grid, each
// owning a (BM/WM) x (BN/WN) patch of v_mfma_f32_16x16x32_bf16 tiles.  Per K
// step the block
//   - copies the x tile (bf16) into LDS,
//   - reads the packed weight tile once, dequantizes it in registers
//     (w = bf16(fma(s, q, b)), one rounding) and stores the bf16 tile in LDS,
// then every wave feeds its MFMAs from LDS.  LDS rows carry 8 bf16 of padding so
// the 16-byte fragment reads of 16 consecutive rows hit distinct banks.  The
// next step's global loads are issued before the current step's MFMAs (register
// double buffering) and LDS is double buffered, one barrier per step.
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"
#include "fmxq_qmv_impl.hpp"

namespace fmxq {

constexpr int kBK = 64;
constexpr int kLdsStride = kBK + 8;  // bf16 elements per LDS row

template <int BITS, int BM, int BN, int WM, int WN>
struct QmmTile {
  static constexpr int CH = 128 / BITS;              // weight values per 16-byte quad
  static constexpr int QPR = kBK / CH;               // quads per weight row per K step
  static constexpr int BTOTAL = BN * QPR;            // weight quads per K step
  static constexpr int ATOTAL = BM * (kBK / 8);      // x 16-byte chunks per K step
  static constexpr int BQUADS = (BTOTAL + 255) / 256;  // per thread
  static constexpr int AQUADS = (ATOTAL + 255) / 256;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 16, TN = WTN / 16;
  static_assert(BTOTAL % 256 == 0 || BTOTAL < 256, "weight tile split");
  static_assert(ATOTAL % 256 == 0 || ATOTAL < 256, "x tile split");
  static_assert(WM * WN == 4, "4 waves");
  static_assert(TM >= 1 && TN >= 1, "wave tile at least 16x16");
};

// Dequantize one 16-byte weight quad into bf16 pairs (CH/2 pairs).
template <int BITS>
__device__ __forceinline__ void dequant_quad(const u32x4 wv, float s, float b, uint32_t* out) {
  if constexpr (BITS == 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = wv[j];
      const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
      // element order within the word: 0..7 = lo.b0, hi.b0, lo.b1, hi.b1, ...
      const float q0 = (float)(lo & 0xffu), q1 = (float)(hi & 0xffu);
      const float q2 = (float)((lo >> 8) & 0xffu), q3 = (float)((hi >> 8) & 0xffu);
      const float q4 = (float)((lo >> 16) & 0xffu), q5 = (float)((hi >> 16) & 0xffu);
      const float q6 = (float)(lo >> 24), q7 = (float)(hi >> 24);
      out[4 * j + 0] = pack_bf16x2(__builtin_fmaf(s, q0, b), __builtin_fmaf(s, q1, b));
      out[4 * j + 1] = pack_bf16x2(__builtin_fmaf(s, q2, b), __builtin_fmaf(s, q3, b));
      out[4 * j + 2] = pack_bf16x2(__builtin_fmaf(s, q4, b), __builtin_fmaf(s, q5, b));
      out[4 * j + 3] = pack_bf16x2(__builtin_fmaf(s, q6, b), __builtin_fmaf(s, q7, b));
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = wv[j];
      const float q0 = (float)(w & 0xffu), q1 = (float)((w >> 8) & 0xffu);
      const float q2 = (float)((w >> 16) & 0xffu), q3 = (float)(w >> 24);
      out[2 * j + 0] = pack_bf16x2(__builtin_fmaf(s, q0, b), __builtin_fmaf(s, q1, b));
      out[2 * j + 1] = pack_bf16x2(__builtin_fmaf(s, q2, b), __builtin_fmaf(s, q3, b));
    }
  }
}

template <int BITS, int BM, int BN, int WM, int WN>
__global__ __launch_bounds__(256) void qmm_kernel(QmmArgs a) {
  using T = QmmTile<BITS, BM, BN, WM, WN>;
  constexpr int CH = T::CH;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][kLdsStride];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN][kLdsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t m0 = (int64_t)blockIdx.y * BM;
  const int64_t n0 = (int64_t)blockIdx.x * BN;
  const int64_t wpr = a.K * BITS / 32;
  const int gshift = __builtin_ctz((unsigned)a.group_size);  // a power of two
  const int64_t gpr = a.K >> gshift;
  const int64_t nk = (a.K + kBK - 1) / kBK;

  // Register staging for one K step.
  constexpr int AQ = T::AQUADS;
  u32x4 areg[AQ];
  u32x4 breg[T::BQUADS];
  float sreg[T::BQUADS], breg_b[T::BQUADS];

  auto load_step = [&](int64_t kt) {
    const int64_t k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < AQ; ++i) {
      const int idx = tid + i * 256;
      const int row = idx / (kBK / 8), c = idx % (kBK / 8);
      const int64_t m = m0 + row, k = k0 + c * 8;
      if (idx < T::ATOTAL && m < a.M && k < a.K)
        areg[i] = *reinterpret_cast<const u32x4*>(a.x + m * a.ldx + k);
      else
        areg[i] = u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < T::BQUADS; ++i) {
      const int idx = tid + i * 256;
      const int row = idx / T::QPR, qd = idx % T::QPR;
      const int64_t n = n0 + row, k = k0 + qd * CH;
      if (idx < T::BTOTAL && n < a.N && k < a.K) {
        breg[i] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(a.w + n * wpr + k * BITS / 32));
        const int64_t g = k >> gshift;
        sreg[i] = bf16_bits_to_f32(a.scales[n * gpr + g]);
        breg_b[i] = bf16_bits_to_f32(a.biases[n * gpr + g]);
      } else {
        breg[i] = u32x4{0u, 0u, 0u, 0u};
        sreg[i] = 0.f;
        breg_b[i] = 0.f;
      }
    }
  };

  auto store_step = [&](int buf) {
#pragma unroll
    for (int i = 0; i < AQ; ++i) {
      const int idx = tid + i * 256;
      const int row = idx / (kBK / 8), c = idx % (kBK / 8);
      if (idx < T::ATOTAL) *reinterpret_cast<u32x4*>(&As[buf][row][c * 8]) = areg[i];
    }
#pragma unroll
    for (int i = 0; i < T::BQUADS; ++i) {
      const int idx = tid + i * 256;
      const int row = idx / T::QPR, qd = idx % T::QPR;
      if (idx >= T::BTOTAL) continue;
      uint32_t d[CH / 2];
      dequant_quad<BITS>(breg[i], sreg[i], breg_b[i], d);
#pragma unroll
      for (int v = 0; v < CH / 8; ++v) {
        u32x4 o = {d[4 * v], d[4 * v + 1], d[4 * v + 2], d[4 * v + 3]};
        *reinterpret_cast<u32x4*>(&Bs[buf][row][qd * CH + v * 8]) = o;
      }
    }
  };

  f32x4 acc[T::TM][T::TN];
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // This block's share of the K steps (the whole axis unless split-K).
  const int64_t kt0 = (int64_t)blockIdx.z * nk / a.splits;
  const int64_t kt1 = (int64_t)(blockIdx.z + 1) * nk / a.splits;

  load_step(kt0);
  store_step(0);
  __syncthreads();

  int buf = 0;
  for (int64_t kt = kt0; kt < kt1; ++kt) {
    const bool more = kt + 1 < kt1;
    if (more) load_step(kt + 1);
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ++ks) {
      bf16x8 af[T::TM], bfr[T::TN];
      const int kc = ks * 32 + (lane >> 4) * 8;
#pragma unroll
      for (int i = 0; i < T::TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(&As[buf][wm * T::WTM + i * 16 + (lane & 15)][kc]);
#pragma unroll
      for (int j = 0; j < T::TN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(&Bs[buf][wn * T::WTN + j * 16 + (lane & 15)][kc]);
#pragma unroll
      for (int i = 0; i < T::TM; ++i)
#pragma unroll
        for (int j = 0; j < T::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_step(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

  // Epilogue: lane l, register r of tile (i, j) holds row 4*(l/16)+r, column l%16.
  if (a.splits == 1) {
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
      for (int j = 0; j < T::TN; ++j) {
        const int64_t n = n0 + wn * T::WTN + j * 16 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t m = m0 + wm * T::WTM + i * 16 + (lane >> 4) * 4 + r;
          if (m < a.M && n < a.N) a.y[m * a.ldy + n] = finish_out(acc[i][j][r], a.bias, n);
        }
      }
    return;
  }

  // Split-K: add the partial tile into the fp32 workspace, then the last split
  // to arrive at this tile converts it, writes y and zeroes the workspace tile
  // and the tile counter for the next call on this stream.
#pragma unroll
  for (int i = 0; i < T::TM; ++i)
#pragma unroll
    for (int j = 0; j < T::TN; ++j) {
      const int64_t n = n0 + wn * T::WTN + j * 16 + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * T::WTM + i * 16 + (lane >> 4) * 4 + r;
        if (m < a.M && n < a.N) atomicAdd(a.ws + m * a.N + n, acc[i][j][r]);
      }
    }
  __threadfence();
  __syncthreads();
  __shared__ uint32_t last;
  const int64_t tile = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
  if (tid == 0) last = atomicAdd(a.tile_count + tile, 1u) == (uint32_t)(a.splits - 1);
  __syncthreads();
  if (!last) return;
  __threadfence();
  for (int e = tid; e < BM * BN; e += 256) {
    const int64_t m = m0 + e / BN, n = n0 + e % BN;
    if (m < a.M && n < a.N) {
      float* p = a.ws + m * a.N + n;
      const float v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      a.y[m * a.ldy + n] = finish_out(v, a.bias, n);
      *p = 0.f;
    }
  }
  if (tid == 0) a.tile_count[tile] = 0u;
}

// Tile shape by M: skinny tiles for verify-sized M, 128x128 for prefill.
struct TileCfg {
  int bm, bn;
};
static TileCfg tile_for(int64_t M) {
  if (M <= 16) return {16, 64};
  if (M <= 32) return {32, 64};
  if (M <= 64) return {64, 128};
  return {128, 128};
}

// Split K until there are enough blocks to cover the chip a few times over,
// keeping at least 4 K steps per split.
QmmPlan qmm_plan(int64_t M, int64_t N, int64_t K) {
  const TileCfg t = tile_for(M);
  const int64_t tiles = ((N + t.bn - 1) / t.bn) * ((M + t.bm - 1) / t.bm);
  const int64_t nk = (K + kBK - 1) / kBK;
  int64_t s = (1024 + tiles - 1) / tiles;
  const int64_t smax = nk / 4;
  if (s > smax) s = smax;
  if (s > 32) s = 32;
  if (s < 2) return {1, 0, 0};
  return {(int)s, M * N, tiles};
}

template <int BITS, int BM, int BN, int WM, int WN>
static hipError_t launch_tile(const QmmArgs& a, hipStream_t stream) {
  dim3 grid((unsigned)((a.N + BN - 1) / BN), (unsigned)((a.M + BM - 1) / BM), (unsigned)a.splits);
  qmm_kernel<BITS, BM, BN, WM, WN><<<grid, 256, 0, stream>>>(a);
  return hipGetLastError();
}

template <int BITS>
static hipError_t launch_qmm_bits(const QmmArgs& a, hipStream_t stream) {
  if (a.M <= 16) return launch_tile<BITS, 16, 64, 1, 4>(a, stream);
  if (a.M <= 32) return launch_tile<BITS, 32, 64, 2, 2>(a, stream);
  if (a.M <= 64) return launch_tile<BITS, 64, 128, 2, 2>(a, stream);
  return launch_tile<BITS, 128, 128, 2, 2>(a, stream);
}

hipError_t launch_qmm(const QmmArgs& a, hipStream_t stream) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (a.splits > 1 && (!a.ws || !a.tile_count)) return hipErrorInvalidValue;
  return a.bits == 4 ? launch_qmm_bits<4>(a, stream) : launch_qmm_bits<8>(a, stream);
}

}  // namespace fmxq
