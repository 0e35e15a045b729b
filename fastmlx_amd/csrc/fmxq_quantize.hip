// fmxq_quantize.hip -- MLX affine quantization (mlx_quantize), the requantize
// step of DeepSeek-V3's kv_b_proj absorption (compute/models/deepseekv3.go:662-669
// through mlxgo.Quantize, mlxgo/binding_cgo.go:684-697): bf16 w [rows, K] to the
// packed uint32 words, bf16 scales and bf16 biases that the quantized kernels
// consume.
//
// Per group of G values along K, in fp32 (MLX's affine algorithm):
//   delta = max((max - min) / (2^bits - 1), 1e-7)
//   the end of larger magnitude is the edge: min with scale +delta, else max
//   with scale -delta, so q = 0 sits on the edge and q grows inward;
//   q0 = rint(edge / scale); if q0 != 0: scale = edge / q0 and bias = edge (the
//   edge is reproduced exactly and zero falls on grid point -q0), else bias = 0;
//   q = clamp(rint((w - bias) / scale), 0, 2^bits - 1).
// scale and bias are stored rounded to nearest-even bf16.  Divisions are IEEE
// (HIP's default correctly rounded fp32 divide; the per-value quotient is taken
// from a reciprocal product unless it lies near a rounding boundary) and rint
// rounds half to even, so every step matches the CPU restatement bit for bit.
//
// Layout: a lane owns 32 consecutive values; the G / 32 lanes of a group are
// adjacent lanes of one wave and meet with xor shuffles.  A lane packs its values
// into 4 (4-bit) or 8 (8-bit) words written as 16-byte stores, so the stores of a
// wave are contiguous; the group's first lane writes the scale and bias.  The
// kernel reads 2 bytes and writes bits / 8 + 4 / G bytes per value (HBM-bound).
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"

namespace fmxq {
namespace {

// A lane owns 32 consecutive values (64 bytes, four 16-byte loads): G / 32 lanes
// per group, adjacent in the wave, meet with xor shuffles, so the per-group work
// (reductions, the two IEEE divisions of the scale) is shared by few lanes.
template <int BITS, int G>
__global__ __launch_bounds__(256) void quantize_kernel(const uint16_t* __restrict__ w,
                                                       uint32_t* __restrict__ wq,
                                                       uint16_t* __restrict__ scales,
                                                       uint16_t* __restrict__ biases,
                                                       int64_t lanes) {
#pragma clang fp contract(off)
  constexpr int LPG = G / 32;
  constexpr int WPL = BITS;  // packed words per lane: 32 values * BITS / 32
  constexpr float n_bins = (float)((1 << BITS) - 1);
  // lanes is a multiple of LPG and the stride a multiple of 64, so the lanes of a
  // group enter and leave the loop together and every shuffle partner is live.
  for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < lanes;
       u += (int64_t)gridDim.x * 256) {
    const u32x4* src = reinterpret_cast<const u32x4*>(w + u * 32);
    u32x4 raw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) raw[i] = src[i];
    float v[32];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[8 * i + 2 * j] = bf16_lo(raw[i][j]);
        v[8 * i + 2 * j + 1] = bf16_hi(raw[i][j]);
      }
    float mn = v[0], mx = v[0];
#pragma unroll
    for (int j = 1; j < 32; ++j) {
      mn = fminf(mn, v[j]);
      mx = fmaxf(mx, v[j]);
    }
#pragma unroll
    for (int off = LPG / 2; off >= 1; off >>= 1) {
      mn = fminf(mn, __shfl_xor(mn, off, LPG));
      mx = fmaxf(mx, __shfl_xor(mx, off, LPG));
    }
    float delta = (mx - mn) / n_bins;
    if (!(delta > 1e-7f)) delta = 1e-7f;
    const bool side = fabsf(mn) > fabsf(mx);
    float scale = side ? delta : -delta;
    const float edge = side ? mn : mx;
    const float q0 = __builtin_rintf(edge / scale);
    float bias = 0.f;
    if (q0 != 0.f) {
      scale = edge / q0;
      bias = edge;
    }
    // q = rint(a / scale) with the IEEE quotient.  a * rcp(scale) is within 3 ulp
    // of the quotient (below 2^-13 for |quotient| < 2^9), so the two round to the
    // same integer unless a half-integer lies between them; only a product within
    // 2^-12 of a half-integer takes the exact division (a wave-uniform branch).
    const float rs = __builtin_amdgcn_rcpf(scale);
    float q[32];
    bool near = false;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const float t = (v[j] - bias) * rs;
      q[j] = __builtin_rintf(t);
      near |= __builtin_fabsf(t - q[j]) > 0.5f - 0x1p-12f;
    }
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(near) != 0, 0)) {
#pragma unroll
      for (int j = 0; j < 32; ++j) q[j] = __builtin_rintf((v[j] - bias) / scale);
    }
    // Clamp, then pack with v_cvt_pk_u8_f32 (float -> byte lane of the word); two
    // 4-bit values first meet in one exact float, q_even + 16 q_odd.
    uint32_t word[WPL];
#pragma unroll
    for (int i = 0; i < WPL; ++i) {
      uint32_t acc = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        float byte;
        if constexpr (BITS == 8) {
          byte = __builtin_amdgcn_fmed3f(q[4 * i + k], 0.f, n_bins);
        } else {
          const float lo = __builtin_amdgcn_fmed3f(q[8 * i + 2 * k], 0.f, n_bins);
          const float hi = __builtin_amdgcn_fmed3f(q[8 * i + 2 * k + 1], 0.f, n_bins);
          byte = __builtin_fmaf(hi, 16.f, lo);
        }
        acc = __builtin_amdgcn_cvt_pk_u8_f32(byte, k, acc);
      }
      word[i] = acc;
    }
    u32x4* dst = reinterpret_cast<u32x4*>(wq + u * WPL);
#pragma unroll
    for (int i = 0; i < WPL / 4; ++i)
      dst[i] = u32x4{word[4 * i], word[4 * i + 1], word[4 * i + 2], word[4 * i + 3]};
    if ((u & (LPG - 1)) == 0) {
      scales[u / LPG] = (uint16_t)f32_to_bf16_rne(scale);
      biases[u / LPG] = (uint16_t)f32_to_bf16_rne(bias);
    }
  }
}

template <int BITS>
hipError_t launch_bits(const uint16_t* w, uint32_t* wq, uint16_t* scales, uint16_t* biases,
                       int64_t lanes, int group_size, unsigned blocks, hipStream_t stream) {
  switch (group_size) {
    case 32:
      quantize_kernel<BITS, 32><<<blocks, 256, 0, stream>>>(w, wq, scales, biases, lanes);
      break;
    case 64:
      quantize_kernel<BITS, 64><<<blocks, 256, 0, stream>>>(w, wq, scales, biases, lanes);
      break;
    case 128:
      quantize_kernel<BITS, 128><<<blocks, 256, 0, stream>>>(w, wq, scales, biases, lanes);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_quantize(const uint16_t* w, uint32_t* wq, uint16_t* scales, uint16_t* biases,
                           int64_t rows, int64_t K, int group_size, int bits,
                           hipStream_t stream) {
  // K % group_size == 0 (checked by the caller) makes every group whole, so the
  // flattened [rows * K] array is a sequence of groups of whole 32-value lanes.
  const int64_t lanes = rows * (K / 32);
  if (lanes == 0) return hipSuccess;
  int64_t blocks = (lanes + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (bits == 4)
    return launch_bits<4>(w, wq, scales, biases, lanes, group_size, (unsigned)blocks, stream);
  if (bits == 8)
    return launch_bits<8>(w, wq, scales, biases, lanes, group_size, (unsigned)blocks, stream);
  return hipErrorInvalidValue;
}

}  // namespace fmxq
