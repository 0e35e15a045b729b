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
// (HIP's default correctly rounded fp32 divide) and rint rounds half to even,
// so every step matches the CPU restatement bit for bit.
//
// Layout: one lane per 8 consecutive values (a 16-byte load); the G / 8 lanes of
// a group are adjacent lanes of one wave and meet with xor shuffles.  A lane
// packs its 8 values into one word (4-bit) or two (8-bit), so the stores of a
// wave are contiguous; the group's first lane writes the scale and bias.  The
// kernel reads 2 bytes and writes bits / 8 + 4 / G bytes per value (HBM-bound).
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"

namespace fmxq {
namespace {

template <int BITS, int L>  // L = group_size / 8 lanes per group
__global__ __launch_bounds__(256) void quantize_kernel(const uint16_t* __restrict__ w,
                                                       uint32_t* __restrict__ wq,
                                                       uint16_t* __restrict__ scales,
                                                       uint16_t* __restrict__ biases,
                                                       int64_t units) {
#pragma clang fp contract(off)
  constexpr float n_bins = (float)((1 << BITS) - 1);
  // units is a multiple of L and the stride a multiple of 64, so the lanes of a
  // group enter and leave the loop together and every shuffle partner is live.
  for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < units;
       u += (int64_t)gridDim.x * 256) {
    const u32x4 raw = *reinterpret_cast<const u32x4*>(w + u * 8);
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[2 * j] = bf16_lo(raw[j]);
      v[2 * j + 1] = bf16_hi(raw[j]);
    }
    float mn = v[0], mx = v[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) {
      mn = fminf(mn, v[j]);
      mx = fmaxf(mx, v[j]);
    }
#pragma unroll
    for (int off = L / 2; off >= 1; off >>= 1) {
      mn = fminf(mn, __shfl_xor(mn, off, L));
      mx = fmaxf(mx, __shfl_xor(mx, off, L));
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
    uint32_t word[BITS / 4] = {};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float q = __builtin_rintf((v[j] - bias) / scale);
      q = q < 0.f ? 0.f : q > n_bins ? n_bins : q;
      constexpr int per = 32 / BITS;
      word[j / per] |= (uint32_t)q << ((j % per) * BITS);
    }
    if constexpr (BITS == 4) {
      wq[u] = word[0];
    } else {
      *reinterpret_cast<u32x2*>(wq + 2 * u) = u32x2{word[0], word[1]};
    }
    if ((u & (L - 1)) == 0) {
      scales[u / L] = (uint16_t)f32_to_bf16_rne(scale);
      biases[u / L] = (uint16_t)f32_to_bf16_rne(bias);
    }
  }
}

template <int BITS>
hipError_t launch_bits(const uint16_t* w, uint32_t* wq, uint16_t* scales, uint16_t* biases,
                       int64_t units, int group_size, unsigned blocks, hipStream_t stream) {
  switch (group_size) {
    case 32:
      quantize_kernel<BITS, 4><<<blocks, 256, 0, stream>>>(w, wq, scales, biases, units);
      break;
    case 64:
      quantize_kernel<BITS, 8><<<blocks, 256, 0, stream>>>(w, wq, scales, biases, units);
      break;
    case 128:
      quantize_kernel<BITS, 16><<<blocks, 256, 0, stream>>>(w, wq, scales, biases, units);
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
  // flattened [rows * K] array is a sequence of groups and units never straddle.
  const int64_t units = rows * (K / 8);
  if (units == 0) return hipSuccess;
  int64_t blocks = (units + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (bits == 4)
    return launch_bits<4>(w, wq, scales, biases, units, group_size, (unsigned)blocks, stream);
  if (bits == 8)
    return launch_bits<8>(w, wq, scales, biases, units, group_size, (unsigned)blocks, stream);
  return hipErrorInvalidValue;
}

}  // namespace fmxq
