// fmxq_dequant.hip -- affine dequantize, bit-exact.
//
// Replaces mlx_dequantize (called at mlxgo/binding_cgo.go:675-682; callers
// compute/models/quant.go:139 qembed and deepseekv3.go:633 absorbKVB).
//
// Rounding definition (the one the build adopts and the oracle's DEQ_MLX mode
// restates): MLX composes dequantize on its CPU device as multiply(q, scales)
// followed by add(., biases), both bf16 ops, so the value is
//     w = bf16( bf16(q * s) + b )
// with both roundings to nearest-even.  q * s is exact in fp32 (q < 2^8, s has
// an 8-bit significand), and the fp32 sum of two bf16 values is exact unless
// their exponents differ by more than 16, so the fp32 steps below reproduce the
// bf16-op chain.  Software RNE keeps NaN payload handling identical to the oracle.
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"

namespace fmxq {

// Output row r reads table row idx[r] when idx is given (the take-then-dequantize
// of quantized embedding lookups, compute/models/quant.go:117-142), else row r.
// A row index >= table_rows yields a zero row and raises *err_flag.
template <int BITS>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint16_t* __restrict__ biases,
                                                      const uint32_t* __restrict__ idx,
                                                      int64_t table_rows, uint32_t* err_flag,
                                                      uint16_t* __restrict__ out, int64_t rows,
                                                      int64_t K, int group_size) {
  // Each thread owns 4 consecutive packed words of one row: 32 (4-bit) or 16
  // (8-bit) outputs, written as 16-byte stores.  K % 32 == 0 is guaranteed by
  // the host, so a row holds a whole number of 4-word quads.
  constexpr int PER = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int64_t wpr = K / PER;
  const int64_t quads_per_row = wpr / 4;
  const int64_t total = rows * quads_per_row;
  const int64_t gpr = K / group_size;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / quads_per_row;
    const int64_t qd = t - r * quads_per_row;
    const int64_t k0 = qd * 4 * PER;
    int64_t src = r;
    if (idx) {
      src = idx[r];
      if (src >= table_rows) {
        u32x4* dst = reinterpret_cast<u32x4*>(out + r * K + k0);
#pragma unroll
        for (int v = 0; v < PER / 2; ++v) dst[v] = u32x4{0u, 0u, 0u, 0u};
        atomicOr(err_flag, 1u);
        continue;
      }
    }
    const u32x4 words = *reinterpret_cast<const u32x4*>(w + src * wpr + qd * 4);
    uint32_t outw[4 * PER / 2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t g = (k0 + j * PER) / group_size;
      const float s = bf16_bits_to_f32(scales[src * gpr + g]);
      const float b = bf16_bits_to_f32(biases[src * gpr + g]);
      const uint32_t word = words[j];
#pragma unroll
      for (int p = 0; p < PER; p += 2) {
        const float q0 = (float)((word >> (p * BITS)) & MASK);
        const float q1 = (float)((word >> ((p + 1) * BITS)) & MASK);
        const float m0 = bf16_bits_to_f32(f32_to_bf16_rne(q0 * s));
        const float m1 = bf16_bits_to_f32(f32_to_bf16_rne(q1 * s));
        const uint32_t v0 = f32_to_bf16_rne(m0 + b);
        const uint32_t v1 = f32_to_bf16_rne(m1 + b);
        outw[(j * PER + p) / 2] = v0 | (v1 << 16);
      }
    }
    // 4 words hold 4*PER values = 2*PER bf16 pairs = PER/2 16-byte stores.
    u32x4* dst = reinterpret_cast<u32x4*>(out + r * K + k0);
#pragma unroll
    for (int v = 0; v < PER / 2; ++v) {
      u32x4 o;
      o[0] = outw[v * 4 + 0];
      o[1] = outw[v * 4 + 1];
      o[2] = outw[v * 4 + 2];
      o[3] = outw[v * 4 + 3];
      dst[v] = o;
    }
  }
}

hipError_t launch_dequantize(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                             uint16_t* out, int64_t rows, int64_t K, int group_size, int bits,
                             hipStream_t stream, const uint32_t* idx, int64_t table_rows,
                             uint32_t* err_flag) {
  const int64_t per = 32 / bits;
  const int64_t total = rows * (K / per / 4);
  if (total == 0) return hipSuccess;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (bits == 4)
    dequant_kernel<4><<<(unsigned)blocks, 256, 0, stream>>>(w, scales, biases, idx, table_rows,
                                                            err_flag, out, rows, K, group_size);
  else
    dequant_kernel<8><<<(unsigned)blocks, 256, 0, stream>>>(w, scales, biases, idx, table_rows,
                                                            err_flag, out, rows, K, group_size);
  return hipGetLastError();
}

}  // namespace fmxq
