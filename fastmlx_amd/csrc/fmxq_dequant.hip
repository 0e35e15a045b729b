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
// bf16-op chain.  The roundings are v_cvt_pk_bf16_f32 (nearest-even); a NaN
// result is a quiet NaN, as in the oracle, though its payload bits may differ.
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"

namespace fmxq {

// Output row r reads table row idx[r] when idx is given (the take-then-dequantize
// of quantized embedding lookups, compute/models/quant.go:117-142), else row r.
// A row index >= table_rows yields a zero row and raises *err_flag.
//
// A thread owns one quad: 4 consecutive packed words, 32 (4-bit) or 16 (8-bit)
// outputs written as 16-byte stores.  K % GS == 0 makes the flattened [rows * K]
// array a sequence of whole groups, and GS >= 32 >= the values of a quad, so a
// quad sits inside one group whose flattened index is its first value / GS: no
// row arithmetic except for the table lookup.
template <int BITS, int GS, bool IDX>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint16_t* __restrict__ biases,
                                                      const uint32_t* __restrict__ idx,
                                                      int64_t table_rows, uint32_t* err_flag,
                                                      uint16_t* __restrict__ out, int64_t quads,
                                                      int64_t qpr) {
  constexpr int PER = 32 / BITS;
  constexpr int VPQ = 4 * PER;  // values per quad
  static_assert(GS % VPQ == 0, "a quad lies inside one group");
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < quads;
       t += (int64_t)gridDim.x * blockDim.x) {
    u32x4* dst = reinterpret_cast<u32x4*>(out + t * VPQ);
    int64_t src = t;
    if constexpr (IDX) {
      const int64_t r = t / qpr;
      const int64_t row = idx[r];
      if (row >= table_rows) {
#pragma unroll
        for (int v = 0; v < PER / 2; ++v) dst[v] = u32x4{0u, 0u, 0u, 0u};
        atomicOr(err_flag, 1u);
        continue;
      }
      src = row * qpr + (t - r * qpr);
    }
    const u32x4 words = reinterpret_cast<const u32x4*>(w)[src];
    const int64_t g = src * VPQ / GS;
    const float s = bf16_bits_to_f32(scales[g]);
    const float b = bf16_bits_to_f32(biases[g]);
    uint32_t outw[2 * PER];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t word = words[j];
#pragma unroll
      for (int p = 0; p < PER; p += 2) {
        const float q0 = (float)((word >> (p * BITS)) & MASK);
        const float q1 = (float)((word >> ((p + 1) * BITS)) & MASK);
        // v_cvt_pk_bf16_f32 rounds to nearest-even like the oracle's software
        // rounding (checked over subnormal, overflowing and NaN-producing scales)
        const uint32_t m = pack_bf16x2(q0 * s, q1 * s);
        outw[(j * PER + p) / 2] = pack_bf16x2(bf16_lo(m) + b, bf16_hi(m) + b);
      }
    }
    // 4 words hold 4*PER values = 2*PER bf16 pairs = PER/2 16-byte stores.
#pragma unroll
    for (int v = 0; v < PER / 2; ++v)
      dst[v] = u32x4{outw[v * 4 + 0], outw[v * 4 + 1], outw[v * 4 + 2], outw[v * 4 + 3]};
  }
}

template <int BITS, bool IDX>
hipError_t launch_deq_gs(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                         uint16_t* out, int64_t quads, int64_t qpr, int group_size,
                         const uint32_t* idx, int64_t table_rows, uint32_t* err_flag,
                         unsigned blocks, hipStream_t stream) {
  switch (group_size) {
    case 32:
      dequant_kernel<BITS, 32, IDX><<<blocks, 256, 0, stream>>>(w, scales, biases, idx,
                                                                table_rows, err_flag, out, quads,
                                                                qpr);
      break;
    case 64:
      dequant_kernel<BITS, 64, IDX><<<blocks, 256, 0, stream>>>(w, scales, biases, idx,
                                                                table_rows, err_flag, out, quads,
                                                                qpr);
      break;
    case 128:
      dequant_kernel<BITS, 128, IDX><<<blocks, 256, 0, stream>>>(w, scales, biases, idx,
                                                                 table_rows, err_flag, out,
                                                                 quads, qpr);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_dequantize(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                             uint16_t* out, int64_t rows, int64_t K, int group_size, int bits,
                             hipStream_t stream, const uint32_t* idx, int64_t table_rows,
                             uint32_t* err_flag) {
  // K % 32 == 0 is guaranteed by the caller, so a row holds whole quads.
  const int64_t qpr = K / (4 * (32 / bits));
  const int64_t quads = rows * qpr;
  if (quads == 0) return hipSuccess;
  int64_t blocks = (quads + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  const unsigned g = (unsigned)blocks;
  if (bits == 4)
    return idx ? launch_deq_gs<4, true>(w, scales, biases, out, quads, qpr, group_size, idx,
                                        table_rows, err_flag, g, stream)
               : launch_deq_gs<4, false>(w, scales, biases, out, quads, qpr, group_size, idx,
                                         table_rows, err_flag, g, stream);
  if (bits == 8)
    return idx ? launch_deq_gs<8, true>(w, scales, biases, out, quads, qpr, group_size, idx,
                                        table_rows, err_flag, g, stream)
               : launch_deq_gs<8, false>(w, scales, biases, out, quads, qpr, group_size, idx,
                                         table_rows, err_flag, g, stream);
  return hipErrorInvalidValue;
}

}  // namespace fmxq
