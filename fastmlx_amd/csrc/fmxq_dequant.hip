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
// The flattened output is a sequence of 8-value units (one packed word of int4,
// two of int8), each one 16-byte store; K % GS == 0 and GS >= 32 put every unit
// inside one group, whose flattened index is the unit's first value / GS.  A wave
// owns 256 consecutive units and lane l takes units l, l + 64, l + 128, l + 192,
// so every load instruction reads 256 (int4) or 512 (int8) contiguous bytes and
// every store writes 1 KiB contiguous.  (Four consecutive units per lane, one
// 16-byte load and four 16-byte stores 64 bytes apart, measured 14.3 against 7.9
// us on a 32768 x 512 int4 band: every store instruction then touched 32 lines
// with partial writes.)  Packed words are read and bf16 values written
// nontemporally: nothing here is read again by this kernel.
template <int BITS, int GS, bool IDX>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint16_t* __restrict__ biases,
                                                      const uint32_t* __restrict__ idx,
                                                      int64_t table_rows, uint32_t* err_flag,
                                                      uint16_t* __restrict__ out, int64_t units,
                                                      int64_t upr) {
  constexpr int WPU = BITS / 4;  // packed words per unit
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  static_assert(GS % 8 == 0 && GS >= 32, "a unit lies inside one group");
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 256;
  auto convert = [&](const uint32_t (&wd)[WPU], float sv, float bv) {
    u32x4 o;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t word = wd[(2 * p) / (32 / BITS)];
      const int sh = ((2 * p) % (32 / BITS)) * BITS;
      const float q0 = (float)((word >> sh) & MASK);
      const float q1 = (float)((word >> (sh + BITS)) & MASK);
      // v_cvt_pk_bf16_f32 rounds to nearest-even like the oracle's software
      // rounding (checked over subnormal, overflowing and NaN-producing scales)
      const uint32_t m = pack_bf16x2(q0 * sv, q1 * sv);
      o[p] = pack_bf16x2(bf16_lo(m) + bv, bf16_hi(m) + bv);
    }
    return o;
  };
  auto load_unit = [&](int64_t src, uint32_t (&wd)[WPU]) {
    if constexpr (WPU == 1) {
      wd[0] = __builtin_nontemporal_load(w + src);
    } else {
      const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(w) + src);
      wd[0] = v[0];
      wd[1] = v[1];
    }
  };
  for (int64_t base = wave0; base < units; base += (int64_t)gridDim.x * 1024) {
    if constexpr (!IDX) {
      // The lane's four units' words first, then their scales and biases, then
      // the values (this order measured 9.8 -> 7.8 us on a 32768 x 512 band
      // against one that moved a unit's loads next to its store).
      uint32_t wd[4][WPU];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t i = base + lane + 64 * u;
        if (i < units) load_unit(i, wd[u]);
        else
#pragma unroll
          for (int k = 0; k < WPU; ++k) wd[u][k] = 0u;
      }
      float sv[4], bv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        int64_t i = base + lane + 64 * u;
        i = i < units ? i : units - 1;
        const int64_t g = i * 8 / GS;
        sv[u] = bf16_bits_to_f32(scales[g]);
        bv[u] = bf16_bits_to_f32(biases[g]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t i = base + lane + 64 * u;
        if (i >= units) continue;
        __builtin_nontemporal_store(convert(wd[u], sv[u], bv[u]), reinterpret_cast<u32x4*>(out) + i);
      }
    } else {
      // Source unit of each of the lane's four in its table row; a row index
      // past the table gives a zero unit and raises the flag.
      int64_t src[4];
      bool bad[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t i = base + lane + 64 * u;
        const int64_t c = i < units ? i : units - 1;
        const int64_t r = c / upr;
        const int64_t row = idx[r];
        bad[u] = row >= table_rows;
        src[u] = bad[u] ? 0 : row * upr + (c - r * upr);
      }
      uint32_t wd[4][WPU];
#pragma unroll
      for (int u = 0; u < 4; ++u) load_unit(src[u], wd[u]);
      float sv[4], bv[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t g = src[u] * 8 / GS;
        sv[u] = bf16_bits_to_f32(scales[g]);
        bv[u] = bf16_bits_to_f32(biases[g]);
      }
      bool raise = false;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t i = base + lane + 64 * u;
        if (i >= units) continue;
        raise |= bad[u];
        const u32x4 o = bad[u] ? u32x4{0u, 0u, 0u, 0u} : convert(wd[u], sv[u], bv[u]);
        __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(out) + i);
      }
      if (raise) atomicOr(err_flag, 1u);
    }
  }
}

template <int BITS, bool IDX>
hipError_t launch_deq_gs(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                         uint16_t* out, int64_t units, int64_t upr, int group_size,
                         const uint32_t* idx, int64_t table_rows, uint32_t* err_flag,
                         unsigned blocks, hipStream_t stream) {
  switch (group_size) {
    case 32:
      dequant_kernel<BITS, 32, IDX><<<blocks, 256, 0, stream>>>(w, scales, biases, idx,
                                                                table_rows, err_flag, out, units,
                                                                upr);
      break;
    case 64:
      dequant_kernel<BITS, 64, IDX><<<blocks, 256, 0, stream>>>(w, scales, biases, idx,
                                                                table_rows, err_flag, out, units,
                                                                upr);
      break;
    case 128:
      dequant_kernel<BITS, 128, IDX><<<blocks, 256, 0, stream>>>(w, scales, biases, idx,
                                                                 table_rows, err_flag, out,
                                                                 units, upr);
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
  // K % 32 == 0 is guaranteed by the caller, so a row holds whole 8-value units.
  const int64_t upr = K / 8;
  const int64_t units = rows * upr;
  if (units == 0) return hipSuccess;
  int64_t blocks = (units + 1023) / 1024;  // 4 waves x 256 units per block and pass
  if (blocks > 65536) blocks = 65536;
  const unsigned g = (unsigned)blocks;
  if (bits == 4)
    return idx ? launch_deq_gs<4, true>(w, scales, biases, out, units, upr, group_size, idx,
                                        table_rows, err_flag, g, stream)
               : launch_deq_gs<4, false>(w, scales, biases, out, units, upr, group_size, idx,
                                         table_rows, err_flag, g, stream);
  if (bits == 8)
    return idx ? launch_deq_gs<8, true>(w, scales, biases, out, units, upr, group_size, idx,
                                        table_rows, err_flag, g, stream)
               : launch_deq_gs<8, false>(w, scales, biases, out, units, upr, group_size, idx,
                                         table_rows, err_flag, g, stream);
  return hipErrorInvalidValue;
}

}  // namespace fmxq
