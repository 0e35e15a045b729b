// fmxq_common.hpp -- shared device helpers for the gfx950 quantized-linear kernels.
//
// Weight layout (MLX affine quantization, transpose=true):
//   w       [rows, K*bits/32] uint32; element k of a row sits at bit (k % (32/bits))*bits
//           of word k / (32/bits), least significant first
//   scales  [rows, K/group] bf16, biases [rows, K/group] bf16
//   x       [M, K] bf16 row-major; y [M, N] bf16 row-major
// Dequantized value: w = scale * q + bias (see fmxq_dequant.hip for the exact rounding).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fmxq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

// fp32 -> bf16, round to nearest even, through the hardware conversion
// (v_cvt_pk_bf16_f32: one instruction against five for the integer form).  Every
// finite value, subnormals and overflow to infinity included, gets the bits of
// the integer rounding.  A NaN gives some quiet NaN whose payload bits are the
// hardware's choice; the bit-exact dequantize tests accept any NaN where the
// oracle has one, and no other test feeds NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Hardware conversion of two floats into a packed bf16 pair (v_cvt_pk_bf16_f32, RNE).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2 r;
  r.x = (__bf16)lo;
  r.y = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, r);
}

// A compile-time constant materialised in a VGPR.  gfx9 VOP3 encodings take no
// literal and at most one SGPR, so (w & mask) | magic only becomes a single
// v_and_or_b32 when one of the two constants already sits in a VGPR; otherwise
// the compiler splits it into v_and_b32 + v_or_b32 with literals.
__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
  uint32_t v;
  asm("v_mov_b32 %0, %1" : "=v"(v) : "i"(c));
  return v;
}

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                         __builtin_bit_cast(bf16x2, b), c, false);
}

__device__ __forceinline__ uint32_t perm_b32(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

// Epilogue rounding of one output: bf16(acc), then, when an additive bias is
// present, bf16(bf16(acc) + bias) -- the qlinear then add op chain
// (compute/models/quant.go:105-111).
__device__ __forceinline__ uint16_t finish_out(float acc, const uint16_t* bias, int64_t n) {
  uint32_t v = f32_to_bf16_rne(acc);
  if (bias) v = f32_to_bf16_rne(bf16_bits_to_f32(v) + bf16_bits_to_f32(bias[n]));
  return (uint16_t)v;
}

// Wave64 butterfly sum.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace fmxq
