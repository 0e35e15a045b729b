// fmxq_mfma_frag.hpp -- MFMA operand fragments built straight from packed
// weights (exponent trick) and from bf16 x, shared by the skinny GEMV and the
// grouped gather kernel.
//
// For v_mfma_f32_32x32x16_bf16 a lane supplies 8 bf16 values per operand.
// wfrag<4>(w): one int4 word (values q0..q7) -> pairs (q0,q4) (q1,q5) (q2,q6)
//   (q3,q7), each value as bf16(128 + q) = 0x4300 | q.
// wfrag<8>(w): one int8 word (values e0..e3) -> (lo e0, lo e2) (hi e0, hi e2)
//   (lo e1, lo e3) (hi e1, hi e3) with lo as bf16(128 + lo) and hi as
//   bf16(2048 + 16 hi) = 0x4500 | hi, so the pair sums to 2176 + q.
// xfrag4 / xfrag8 put x in the same order, so A . B sums x * (offset + q).
#pragma once
#include "fmxq_common.hpp"

namespace fmxq {

__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  const u32x4 v = {a, b, c, d};
  return __builtin_bit_cast(bf16x8, v);
}

// 16 bytes of x (x0..x7) -> (x0,x4) (x1,x5) (x2,x6) (x3,x7).
__device__ __forceinline__ bf16x8 xfrag4(const u32x4 a) {
  return as_bf16x8(__builtin_amdgcn_perm(a[2], a[0], 0x05040100u),
                   __builtin_amdgcn_perm(a[2], a[0], 0x07060302u),
                   __builtin_amdgcn_perm(a[3], a[1], 0x05040100u),
                   __builtin_amdgcn_perm(a[3], a[1], 0x07060302u));
}
// 8 bytes of x (x0..x3) -> (x0,x2) (x0,x2) (x1,x3) (x1,x3).
__device__ __forceinline__ bf16x8 xfrag8(uint32_t a01, uint32_t a23) {
  const uint32_t e = __builtin_amdgcn_perm(a23, a01, 0x05040100u);
  const uint32_t o = __builtin_amdgcn_perm(a23, a01, 0x07060302u);
  return as_bf16x8(e, e, o, o);
}

__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t magic) {
  return (a & mask) | magic;
}

// The magic constants live in VGPRs (vgpr_const) so each pair is one v_and_or_b32.
template <int BITS>
__device__ __forceinline__ bf16x8 wfrag(uint32_t w) {
  constexpr uint32_t K = 0x000F000Fu;
  if constexpr (BITS == 4) {
    const uint32_t M = vgpr_const(0x43004300u);
    return as_bf16x8(and_or(w, K, M), and_or(w >> 4, K, M), and_or(w >> 8, K, M),
                     and_or(w >> 12, K, M));
  } else {
    const uint32_t LO = vgpr_const(0x43004300u), HI = vgpr_const(0x45004500u);
    return as_bf16x8(and_or(w, K, LO), and_or(w >> 4, K, HI), and_or(w >> 8, K, LO),
                     and_or(w >> 12, K, HI));
  }
}

// One 4-bit word (q0..q7, least significant first) dequantized in natural order:
// the bf16 pairs (w0, w1) (w2, w3) (w4, w5) (w6, w7) of w = bf16(fma(s, q, b)), the
// exact s q + b rounded once.  The even nibbles are masked into bytes (q0 q2 q4 q6)
// and the odd nibbles kept in place (16 q1 ..), so each value is one
// v_cvt_f32_ubyteN; the odd ones take s16 = s / 16, which is exact, so
// s16 * (16 q) = s * q and the fma is the same exact s q + b.  The empty asm hides
// the masks' known bits, which would otherwise turn each byte pick into a
// bit-field extract plus a conversion.
__device__ __forceinline__ bf16x8 deq_frag4(uint32_t w, float s, float s16, float b) {
  uint32_t e = w & 0x0F0F0F0Fu, o = w & 0xF0F0F0F0u;
  asm("" : "+v"(e), "+v"(o));
  const u32x4 r = {
      pack_bf16x2(__builtin_fmaf(s, (float)(e & 0xffu), b), __builtin_fmaf(s16, (float)(o & 0xffu), b)),
      pack_bf16x2(__builtin_fmaf(s, (float)((e >> 8) & 0xffu), b),
                  __builtin_fmaf(s16, (float)((o >> 8) & 0xffu), b)),
      pack_bf16x2(__builtin_fmaf(s, (float)((e >> 16) & 0xffu), b),
                  __builtin_fmaf(s16, (float)((o >> 16) & 0xffu), b)),
      pack_bf16x2(__builtin_fmaf(s, (float)(e >> 24), b), __builtin_fmaf(s16, (float)(o >> 24), b))};
  return __builtin_bit_cast(bf16x8, r);
}

// Two 8-bit words (q0..q7, least significant byte of w0 first) dequantized in
// natural order: the bf16 pairs of w = bf16(fma(s, q, b)), the exact s q + b
// rounded once; each byte is one v_cvt_f32_ubyteN.
__device__ __forceinline__ bf16x8 deq_frag8(uint32_t w0, uint32_t w1, float s, float b) {
  const u32x4 r = {pack_bf16x2(__builtin_fmaf(s, (float)(w0 & 0xffu), b),
                               __builtin_fmaf(s, (float)((w0 >> 8) & 0xffu), b)),
                   pack_bf16x2(__builtin_fmaf(s, (float)((w0 >> 16) & 0xffu), b),
                               __builtin_fmaf(s, (float)(w0 >> 24), b)),
                   pack_bf16x2(__builtin_fmaf(s, (float)(w1 & 0xffu), b),
                               __builtin_fmaf(s, (float)((w1 >> 8) & 0xffu), b)),
                   pack_bf16x2(__builtin_fmaf(s, (float)((w1 >> 16) & 0xffu), b),
                               __builtin_fmaf(s, (float)(w1 >> 24), b))};
  return __builtin_bit_cast(bf16x8, r);
}

// Exponent-trick offset per value and the factor that turns the ones-MFMA sum of
// the A operand back into sum x (int8 A carries every x value twice).
template <int BITS>
__device__ __forceinline__ constexpr float frag_offset() { return BITS == 4 ? 128.f : 2176.f; }
template <int BITS>
__device__ __forceinline__ constexpr float frag_xscale() { return BITS == 4 ? 1.f : 0.5f; }

}  // namespace fmxq
