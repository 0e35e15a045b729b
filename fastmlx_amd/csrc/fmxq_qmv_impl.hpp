// fmxq_qmv_impl.hpp -- the decode GEMV body shared by quantized_matmul (M <= 4)
// and the gathered per-slot product of gather_qmm.
//
// Work split: a wave owns R consecutive output rows over the whole K axis.
// Lane l walks 16-byte chunks c = l, l+64, ... of each row (32 int4 or 16 int8
// values), so a wave-wide load reads 1 KiB of contiguous packed weight per row.
// The x chunk a lane needs is loaded once per chunk and reused for all R rows.
//
// Arithmetic (no MFMA): the packed nibbles are turned into bf16 pairs with the
// exponent trick (0x4300 | q) == bf16(128 + q) and multiplied against x with
// v_dot2_f32_bf16, so the dot product over a chunk is
//     d = sum_k x_k (128 + q_k) = sum_k x_k q_k + 128 * sum_k x_k.
// A chunk never straddles a quantization group (chunk <= 32 <= group), so
//     sum_k x_k (s q_k + b) = s * d + (b - 128 s) * sum_k x_k.
// int8 values are split into two nibbles: q = lo + 16 hi, giving
//     sum_k x_k q_k = d_lo + 16 d_hi - 2176 * sum_k x_k.
// Accumulation is fp32 throughout; the result is rounded to bf16 once.
#pragma once
#include "fmxq_common.hpp"

namespace fmxq {

constexpr uint32_t kMagic = 0x43004300u;   // bf16 pair (128, 128) exponent bits
constexpr uint32_t kNib2 = 0x000F000Fu;    // one nibble in each 16-bit half
constexpr uint32_t kOnes = 0x3F803F80u;    // bf16 pair (1.0, 1.0)

// (w & kNib2) | magic as one v_and_or_b32 (magic from vgpr_const).
__device__ __forceinline__ uint32_t nib_pair(uint32_t w, uint32_t vmagic) {
  return (w & kNib2) | vmagic;
}

// x pairs matching the nibble pairing of one int4 word: (x0,x4) (x1,x5) (x2,x6) (x3,x7).
__device__ __forceinline__ void x_pairs_q4(const u32x4 a, uint32_t* p) {
  p[0] = (a[0] & 0xffffu) | (a[2] << 16);
  p[1] = (a[0] >> 16) | (a[2] & 0xffff0000u);
  p[2] = (a[1] & 0xffffu) | (a[3] << 16);
  p[3] = (a[1] >> 16) | (a[3] & 0xffff0000u);
}

// x pairs for one int8 word (elements e0..e3): (x0,x2) (x1,x3).
__device__ __forceinline__ void x_pairs_q8(uint32_t a01, uint32_t a23, uint32_t* p) {
  p[0] = (a01 & 0xffffu) | (a23 << 16);
  p[1] = (a01 >> 16) | (a23 & 0xffff0000u);
}

// Chunk of x for one row of x: CH values starting at k0, already paired, plus their sum.
template <int BITS>
struct XChunk {
  static constexpr int CH = 128 / BITS;       // values per 16-byte weight chunk
  static constexpr int NP = (BITS == 4) ? 16 : 8;
  uint32_t p[NP];
  float sum;

  __device__ __forceinline__ void load(const uint16_t* __restrict__ xrow, int64_t k0) {
    const u32x4* src = reinterpret_cast<const u32x4*>(xrow + k0);
    float s = 0.f;
    if constexpr (BITS == 4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x4 a = src[j];
        x_pairs_q4(a, p + 4 * j);
        s = dot2_bf16(a[0], kOnes, s);
        s = dot2_bf16(a[1], kOnes, s);
        s = dot2_bf16(a[2], kOnes, s);
        s = dot2_bf16(a[3], kOnes, s);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const u32x4 a = src[j];
        x_pairs_q8(a[0], a[1], p + 4 * j);
        x_pairs_q8(a[2], a[3], p + 4 * j + 2);
        s = dot2_bf16(a[0], kOnes, s);
        s = dot2_bf16(a[1], kOnes, s);
        s = dot2_bf16(a[2], kOnes, s);
        s = dot2_bf16(a[3], kOnes, s);
      }
    }
    sum = s;
  }
};

// Contribution of one 16-byte weight chunk (4 packed words) against one x chunk,
// before scaling: returns d (int4) or d_lo + 16 d_hi (int8).
template <int BITS>
__device__ __forceinline__ float chunk_dot(const u32x4 wv, const XChunk<BITS>& xc) {
  const uint32_t m = vgpr_const(kMagic);
  if constexpr (BITS == 4) {
    float d = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = wv[j];
      d = dot2_bf16(nib_pair(w, m), xc.p[4 * j + 0], d);
      d = dot2_bf16(nib_pair(w >> 4, m), xc.p[4 * j + 1], d);
      d = dot2_bf16(nib_pair(w >> 8, m), xc.p[4 * j + 2], d);
      d = dot2_bf16(nib_pair(w >> 12, m), xc.p[4 * j + 3], d);
    }
    return d;
  } else {
    float dl = 0.f, dh = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = wv[j];
      dl = dot2_bf16(nib_pair(w, m), xc.p[2 * j + 0], dl);
      dh = dot2_bf16(nib_pair(w >> 4, m), xc.p[2 * j + 0], dh);
      dl = dot2_bf16(nib_pair(w >> 8, m), xc.p[2 * j + 1], dl);
      dh = dot2_bf16(nib_pair(w >> 12, m), xc.p[2 * j + 1], dh);
    }
    return dl + 16.f * dh;
  }
}

// The 16 exponent-trick bf16 pairs of one 16-byte weight chunk, unpacked once so
// several x rows can be dotted against them: p[4j + t] = pair t of word j
// (nibbles t and t+4 of the word).
__device__ __forceinline__ void unpack_chunk(const u32x4 wv, uint32_t (&p)[16]) {
  const uint32_t m = vgpr_const(kMagic);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = wv[j];
    p[4 * j + 0] = nib_pair(w, m);
    p[4 * j + 1] = nib_pair(w >> 4, m);
    p[4 * j + 2] = nib_pair(w >> 8, m);
    p[4 * j + 3] = nib_pair(w >> 12, m);
  }
}

// chunk_dot() over pre-unpacked pairs.
template <int BITS>
__device__ __forceinline__ float dot_pairs(const uint32_t (&p)[16], const XChunk<BITS>& xc) {
  if constexpr (BITS == 4) {
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) d = dot2_bf16(p[i], xc.p[i], d);
    return d;
  } else {
    float dl = 0.f, dh = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dl = dot2_bf16(p[4 * j + 0], xc.p[2 * j + 0], dl);
      dh = dot2_bf16(p[4 * j + 1], xc.p[2 * j + 0], dh);
      dl = dot2_bf16(p[4 * j + 2], xc.p[2 * j + 1], dl);
      dh = dot2_bf16(p[4 * j + 3], xc.p[2 * j + 1], dh);
    }
    return dl + 16.f * dh;
  }
}

// Sums V per-lane partials over the 64 lanes in one pass (V a power of two <= 64):
// at each offset o = 32, 16, ... the lanes with bit o set keep the upper half of
// their values and swap the lower half with their partner, halving the count.
// Lane l returns the total of value index l >> (6 - log2 V); every lane with the
// same index holds the same total.  Costs about V + log2(64/V) shuffle-adds
// instead of V full reductions.
// The halves are chosen with a bit select through an opaque mask: written as
// `up ? v[a] : v[b]`, the compiler folds the select into a lane-dependent array
// index, which forces v[] out of registers (into LDS).
template <int V>
__device__ __forceinline__ float wave_sum_multi(float (&v)[V], int lane) {
  static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V must be a power of two <= 64");
#pragma unroll
  for (int c = V, o = 32; c > 1; c >>= 1, o >>= 1) {
    uint32_t msk = (lane & o) ? 0xffffffffu : 0u;
    asm("" : "+v"(msk));
#pragma unroll
    for (int i = 0; i < c / 2; ++i) {
      const uint32_t lo = __float_as_uint(v[i]), hi = __float_as_uint(v[c / 2 + i]);
      const float keep = __uint_as_float((msk & hi) | (~msk & lo));
      const float send = __uint_as_float((msk & lo) | (~msk & hi));
      v[i] = keep + __shfl_xor(send, o, 64);
    }
  }
  // The lanes sharing an index form aligned groups of G = 64 / V.  Within a row of
  // 16 lanes the group sum uses DPP (quad swaps, half-row and row mirrors); wider
  // groups fall back to cross-row shuffles.
  constexpr int G = 64 / V;
  float s = v[0];
  if constexpr (G >= 2) s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0xb1, 0xf, 0xf, false));
  if constexpr (G >= 4) s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x4e, 0xf, 0xf, false));
  if constexpr (G >= 8) s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x141, 0xf, 0xf, false));
  if constexpr (G >= 16) s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x140, 0xf, 0xf, false));
  if constexpr (G >= 32) s += __shfl_xor(s, 16, 64);
  if constexpr (G >= 64) s += __shfl_xor(s, 32, 64);
  return s;
}

// Offset that turns the exponent-trick dot product back into sum x*q.
template <int BITS>
__device__ __forceinline__ constexpr float magic_offset() {
  return BITS == 4 ? 128.f : 2176.f;
}

// One wave computes rows [n0, n0+R) x MM rows of x over the whole K axis.
// xrows[m] points at row m of x; wbase/sbase/bbase at row 0 of the weight
// matrix being read (an expert slice for gather_qmm).
template <int BITS, int MM, int R>
__device__ __forceinline__ void qmv_wave(const uint16_t* const* xrows,
                                         const uint32_t* __restrict__ wbase,
                                         const uint16_t* __restrict__ sbase,
                                         const uint16_t* __restrict__ bbase, int64_t n0,
                                         int64_t N, int64_t K, int group_size, float (&acc)[R][MM]) {
  constexpr int CH = 128 / BITS;
  const int lane = threadIdx.x & 63;
  const int64_t nchunks = K / CH;
  const int64_t wpr = K * BITS / 32;
  const int gshift = __builtin_ctz((unsigned)group_size);  // group_size is a power of two
  const int64_t gpr = K >> gshift;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[r][m] = 0.f;

  for (int64_t c = lane; c < nchunks; c += 64) {
    const int64_t k0 = c * CH;
    const int64_t g = k0 >> gshift;
    u32x4 wv[R];
    float s[R], bc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t n = n0 + r;
      if (n < N) {
        wv[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wbase + n * wpr) + c);
        s[r] = bf16_bits_to_f32(sbase[n * gpr + g]);
        bc[r] = bf16_bits_to_f32(bbase[n * gpr + g]);
      } else {
        wv[r] = u32x4{0u, 0u, 0u, 0u};
        s[r] = 0.f;
        bc[r] = 0.f;
      }
    }
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      XChunk<BITS> xc;
      xc.load(xrows[m], k0);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float d = chunk_dot<BITS>(wv[r], xc);
        const float boff = bc[r] - magic_offset<BITS>() * s[r];
        acc[r][m] += s[r] * d + boff * xc.sum;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[r][m] = wave_sum(acc[r][m]);
}

}  // namespace fmxq
