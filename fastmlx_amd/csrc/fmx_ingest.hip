// fmx_ingest.hip -- device side of the weight ingest: the axis swap of the
// kv_b_proj absorption (deepseekv3.go:651-658), and the int4 affine bias
// biases = -8 * scale of a compressed-tensors int4 checkpoint, computed in fp32
// and rounded once to the scale's own dtype (scaleNeg8, deepseekv3.go:539-551:
// the product against the float32 scalar promotes to float32, then an astype
// back to the scale dtype).  Scaling by -8 changes only the sign and exponent,
// so the result is exact unless it overflows to infinity.
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"

namespace fmxq {
namespace {

template <int KIND>  // 0 bf16, 1 f16, 2 f32
__global__ __launch_bounds__(256) void scale_neg8_kernel(const void* __restrict__ src,
                                                         void* __restrict__ dst, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256) {
    if constexpr (KIND == 0) {
      const float v = bf16_bits_to_f32(static_cast<const uint16_t*>(src)[i]);
      static_cast<uint16_t*>(dst)[i] = (uint16_t)f32_to_bf16_rne(-8.f * v);
    } else if constexpr (KIND == 1) {
      const float v = (float)static_cast<const _Float16*>(src)[i];
      static_cast<_Float16*>(dst)[i] = (_Float16)(-8.f * v);
    } else {
      static_cast<float*>(dst)[i] = -8.f * static_cast<const float*>(src)[i];
    }
  }
}

// One output element per iteration: dst [A, d2, B, d1, C] from src [A, d1, B, d2, C].
// Load-time reshuffle (swapaxes of the kv_b_proj absorption), not a hot path.
template <typename T>
__global__ __launch_bounds__(256) void swap_axes_kernel(const T* __restrict__ src,
                                                        T* __restrict__ dst, int64_t A,
                                                        int64_t d1, int64_t B, int64_t d2,
                                                        int64_t C) {
  const int64_t n = A * d1 * B * d2 * C;
  for (int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x; o < n;
       o += (int64_t)gridDim.x * 256) {
    int64_t t = o;
    const int64_t c = t % C;
    t /= C;
    const int64_t j1 = t % d1;
    t /= d1;
    const int64_t b = t % B;
    t /= B;
    const int64_t j2 = t % d2;
    const int64_t a = t / d2;
    dst[o] = src[(((a * d1 + j1) * B + b) * d2 + j2) * C + c];
  }
}

}  // namespace

hipError_t launch_swap_axes(const void* src, void* dst, int64_t A, int64_t d1, int64_t B,
                            int64_t d2, int64_t C, int elem_bytes, hipStream_t stream) {
  const int64_t n = A * d1 * B * d2 * C;
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  const unsigned g = (unsigned)blocks;
  switch (elem_bytes) {
    case 1:
      swap_axes_kernel<uint8_t><<<g, 256, 0, stream>>>(static_cast<const uint8_t*>(src),
                                                       static_cast<uint8_t*>(dst), A, d1, B, d2, C);
      break;
    case 2:
      swap_axes_kernel<uint16_t><<<g, 256, 0, stream>>>(static_cast<const uint16_t*>(src),
                                                        static_cast<uint16_t*>(dst), A, d1, B, d2,
                                                        C);
      break;
    case 4:
      swap_axes_kernel<uint32_t><<<g, 256, 0, stream>>>(static_cast<const uint32_t*>(src),
                                                        static_cast<uint32_t*>(dst), A, d1, B, d2,
                                                        C);
      break;
    case 8:
      swap_axes_kernel<uint64_t><<<g, 256, 0, stream>>>(static_cast<const uint64_t*>(src),
                                                        static_cast<uint64_t*>(dst), A, d1, B, d2,
                                                        C);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_scale_neg8(const void* src, void* dst, int64_t n, int kind,
                             hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (kind == 0) scale_neg8_kernel<0><<<(unsigned)blocks, 256, 0, stream>>>(src, dst, n);
  else if (kind == 1) scale_neg8_kernel<1><<<(unsigned)blocks, 256, 0, stream>>>(src, dst, n);
  else if (kind == 2) scale_neg8_kernel<2><<<(unsigned)blocks, 256, 0, stream>>>(src, dst, n);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace fmxq
