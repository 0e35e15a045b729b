// fmx_ingest.hip -- device side of the weight ingest: the int4 affine bias
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

}  // namespace

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
