// fmx_index.hip -- index materialization for gather_qmm's MLX batch semantics.
//
// mlx_gather_qmm (called at mlxgo/binding_cgo.go:645-673) broadcasts lhs_indices
// and rhs_indices against each other and, when either is absent, uses the arange
// over x's (or w's) batch axes.  The gather kernels read one uint32 index per
// output item, so the array layer turns any integral index array (or the implicit
// arange) into that flat form here: one thread per output item, coordinates
// decoded from the row-major output batch shape, strided read, range-safe
// conversion.  Index arrays are a few KB at most; this is a launch, not a kernel
// worth a roofline.
#include "fmxq_internal.hpp"

namespace fmxq {

__global__ __launch_bounds__(256) void broadcast_index_kernel(const void* __restrict__ src,
                                                              IndexMap m,
                                                              uint32_t* __restrict__ out,
                                                              int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    int64_t rem = i;
    int64_t off = 0;
    for (int d = m.ndim - 1; d >= 0; --d) {
      const int64_t c = rem % m.shape[d];
      rem /= m.shape[d];
      off += c * m.stride[d];
    }
    uint32_t v;
    if (!src) {
      v = off > 0xffffffffLL ? 0xffffffffu : (uint32_t)off;
    } else if (m.elem_bytes == 4) {
      const uint32_t raw = static_cast<const uint32_t*>(src)[off];
      v = (m.is_signed && (int32_t)raw < 0) ? 0xffffffffu : raw;
    } else if (m.elem_bytes == 8) {
      const uint64_t raw = static_cast<const uint64_t*>(src)[off];
      v = (m.is_signed && (int64_t)raw < 0) || raw > 0xffffffffull ? 0xffffffffu : (uint32_t)raw;
    } else if (m.elem_bytes == 2) {
      const uint16_t raw = static_cast<const uint16_t*>(src)[off];
      v = (m.is_signed && (int16_t)raw < 0) ? 0xffffffffu : raw;
    } else {
      const uint8_t raw = static_cast<const uint8_t*>(src)[off];
      v = (m.is_signed && (int8_t)raw < 0) ? 0xffffffffu : raw;
    }
    out[i] = v;
  }
}

hipError_t launch_broadcast_index(const void* src, const IndexMap& m, uint32_t* out, int64_t n,
                                  hipStream_t stream) {
  if (n == 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  broadcast_index_kernel<<<(unsigned)blocks, 256, 0, stream>>>(src, m, out, n);
  return hipGetLastError();
}

}  // namespace fmxq
