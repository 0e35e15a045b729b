// fmxq_qmv.hip -- decode GEMV (M <= 4) for quantized_matmul and the per-slot
// gathered GEMV of gather_qmm.
//
// Replaces the decode side of mlx_quantized_matmul (mlxgo/binding_cgo.go:636-643,
// reached from compute/models/quant.go:91-101 on every decode step) and the
// short-routing gather of mlx_gather_qmm (switch_glu.go:124-130 -> :179-186).
// The kernel body is in fmxq_qmv_impl.hpp.
#include "fmxq_internal.hpp"
#include "fmxq_qmv_impl.hpp"

namespace fmxq {

template <int BITS, int MM, int R>
__global__ __launch_bounds__(256) void qmv_kernel(QmmArgs a) {
  const int wave = threadIdx.x >> 6;
  const int64_t n0 = ((int64_t)blockIdx.x * 4 + wave) * R;
  if (n0 >= a.N) return;  // uniform per wave
  const uint16_t* xrows[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) xrows[m] = a.x + (int64_t)m * a.ldx;
  float acc[R][MM];
  qmv_wave<BITS, MM, R>(xrows, a.w, a.scales, a.biases, n0, a.N, a.K, a.group_size, acc);
  const int lane = threadIdx.x & 63;
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int64_t n = n0 + r;
      if (n < a.N) {
#pragma unroll
        for (int m = 0; m < MM; ++m) a.y[(int64_t)m * a.ldy + n] = finish_out(acc[r][m], a.bias, n);
      }
    }
  }
}

// Rows per wave: enough waves to cover the chip (about 8 per CU on 256 CUs)
// before a wave takes several rows and shares its x chunk across them.
static int pick_rows_per_wave(int64_t N) {
  if (N >= 4 * 2048) return 4;
  if (N >= 2 * 2048) return 2;
  return 1;
}

template <int BITS, int MM>
static hipError_t launch_qmv_m(const QmmArgs& a, hipStream_t stream) {
  const int R = pick_rows_per_wave(a.N);
  const int64_t rows_per_block = 4 * (int64_t)R;
  const unsigned blocks = (unsigned)((a.N + rows_per_block - 1) / rows_per_block);
  if (R == 4)
    qmv_kernel<BITS, MM, 4><<<blocks, 256, 0, stream>>>(a);
  else if (R == 2)
    qmv_kernel<BITS, MM, 2><<<blocks, 256, 0, stream>>>(a);
  else
    qmv_kernel<BITS, MM, 1><<<blocks, 256, 0, stream>>>(a);
  return hipGetLastError();
}

template <int BITS>
static hipError_t launch_qmv_bits(const QmmArgs& a, hipStream_t stream) {
  switch (a.M) {
    case 1: return launch_qmv_m<BITS, 1>(a, stream);
    case 2: return launch_qmv_m<BITS, 2>(a, stream);
    case 3: return launch_qmv_m<BITS, 3>(a, stream);
    default: return launch_qmv_m<BITS, 4>(a, stream);
  }
}

hipError_t launch_qmv(const QmmArgs& a, hipStream_t stream) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  return a.bits == 4 ? launch_qmv_bits<4>(a, stream) : launch_qmv_bits<8>(a, stream);
}

// ---------------------------------------------------------------------------
// Gathered GEMV: grid (row blocks, slots).  Each slot reads its own x row and
// the weight slice of its expert.  An out-of-range expert id writes zeros for
// that slot and raises err_flag instead of reading outside the stack.

template <int BITS, int R>
__global__ __launch_bounds__(256) void gather_qmv_kernel(GatherArgs a) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // Slots run along x so that neighbouring blocks of a sorted batch read the same
  // expert rows close together in time.
  const int64_t slot = blockIdx.x;
  const int64_t n0 = ((int64_t)blockIdx.y * 4 + wave) * R;
  if (n0 >= a.N) return;
  const int64_t item = slot / a.Mx, row = slot - item * a.Mx;
  const int64_t e = a.rhs[item];
  const int64_t xi = a.lhs ? (int64_t)a.lhs[item] : item / a.lhs_div;
  const int64_t xr = xi * a.Mx + row;
  uint16_t* yrow = a.y + slot * a.N;
  if (e >= a.E || xi >= a.x_batch) {
    if (lane == 0) {
      for (int r = 0; r < R; ++r)
        if (n0 + r < a.N) yrow[n0 + r] = 0;
      atomicOr(a.err_flag, 1u);
    }
    return;
  }
  const int64_t wpr = a.K * BITS / 32, gpr = a.K / a.group_size;
  const uint16_t* xrows[1] = {a.x + xr * a.K};
  float acc[R][1];
  qmv_wave<BITS, 1, R>(xrows, a.w + e * a.N * wpr, a.scales + e * a.N * gpr,
                       a.biases + e * a.N * gpr, n0, a.N, a.K, a.group_size, acc);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (n0 + r < a.N) yrow[n0 + r] = finish_out(acc[r][0], nullptr, n0 + r);
  }
}

template <int BITS>
static hipError_t launch_gather_qmv_bits(const GatherArgs& a, hipStream_t stream) {
  const int64_t S = a.batch * a.Mx;
  const int R = (a.N * S >= 4 * 2048) && (a.N >= 64) ? 2 : 1;
  const int64_t rows_per_block = 4 * (int64_t)R;
  dim3 grid((unsigned)S, (unsigned)((a.N + rows_per_block - 1) / rows_per_block));
  if (R == 2)
    gather_qmv_kernel<BITS, 2><<<grid, 256, 0, stream>>>(a);
  else
    gather_qmv_kernel<BITS, 1><<<grid, 256, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_gather_qmv(const GatherArgs& a, hipStream_t stream) {
  if (a.batch <= 0 || a.Mx <= 0 || a.N <= 0) return hipSuccess;
  return a.bits == 4 ? launch_gather_qmv_bits<4>(a, stream)
                     : launch_gather_qmv_bits<8>(a, stream);
}

}  // namespace fmxq
