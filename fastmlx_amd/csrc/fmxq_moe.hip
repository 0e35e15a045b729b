// fmxq_moe.hip -- the device pieces around gather_qmm in a SwitchGLU MoE layer.
//
// switchGLUCore (compute/models/switch_glu.go:107-153) brackets its three
// gather_qmm calls with argsort / inverse argsort / floor_divide / take (the
// sort branch, :135-150) and silu(gate) * up (:126-127, :146-147).  Here those
// become:
//   - sort_slots_kernel: a counting sort of the flattened routing slots by
//     expert id in one block (replaces argsort + take + floor_divide); the
//     order inside an expert is arbitrary, which cannot change any value
//     because every slot is its own GEMM row;
//   - silu_mul_kernel: h = bf16(bf16(g * bf16(sigmoid(g))) * u), the rounding of
//     the silu (sigmoid then mul, qwen3_forward.go:229-239) then mul op chain;
//   - the unsort is fused into the down projection's store (GatherArgs::yrow).
// moe_combine_kernel is the weighted top-k sum plus optional shared expert of
// qwen3next_forward.go:519-524 and deepseekv3_forward.go:436-440.
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"

namespace fmxq {

// One block: counts per expert in LDS, exclusive scan, scatter.  Ids >= E go
// to a final bucket (the gather kernels zero those rows and raise the flag).
__global__ __launch_bounds__(1024) void sort_slots_kernel(const uint32_t* __restrict__ inds,
                                                          int64_t S, int64_t topk, int64_t E,
                                                          uint32_t* __restrict__ order,
                                                          uint32_t* __restrict__ rhs_sorted,
                                                          uint32_t* __restrict__ lhs_sorted) {
  extern __shared__ uint32_t cnt[];  // E + 1 counters, then E + 1 cursors
  const int64_t nb = E + 1;
  uint32_t* cur = cnt + nb;
  for (int64_t i = threadIdx.x; i < nb; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  for (int64_t s = threadIdx.x; s < S; s += blockDim.x) {
    const uint32_t e = inds[s];
    atomicAdd(&cnt[e < (uint64_t)E ? e : E], 1u);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t run = 0;
    for (int64_t i = 0; i < nb; ++i) {
      cur[i] = run;
      run += cnt[i];
    }
  }
  __syncthreads();
  for (int64_t s = threadIdx.x; s < S; s += blockDim.x) {
    const uint32_t e = inds[s];
    const uint32_t pos = atomicAdd(&cur[e < (uint64_t)E ? e : E], 1u);
    order[pos] = (uint32_t)s;
    rhs_sorted[pos] = e;
    lhs_sorted[pos] = (uint32_t)(s / topk);
  }
}

__device__ __forceinline__ float r16(float v) { return bf16_bits_to_f32(f32_to_bf16_rne(v)); }

// 8 elements per thread; n is a multiple of 8.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ g,
                                                       const uint16_t* __restrict__ u,
                                                       uint16_t* __restrict__ h, int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
    const u32x4 gv = reinterpret_cast<const u32x4*>(g)[i];
    const u32x4 uv = reinterpret_cast<const u32x4*>(u)[i];
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float g0 = bf16_lo(gv[j]), g1 = bf16_hi(gv[j]);
      const float s0 = r16(1.f / (1.f + __expf(-g0))), s1 = r16(1.f / (1.f + __expf(-g1)));
      const float h0 = r16(r16(g0 * s0) * bf16_lo(uv[j]));
      const float h1 = r16(r16(g1 * s1) * bf16_hi(uv[j]));
      o[j] = f32_to_bf16_rne(h0) | (f32_to_bf16_rne(h1) << 16);
    }
    reinterpret_cast<u32x4*>(h)[i] = o;
  }
}

// out[t] = bf16( bf16(sum_j bf16(y[t,j] * w[t,j])) + shared_term ), shared_term =
// bf16(bf16(sigmoid(sg[t])) * shared[t]) with a gate, shared[t] without, none if
// shared is null.  One thread per (t, d) pair of 2 columns.
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t* __restrict__ y,
                                                          const uint16_t* __restrict__ w,
                                                          const uint16_t* __restrict__ shared,
                                                          const uint16_t* __restrict__ sgate,
                                                          uint16_t* __restrict__ out, int64_t T,
                                                          int64_t topk, int64_t D) {
  const int64_t pairs = D / 2;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < T * pairs;
       i += (int64_t)gridDim.x * 256) {
    const int64_t t = i / pairs, d = (i - t * pairs) * 2;
    float a0 = 0.f, a1 = 0.f;
    for (int64_t j = 0; j < topk; ++j) {
      const float wj = bf16_bits_to_f32(w[t * topk + j]);
      const uint32_t v = *reinterpret_cast<const uint32_t*>(y + (t * topk + j) * D + d);
      a0 += r16(bf16_lo(v) * wj);
      a1 += r16(bf16_hi(v) * wj);
    }
    a0 = r16(a0);
    a1 = r16(a1);
    if (shared) {
      const uint32_t sv = *reinterpret_cast<const uint32_t*>(shared + t * D + d);
      float s0 = bf16_lo(sv), s1 = bf16_hi(sv);
      if (sgate) {
        const float gt = r16(1.f / (1.f + __expf(-bf16_bits_to_f32(sgate[t]))));
        s0 = r16(gt * s0);
        s1 = r16(gt * s1);
      }
      a0 = r16(a0 + s0);
      a1 = r16(a1 + s1);
    }
    *reinterpret_cast<uint32_t*>(out + t * D + d) = f32_to_bf16_rne(a0) | (f32_to_bf16_rne(a1) << 16);
  }
}

static unsigned grid_for(int64_t items, int64_t per_block) {
  int64_t b = (items + per_block - 1) / per_block;
  if (b > 65536) b = 65536;
  return (unsigned)(b < 1 ? 1 : b);
}

hipError_t launch_sort_slots(const uint32_t* inds, int64_t S, int64_t topk, int64_t E,
                             uint32_t* order, uint32_t* rhs_sorted, uint32_t* lhs_sorted,
                             hipStream_t stream) {
  const size_t lds = (size_t)(E + 1) * 2 * sizeof(uint32_t);
  sort_slots_kernel<<<1, 1024, lds, stream>>>(inds, S, topk, E, order, rhs_sorted, lhs_sorted);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* h, int64_t n,
                           hipStream_t stream) {
  const int64_t n8 = n / 8;
  silu_mul_kernel<<<grid_for(n8, 256), 256, 0, stream>>>(g, u, h, n8);
  return hipGetLastError();
}

hipError_t launch_moe_combine(const uint16_t* y, const uint16_t* w, const uint16_t* shared,
                              const uint16_t* sgate, uint16_t* out, int64_t T, int64_t topk,
                              int64_t D, hipStream_t stream) {
  moe_combine_kernel<<<grid_for(T * (D / 2), 256), 256, 0, stream>>>(y, w, shared, sgate, out, T,
                                                                     topk, D);
  return hipGetLastError();
}

}  // namespace fmxq
