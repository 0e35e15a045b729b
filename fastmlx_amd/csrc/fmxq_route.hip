// fmxq_route.hip -- MoE routers: the expert choice and weights that feed
// switchGLU (switch_glu.go:107-153) and the weighted combine.
//
//   - route_kernel<.., GROUP=false>: the softmax router of qwen3NextMoE
//     (qwen3next_forward.go:513-518): gates = softmax(logits), the top_k gates,
//     optionally renormalized over the selection.
//   - route_kernel<.., GROUP=true>: DeepSeek-V3's group-limited router
//     (routeExperts, deepseekv3_forward.go:452-491; CPU restatement
//     GroupExpertSelect, deepseekv3.go:305-384): sigmoid scores plus the
//     correction bias, the topk_group groups with the best sum of their two
//     best biased scores kept (the others' biased scores set to 0), the top_k
//     experts by biased score, their unbiased sigmoid scores optionally
//     renormalized over the selection and scaled by routed_scaling_factor.
//
// One wave per token row.  Element e of the row sits in lane e % 64, slot
// e / 64.  Selection is k rounds of a wave-wide argmax; equal values go to the
// lower index, which is the order the reference's stable sorts produce.  The
// arithmetic is fp32 (the reference fixture for the group router is a float32
// sigmoid compared at 1e-5).  Outputs are written in selection order (highest
// first): inds [T, k] uint32 and weights [T, k] fp32 or bf16.
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"

namespace fmxq {
namespace {

constexpr float kNegInf = -__builtin_inff();

// (v, i) beats (bv, bi) when larger, or equal with the lower index.
__device__ __forceinline__ bool beats(float v, uint32_t i, float bv, uint32_t bi) {
  return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void wave_argmax(float& v, uint32_t& i) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const uint32_t oi = (uint32_t)__shfl_xor((int)i, off, 64);
    if (beats(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// The two largest of the wave's (t1 >= t2) pairs.
__device__ __forceinline__ void wave_top2(float& t1, float& t2) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float o1 = __shfl_xor(t1, off, 64), o2 = __shfl_xor(t2, off, 64);
    const float hi = fmaxf(t1, o1);
    const float lo = fmaxf(fminf(t1, o1), fmaxf(t2, o2));
    t1 = hi;
    t2 = lo;
  }
}

template <typename TIn>
__device__ __forceinline__ float load_in(const TIn* p, int64_t i);
template <>
__device__ __forceinline__ float load_in<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float load_in<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_bits_to_f32(p[i]);
}

template <typename TIn, int EPL, bool GROUP, bool OUT_BF16>
__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.T) return;  // whole waves only: T rows, 4 per block
  const TIn* in = static_cast<const TIn*>(a.logits) + row * a.E;

  float v[EPL];    // selection key
  float src[EPL];  // value the weight is taken from
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int64_t e = lane + 64 * j;
    v[j] = e < a.E ? load_in<TIn>(in, e) : kNegInf;
  }

  if constexpr (!GROUP) {
    float m = kNegInf;
#pragma unroll
    for (int j = 0; j < EPL; ++j) m = fmaxf(m, v[j]);
    m = wave_max(m);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int64_t e = lane + 64 * j;
      v[j] = e < a.E ? expf(v[j] - m) : 0.f;
      s += v[j];
    }
    s = wave_sum(s);
    const float inv = 1.f / s;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int64_t e = lane + 64 * j;
      v[j] = e < a.E ? v[j] * inv : kNegInf;
      src[j] = v[j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const int64_t e = lane + 64 * j;
      if (e < a.E) {
        src[j] = 1.f / (1.f + expf(-v[j]));
        v[j] = src[j] + (a.bias ? a.bias[e] : 0.f);
      } else {
        src[j] = 0.f;
        v[j] = kNegInf;
      }
    }
    if (a.n_group > 1) {
      const int per = (int)(a.E / a.n_group);
      // Group score: the sum of the group's two best biased scores (one when a
      // group holds a single expert).  Every lane ends up with all of them.
      uint64_t keep = 0;
      float gs_lane = kNegInf;  // lane g holds group g's score
      for (int g = 0; g < a.n_group; ++g) {
        float t1 = kNegInf, t2 = kNegInf;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
          const int64_t e = lane + 64 * j;
          if (e < a.E && e / per == g) {
            const float x = v[j];
            t2 = fmaxf(t2, fminf(t1, x));
            t1 = fmaxf(t1, x);
          }
        }
        wave_top2(t1, t2);
        const float score = per > 1 ? t1 + t2 : t1;
        if (lane == g) gs_lane = score;
      }
      // Keep the topk_group best groups (ties to the lower group index).
      for (int r = 0; r < a.topk_group && r < a.n_group; ++r) {
        float bv = gs_lane;
        uint32_t bi = lane < a.n_group ? (uint32_t)lane : 0xffffffffu;
        if (lane >= a.n_group) bv = kNegInf;
        wave_argmax(bv, bi);
        if (bi < 64) keep |= (uint64_t)1 << bi;
        if ((uint32_t)lane == bi) gs_lane = kNegInf;
      }
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const int64_t e = lane + 64 * j;
        if (e < a.E && !((keep >> (e / per)) & 1)) v[j] = 0.f;
      }
    }
  }

  // Top-k: lane r keeps the r-th pick.
  const int k = a.k;
  uint32_t my_idx = 0xffffffffu;
  float my_w = 0.f;
  for (int r = 0; r < k; ++r) {
    float bv = kNegInf;
    uint32_t bi = 0xffffffffu;
    float bw = 0.f;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
      const uint32_t e = (uint32_t)(lane + 64 * j);
      if (beats(v[j], e, bv, bi)) {
        bv = v[j];
        bi = e;
        bw = src[j];
      }
    }
    wave_argmax(bv, bi);
    // The winner's source value comes from the lane that owns it.
    const float w = __shfl(bw, (int)(bi & 63), 64);
#pragma unroll
    for (int j = 0; j < EPL; ++j)
      if ((uint32_t)(lane + 64 * j) == bi) v[j] = kNegInf;
    if (lane == r) {
      my_idx = bi;
      my_w = w;
    }
  }
  // GroupExpertSelect renormalizes only a selection of two or more
  // (deepseekv3.go:363); qwen3NextMoE renormalizes any selection
  // (qwen3next_forward.go:517-518).
  if (a.norm && (!GROUP || k > 1)) {
    const float s = wave_sum(lane < k ? my_w : 0.f);
    if (s != 0.f) my_w = my_w / s;
  }
  my_w *= a.scale;
  if (lane < k) {
    a.inds[row * k + lane] = my_idx;
    if constexpr (OUT_BF16)
      static_cast<uint16_t*>(a.weights)[row * k + lane] = (uint16_t)f32_to_bf16_rne(my_w);
    else
      static_cast<float*>(a.weights)[row * k + lane] = my_w;
  }
}

template <typename TIn, bool GROUP, bool OUT_BF16>
hipError_t launch_epl(const RouteArgs& a, hipStream_t stream) {
  const unsigned blocks = (unsigned)((a.T + 3) / 4);
  if (a.E <= 64) route_kernel<TIn, 1, GROUP, OUT_BF16><<<blocks, 256, 0, stream>>>(a);
  else if (a.E <= 128) route_kernel<TIn, 2, GROUP, OUT_BF16><<<blocks, 256, 0, stream>>>(a);
  else if (a.E <= 256) route_kernel<TIn, 4, GROUP, OUT_BF16><<<blocks, 256, 0, stream>>>(a);
  else if (a.E <= 512) route_kernel<TIn, 8, GROUP, OUT_BF16><<<blocks, 256, 0, stream>>>(a);
  else route_kernel<TIn, 16, GROUP, OUT_BF16><<<blocks, 256, 0, stream>>>(a);
  return hipGetLastError();
}

template <bool GROUP>
hipError_t launch_route_kind(const RouteArgs& a, hipStream_t stream) {
  if (a.in_bf16)
    return a.out_bf16 ? launch_epl<uint16_t, GROUP, true>(a, stream)
                      : launch_epl<uint16_t, GROUP, false>(a, stream);
  return a.out_bf16 ? launch_epl<float, GROUP, true>(a, stream)
                    : launch_epl<float, GROUP, false>(a, stream);
}

}  // namespace

hipError_t launch_route(const RouteArgs& a, bool group, hipStream_t stream) {
  if (a.T <= 0) return hipSuccess;
  if (a.E < 1 || a.E > kRouteMaxExperts || a.k < 1 || a.k > 64 || a.k > a.E)
    return hipErrorInvalidValue;
  if (group && (a.n_group < 1 || a.n_group > 64 || a.E % a.n_group != 0 || a.topk_group < 1))
    return hipErrorInvalidValue;
  return group ? launch_route_kind<true>(a, stream) : launch_route_kind<false>(a, stream);
}

}  // namespace fmxq
