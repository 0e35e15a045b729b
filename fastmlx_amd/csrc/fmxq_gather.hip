// fmxq_gather.hip -- grouped gather_qmm for expert-sorted slot batches.
//
// Replaces the sorted branch of mlx_gather_qmm (mlxgo/binding_cgo.go:645-673)
// as switchGLUCore calls it once routing fans out to 64 or more slots
// (compute/models/switch_glu.go:135-152, sorted=true): x rows gathered by
// order // top_k, rhs = expert ids in ascending order.
//
// A block owns 32 consecutive slots and 32 output columns.  It walks the runs of
// equal expert id among its slots (a wave ballot finds each run) and, per run,
// makes one MFMA pass over that expert's 32 weight rows with the run's gathered
// x rows as the A operand (the operand scheme of fmxq_mfma_frag.hpp, as in the
// skinny GEMV).  A run of length r costs one read of the expert's tile whatever
// r is, so a sorted batch reads each expert's weights about once per 32-slot
// tile instead of once per slot.  Output rows stay in slot order.  The K axis
// is split over the 4 waves of the block, which meet in LDS after every run.
// Results do not depend on the slot order inside a run: every output row is
// its own MFMA row with the same K order.
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"
#include "fmxq_mfma_frag.hpp"

namespace fmxq {

struct GStage {
  u32x4 w;
  uint32_t sb;
  u32x4 x[4];
};

template <int BITS>
__global__ __launch_bounds__(256) void gather_mfma_kernel(GatherArgs a) {
  constexpr int KS = 4;
  constexpr int U = BITS == 4 ? 64 : 32;
  constexpr float OFF = frag_offset<BITS>();
  constexpr float XSCALE = frag_xscale<BITS>();
  __shared__ float red[KS - 1][16][64];

  const int lane = threadIdx.x & 63, ks = threadIdx.x >> 6;
  const int ml = lane & 31, half = lane >> 5;
  const int64_t S = a.batch * a.Mx;
  const int64_t s0 = (int64_t)blockIdx.y * 32;
  const int64_t nb = (int64_t)blockIdx.x * 32;
  const int nslots = (int)((S - s0) < 32 ? (S - s0) : 32);
  const int64_t nu = a.K / U;
  const int64_t u0 = ks * nu / KS, u1 = (ks + 1) * nu / KS;
  const int gshift = __builtin_ctz((unsigned)a.group_size);  // a power of two
  const int64_t wpr = a.K * BITS / 32, gpr = a.K >> gshift;

  // Slot of this lane (lane halves mirror each other) and its x row / expert.
  const int64_t slot = s0 + (ml < nslots ? ml : 0);
  const int64_t item = slot / a.Mx, row = slot - item * a.Mx;
  const int64_t xi = a.lhs ? (int64_t)a.lhs[item] : item / a.lhs_div;
  uint32_t e = a.rhs[item];
  if ((int64_t)e >= a.E || xi >= a.x_batch) e = 0xffffffffu;  // out of range: zeros + flag
  const int64_t xoff = (xi < a.x_batch ? xi * a.Mx + row : 0) * a.K;
  int64_t n = nb + ml;
  n = n < a.N ? n : a.N - 1;

  const bf16x8 ones = as_bf16x8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
  int done = 0;
  while (done < nslots) {
    const uint32_t er = __builtin_amdgcn_readlane(e, done);
    // Lanes 0..31 whose slot continues the run starting at `done`.
    const uint64_t same = __ballot(half == 0 && ml >= done && ml < nslots && e == er);
    const uint64_t tail = ~(same >> done);
    const int len = (int)__builtin_ctzll(tail);
    const int end = done + len;
    const int64_t yr = a.yrow ? (int64_t)a.yrow[s0 + (ml < nslots ? ml : 0)] : s0 + ml;
    uint16_t* yslot = a.y + yr * a.N;
    if (er == 0xffffffffu) {
      if (ks == 0 && half == 0 && ml >= done && ml < end) {
        for (int c = 0; c < 32; ++c)
          if (nb + c < a.N) yslot[nb + c] = 0;
        atomicOr(a.err_flag, 1u);
      }
      done = end;
      continue;
    }
    // x row for A: lanes inside the run use their own slot, the others the run's first.
    const int64_t xo = __builtin_amdgcn_readlane((int)(xoff & 0xffffffff), done) |
                       ((int64_t)__builtin_amdgcn_readlane((int)(xoff >> 32), done) << 32);
    const bool in_run = ml >= done && ml < end;
    const uint16_t* xrow = a.x + (in_run ? xoff : xo) + half * (U / 2);
    const int64_t ebase = (int64_t)er * a.N;
    const uint32_t* wrow = a.w + (ebase + n) * wpr + half * 4;
    const uint16_t* srow = a.scales + (ebase + n) * gpr;
    const uint16_t* brow = a.biases + (ebase + n) * gpr;

    auto load = [&](GStage& st, int64_t u) {
      u = u < u1 ? u : u1 - 1;
      const int64_t g = (u * U + half * (U / 2)) >> gshift;
      st.w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + u * 8));
      st.sb = (uint32_t)srow[g] | ((uint32_t)brow[g] << 16);
      const u32x4* xs = reinterpret_cast<const u32x4*>(xrow + u * U);
      if constexpr (BITS == 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) st.x[j] = xs[j];
      } else {
        st.x[0] = xs[0];
        st.x[1] = xs[1];
      }
    };
    f32x16 acc = {};
    auto compute = [&](const GStage& st) {
      bf16x8 A[4];
      if constexpr (BITS == 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) A[j] = xfrag4(st.x[j]);
      } else {
        A[0] = xfrag8(st.x[0][0], st.x[0][1]);
        A[1] = xfrag8(st.x[0][2], st.x[0][3]);
        A[2] = xfrag8(st.x[1][0], st.x[1][1]);
        A[3] = xfrag8(st.x[1][2], st.x[1][3]);
      }
      f32x16 xs = {}, P = {};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xs = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[j], ones, xs, 0, 0, 0);
        P = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[j], wfrag<BITS>(st.w[j]), P, 0, 0, 0);
      }
      const float s = bf16_lo(st.sb);
      const float bo = __builtin_fmaf(-OFF, s, bf16_hi(st.sb)) * XSCALE;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = __builtin_fmaf(s, P[r], __builtin_fmaf(bo, xs[r], acc[r]));
    };
    if (u1 > u0) {
      GStage st0, st1;
      load(st0, u0);
      load(st1, u0 + 1);
      for (int64_t u = u0; u < u1; u += 2) {
        compute(st0);
        load(st0, u + 2);
        if (u + 1 < u1) compute(st1);
        load(st1, u + 3);
      }
    }
    if (ks > 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) red[ks - 1][r][lane] = acc[r];
    }
    __syncthreads();
    if (ks == 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float v = acc[r] + red[0][r][lane] + red[1][r][lane] + red[2][r][lane];
        // C layout: register r of lane l is row 8*(r/4) + 4*(l/32) + r%4, column l%32.
        const int m = (r / 4) * 8 + half * 4 + (r % 4);
        if (m >= done && m < end && nb + ml < a.N) {
          const int64_t orow = a.yrow ? (int64_t)a.yrow[s0 + m] : s0 + m;
          a.y[orow * a.N + nb + ml] = finish_out(v, nullptr, 0);
        }
      }
    }
    __syncthreads();
    done = end;
  }
}

bool gather_mfma_supported(const GatherArgs& a) {
  if (a.bits == 4) return a.group_size >= 64 && a.K % 64 == 0;
  return a.group_size >= 32 && a.K % 32 == 0;
}

hipError_t launch_gather_mfma(const GatherArgs& a, hipStream_t stream) {
  const int64_t S = a.batch * a.Mx;
  if (S <= 0 || a.N <= 0) return hipSuccess;
  dim3 grid((unsigned)((a.N + 31) / 32), (unsigned)((S + 31) / 32));
  if (a.bits == 4)
    gather_mfma_kernel<4><<<grid, 256, 0, stream>>>(a);
  else
    gather_mfma_kernel<8><<<grid, 256, 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace fmxq
