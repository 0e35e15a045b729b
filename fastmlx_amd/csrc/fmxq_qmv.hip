// fmxq_qmv.hip -- decode GEMV (M <= 8) for quantized_matmul and the per-slot
// gathered GEMV of gather_qmm.
//
// Replaces the decode side of mlx_quantized_matmul (mlxgo/binding_cgo.go:636-643,
// reached from compute/models/quant.go:91-101 on every decode step) and the
// short-routing gather of mlx_gather_qmm (switch_glu.go:124-130 -> :179-186).
//
// qmvx_kernel (below) is the main decode kernel: x rows live in registers and a
// wave walks several weight rows.  qmv_kernel is the general M <= 4 fallback for
// rows too long to keep x in registers: a block is 4 waves, the K axis is split
// into KS slices so that every wave owns at most CPL 16-byte chunks per row, and
// every weight load of a wave is issued before any arithmetic.  The arithmetic
// per chunk is chunk_dot() (fmxq_qmv_impl.hpp): bf16(128+q) operands from the
// exponent trick against x pairs, v_dot2_f32_bf16.
#include "fmxq_internal.hpp"
#include "fmxq_qmv_impl.hpp"

namespace fmxq {

template <int CTRL, int RMASK>
__device__ __forceinline__ float dpp_add(float a) {
  const int b = __builtin_amdgcn_update_dpp(0, __float_as_int(a), CTRL, RMASK, 0xf, false);
  return a + __int_as_float(b);
}

// Sum over the 64 lanes; the result is returned in every lane.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = dpp_add<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
  v = dpp_add<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
  v = dpp_add<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_add<0x140, 0xf>(v);  // row_mirror
  v = dpp_add<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
  v = dpp_add<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// ---------------------------------------------------------------------------
// Decode GEMV for M <= 8 with x held in registers.
//
// A block is WAVES (4 or 8) waves: WAVES/KS row groups x KS slices of the K
// axis.  Lane l of the wave for slice ks owns 16-byte chunks c0 + l + 64 i
// (i < CPL) of every row the
// wave visits, so it builds the x pairs and x sums of those chunks (for each of
// the MM rows of x) once and keeps them in registers while the wave walks RPW
// weight rows, R rows at a time, with the next R rows' weights already in flight
// (two register buffers, indices fixed at compile time).  A wave's weight load is
// 1 KiB contiguous per row.  Each packed word is unpacked once (exponent trick, 7
// VALU) and dotted against every x row (4 v_dot2 each); a 3-op group correction
// per chunk and row follows.  The RPW x MM partial sums are reduced together at
// the end (wave_sum_multi).  MM is M padded to a power of two; only the first MX
// x rows are built and dotted (MX = M for M = 5..7: M = 5 on 1024x4096 took 5.5
// us with all 8 rows, 4.6 us with 5), the padding rows' partials being zero.
template <int BITS, int MM, int CPL, int R, int RPW, int KS, int WAVES = 4, int MX = MM>
__global__ __launch_bounds__(WAVES * 64) void qmvx_kernel(QmmArgs a) {
  constexpr int CH = 128 / BITS;  // values per 16-byte chunk
  constexpr int RG = WAVES / KS;
  constexpr int V = RPW * MM;     // partial sums per lane
  constexpr int LV = __builtin_ctz(V);
  static_assert(RPW % R == 0, "rows per wave must be a multiple of R");
  static_assert((V & (V - 1)) == 0 && V <= 64, "RPW * MM must be a power of two <= 64");
  __shared__ float part[KS > 1 ? RG : 1][KS][V];
  // The wave index is uniform; readfirstlane lets row and slice math run on SALU.
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rg = wave / KS, ks = wave % KS;
  const int nch = (int)(a.K / CH);
  const int c0 = ks * nch / KS, c1 = (ks + 1) * nch / KS;
  const int gshift = __builtin_ctz((unsigned)a.group_size);
  const int chunk_gshift = gshift - __builtin_ctz((unsigned)CH);  // chunk -> group
  const int64_t wpr = a.K * BITS / 32, gpr = a.K >> gshift;
  const int64_t nbase = ((int64_t)blockIdx.x * RG + rg) * RPW;

  bool live[CPL];
  int cc[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = c0 + lane + 64 * i;
    live[i] = c < c1;
    cc[i] = live[i] ? c : c0;
  }

  XChunk<BITS> xc[MX][CPL];
  u32x4 wv0[R][CPL], wv1[R][CPL];
  // Scale and bias bits stay in separate registers until the arithmetic: packing
  // them at load time would make the compiler wait for each load right away.
  uint32_t sb0[R][CPL][2], sb1[R][CPL][2];
  auto load = [&](u32x4 (&wv)[R][CPL], uint32_t (&sb)[R][CPL][2], int rb) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int64_t n = nbase + rb + r;
      n = n < a.N ? n : a.N - 1;
      const u32x4* wr = reinterpret_cast<const u32x4*>(a.w + n * wpr);
      const uint16_t* sr = a.scales + n * gpr;
      const uint16_t* br = a.biases + n * gpr;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        wv[r][i] = __builtin_nontemporal_load(wr + cc[i]);
        const int g = cc[i] >> chunk_gshift;
        sb[r][i][0] = sr[g];
        sb[r][i][1] = br[g];
      }
    }
  };
  float res[V];  // res[r * MM + m]: this lane's partial for weight row r, x row m
  auto compute = [&](const u32x4 (&wv)[R][CPL], const uint32_t (&sb)[R][CPL][2], int rb) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float acc[MM];
#pragma unroll
      for (int m = 0; m < MM; ++m) acc[m] = 0.f;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const float s = bf16_bits_to_f32(sb[r][i][0]);
        const float bo = __builtin_fmaf(-magic_offset<BITS>(), s, bf16_bits_to_f32(sb[r][i][1]));
        if constexpr (MM == 1) {
          const float t = __builtin_fmaf(s, chunk_dot<BITS>(wv[r][i], xc[0][i]), bo * xc[0][i].sum);
          acc[0] += live[i] ? t : 0.f;
        } else {
          uint32_t p[16];
          unpack_chunk(wv[r][i], p);
#pragma unroll
          for (int m = 0; m < MX; ++m) {
            const float t = __builtin_fmaf(s, dot_pairs<BITS>(p, xc[m][i]), bo * xc[m][i].sum);
            acc[m] += live[i] ? t : 0.f;
          }
        }
      }
#pragma unroll
      for (int m = 0; m < MM; ++m) res[(rb + r) * MM + m] = acc[m];
    }
  };
  // With several x rows, sched_barrier(0) pins each prefetch ahead of the compute
  // that follows it: left alone, the scheduler sinks later rows' loads below the
  // (long) multi-row math to save registers, which serialises memory latency.
  auto pin = [] {
    if constexpr (MM > 1) __builtin_amdgcn_sched_barrier(0);
  };
  // The first weight rows are requested before x is built (x is an L2 hit for
  // all but the first waves; the weights are not).  Rows of x beyond M repeat
  // row M-1; their outputs are never stored.
  load(wv0, sb0, 0);
  // Keep all of the first group's weight loads ahead of x; left alone the
  // scheduler issues the x loads first and holds back the last weight rows to
  // reuse x's registers.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int m = 0; m < MX; ++m) {
    const uint16_t* xr = a.x + (int64_t)(m < a.M ? m : a.M - 1) * a.ldx;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      xc[m][i].load(xr, (int64_t)cc[i] * CH);
      if (!live[i]) xc[m][i].sum = 0.f;
    }
  }
  pin();
#pragma unroll
  for (int rb = 0; rb < RPW; rb += 2 * R) {
    if (rb + R < RPW) load(wv1, sb1, rb + R);
    pin();
    compute(wv0, sb0, rb);
    if (rb + R < RPW) {
      if (rb + 2 * R < RPW) load(wv0, sb0, rb + 2 * R);
      pin();
      compute(wv1, sb1, rb + R);
    }
  }

  // Lane l now holds the total of partial index l >> (6 - LV); the first lane of
  // each run of 64 / V lanes writes it.
  const float tot = wave_sum_multi<V>(res, lane);
  const int idx = lane >> (6 - LV);
  const bool writer = (lane & ((64 >> LV) - 1)) == 0;
  const int rr = idx / MM, mr = idx % MM;
  const int64_t n = nbase + rr;
  if constexpr (KS > 1) {
    if (writer) part[rg][ks][idx] = tot;
    __syncthreads();
    if (ks == 0 && writer) {
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < KS; ++k) v += part[rg][k][idx];
      if (n < a.N && mr < a.M) a.y[(int64_t)mr * a.ldy + n] = finish_out(v, a.bias, n);
    }
  } else {
    if (writer && n < a.N && mr < a.M) a.y[(int64_t)mr * a.ldy + n] = finish_out(tot, a.bias, n);
  }
}

// ---------------------------------------------------------------------------
// Decode GEMV for exactly one row of x, the shape of every decode step.
//
// Same work split as qmvx_kernel with one 16-byte chunk per lane (CPL) and a
// wave walking RPW weight rows in groups of R with P groups in flight: every
// load of the first P groups is issued before x is read, the next group's loads
// are issued as each group's arithmetic finishes.  Scale and bias bits are
// packed into one register per (row, chunk).
template <int BITS, int CPL, int R, int RPW, int KS, int WAVES, int P>
__global__ __launch_bounds__(WAVES * 64) void qmv1_kernel(QmmArgs a) {
  constexpr int CH = 128 / BITS;
  constexpr int RG = WAVES / KS;
  constexpr int V = RPW;
  constexpr int LV = __builtin_ctz(V);
  constexpr int G = RPW / R;  // row groups per wave
  static_assert(RPW % R == 0 && P >= 1 && P <= G, "row groups");
  static_assert((V & (V - 1)) == 0 && V <= 64, "RPW must be a power of two <= 64");
  __shared__ float part[KS > 1 ? RG : 1][KS][V];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rg = wave / KS, ks = wave % KS;
  const int nch = (int)(a.K / CH);
  const int c0 = ks * nch / KS, c1 = (ks + 1) * nch / KS;
  const int gshift = __builtin_ctz((unsigned)a.group_size);
  const int chunk_gshift = gshift - __builtin_ctz((unsigned)CH);
  const int64_t wpr = a.K * BITS / 32, gpr = a.K >> gshift;
  const int64_t nbase = ((int64_t)blockIdx.x * RG + rg) * RPW;

  bool live[CPL];
  int cc[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = c0 + lane + 64 * i;
    live[i] = c < c1;
    cc[i] = live[i] ? c : c0;
  }
  u32x4 wv[P][R][CPL];
  uint32_t sb[P][R][CPL];
  auto load = [&](int slot, int rb) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      int64_t n = nbase + rb + r;
      n = n < a.N ? n : a.N - 1;  // rows past N load row N-1; their outputs are not stored
      const u32x4* wr = reinterpret_cast<const u32x4*>(a.w + n * wpr);
      const uint16_t* sr = a.scales + n * gpr;
      const uint16_t* br = a.biases + n * gpr;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        wv[slot][r][i] = __builtin_nontemporal_load(wr + cc[i]);
        const int g = cc[i] >> chunk_gshift;
        sb[slot][r][i] = (uint32_t)sr[g] | ((uint32_t)br[g] << 16);
      }
    }
  };
#pragma unroll
  for (int g = 0; g < P; ++g) load(g, g * R);
  XChunk<BITS> xc[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    xc[i].load(a.x, (int64_t)cc[i] * CH);
    if (!live[i]) xc[i].sum = 0.f;
  }
  float res[V];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int slot = g % P;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const float s = bf16_lo(sb[slot][r][i]);
        const float bo = __builtin_fmaf(-magic_offset<BITS>(), s, bf16_hi(sb[slot][r][i]));
        const float t = __builtin_fmaf(s, chunk_dot<BITS>(wv[slot][r][i], xc[i]), bo * xc[i].sum);
        acc += live[i] ? t : 0.f;
      }
      res[g * R + r] = acc;
    }
    if (g + P < G) load(slot, (g + P) * R);
  }
  // Lane l holds the total of row l >> (6 - LV); the first lane of each run writes.
  const float tot = wave_sum_multi<V>(res, lane);
  const int idx = lane >> (6 - LV);
  const bool writer = (lane & ((64 >> LV) - 1)) == 0;
  const int64_t n = nbase + idx;
  if constexpr (KS > 1) {
    if (writer) part[rg][ks][idx] = tot;
    __syncthreads();
    if (ks == 0 && writer) {
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < KS; ++k) v += part[rg][k][idx];
      if (n < a.N) a.y[n] = finish_out(v, a.bias, n);
    }
  } else {
    if (writer && n < a.N) a.y[n] = finish_out(tot, a.bias, n);
  }
}

template <int BITS, int CPL, int R, int RPW, int KS, int WAVES, int P>
static hipError_t launch_qmv1_cfg(const QmmArgs& a, hipStream_t stream) {
  constexpr int64_t rows_per_block = (WAVES / KS) * RPW;
  const unsigned blocks = (unsigned)((a.N + rows_per_block - 1) / rows_per_block);
  qmv1_kernel<BITS, CPL, R, RPW, KS, WAVES, P><<<blocks, WAVES * 64, 0, stream>>>(a);
  return hipGetLastError();
}

// Shapes measured on the Llama-3-8B projections (graphs of launches over
// distinct weight copies): 4-bit rows of 65..128 chunks (K = 4096) and of
// 257..512 chunks (K = 14336).  Returns hipErrorNotSupported for other shapes.
static hipError_t launch_qmv1(const QmmArgs& a, hipStream_t stream) {
  if (a.M != 1 || a.bits != 4 || a.ldx % 8 != 0) return hipErrorNotSupported;
  const int64_t nch = a.K / 32;
  if (nch > 64 && nch <= 128) {
    if (a.N >= 8192) return launch_qmv1_cfg<4, 1, 4, 4, 2, 4, 1>(a, stream);
    return launch_qmv1_cfg<4, 1, 2, 2, 2, 4, 1>(a, stream);
  }
  if (nch > 256 && nch <= 512) return launch_qmv1_cfg<4, 1, 4, 4, 8, 8, 1>(a, stream);
  return hipErrorNotSupported;
}

// ---------------------------------------------------------------------------
// Decode GEMV for one x row, int4 group 64, K a multiple of 2048: a wave owns a
// 64-chunk (2048-value) K slice of RW rows, lane l chunk l of the slice.  All RW
// weight loads of a wave are in flight at once, and the lane's x chunk serves all
// RW rows.  Loads are issued x, scales and biases, then weights, so the x pairs
// and the scale/bias table are built while the weights are on their way:
//   - with two slices (4096-deep rows) the scales (and the biases) of the block's
//     RG * RW rows are one contiguous run of the array: thread t loads its
//     16-byte piece t of each, so the run reaches memory as whole coalesced lines
//     rather than as each wave's 64-byte slice of every row (4096 x 4096: 3.97 ->
//     3.87 us, 1024 x 4096: 2.71 -> 2.65 us); the pieces are interleaved into
//     (scale | bias << 16) words in a block LDS table [rows][K / 64], from which
//     lane l of slice ks reads group 32 ks + l / 2 of each row after one barrier;
//   - longer rows keep per-wave pieces (lane L -> row L / 4, groups 8 (L % 4) ..
//     +7 of the slice) in a wave-private table [RW][32], no barrier;
//   - a block is RG row groups x KS slices; the slices meet in LDS.
// Arithmetic as in qmv1_kernel.
//
// With FMXQ_QMV1_TIMELINE (the diagnostic build of fastmlx_amd/diag only; the
// library compiles none of it) each wave reads the 100 MHz s_memrealtime clock at
// its start, once its weight loads are issued, after its first row's arithmetic
// (so after its first weight bytes arrived), after its last row's, and at its end,
// and lane 0 stores the five stamps and the wave's XCC and hardware ids to
// a.tl_stamps[6 * wave] with vector stores.
#ifdef FMXQ_QMV1_TIMELINE
#define FMXQ_TL_STAMP(v) v = __builtin_amdgcn_s_memrealtime()
#define FMXQ_TL_AFTER(v, r) asm volatile("" ::"v"(r))
#else
#define FMXQ_TL_STAMP(v) (void)0
#define FMXQ_TL_AFTER(v, r) (void)0
#endif
// The kernel body for block bx of the product a (bx is blockIdx.x, or the block's
// index within its matrix in the grouped launch below).
template <int RW, int KS, int RG>
__device__ __forceinline__ void qmv1_slice_body(const QmmArgs& a, int64_t bx) {
#ifdef FMXQ_QMV1_TIMELINE
  uint64_t tl[5] = {};
#endif
  FMXQ_TL_STAMP(tl[0]);
  constexpr int LV = __builtin_ctz(RW);
  // Two-slice (4096-deep) rows load the block's scales as contiguous runs into a
  // shared table; longer rows keep each wave's own pieces (measured no faster as
  // runs on 4096 x 14336).
  constexpr bool BS = KS <= 2;
  constexpr int PPR = KS * 4;             // 16-byte scale pieces per row (K / 512)
  constexpr int NPC = RG * RW * PPR;      // pieces of the block's rows
  constexpr int NP = (RW * 4 + 63) / 64;  // per-wave form: piece loads per lane
  static_assert(!BS || NPC <= KS * RG * 64, "one piece per thread");
  __shared__ float part[RG][KS][RW];
  __shared__ __attribute__((aligned(16))) uint32_t sbt[BS ? RG * RW : KS * RG][BS ? KS * 32 : RW * 32];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rg = wave / KS, ks = wave % KS;
  const int c = ks * 64 + lane;
  const int64_t wpr = a.K / 8, gpr = a.K / 64;
  const int64_t nbase = (bx * RG + rg) * RW;
  // Row indices in 32 bits (launch_qmv1_slice keeps N below 2^31), wave-uniform
  // for the weight rows: the clamp and the row offsets then stay on the scalar
  // unit (gfx9 has no 64-bit signed scalar compare, so an int64 clamp would move
  // every row address to 64-bit vector arithmetic).
  const int nb32 = __builtin_amdgcn_readfirstlane((int)nbase);
  const int nlast = (int)a.N - 1;
  u32x4 xr[4];
  {
    const u32x4* xs = reinterpret_cast<const u32x4*>(a.x + (int64_t)c * 32);
#pragma unroll
    for (int j = 0; j < 4; ++j) xr[j] = xs[j];
  }
  // Block form: the scales and biases of the block's rows are one contiguous run
  // of each array, thread t loading 16-byte piece t of both.  Per-wave form: lane
  // L loads piece L % 4 of the wave's slice of row L / 4.  Rows past N re-read
  // row N - 1.
  const int tid = threadIdx.x;
  const int prow = BS ? tid / PPR : 0, ppc = BS ? tid % PPR : 0;
  u32x4 ps[NP], pb[NP];
  if constexpr (BS) {
    if (tid < NPC) {
      const int n =
          min(__builtin_amdgcn_readfirstlane((int)(bx * RG * RW)) + prow, nlast);
      const int64_t off = (int64_t)n * gpr + ppc * 8;
      ps[0] = *reinterpret_cast<const u32x4*>(a.scales + off);
      pb[0] = *reinterpret_cast<const u32x4*>(a.biases + off);
    }
  } else {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int L = lane + 64 * p;
      const int r = L >> 2, pc = L & 3;
      if (r < RW) {
        const int n = min(nb32 + r, nlast);
        const int64_t off = (int64_t)n * gpr + ks * 32 + pc * 8;
        ps[p] = *reinterpret_cast<const u32x4*>(a.scales + off);
        pb[p] = *reinterpret_cast<const u32x4*>(a.biases + off);
      }
    }
  }
  // Keep the weight loads behind x and the pieces: the wait for those then does
  // not hold on the weights.
  __builtin_amdgcn_sched_barrier(0);
  u32x4 wv[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    // rows past N load row N-1; their outputs are not stored
    const int n = __builtin_amdgcn_readfirstlane(min(nb32 + r, nlast));
    wv[r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.w + (int64_t)n * wpr) + c);
  }
  __builtin_amdgcn_sched_barrier(0);
  FMXQ_TL_STAMP(tl[1]);
  XChunk<4> xc;
  {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x_pairs_q4(xr[j], xc.p + 4 * j);
      s = dot2_bf16(xr[j][0], kOnes, s);
      s = dot2_bf16(xr[j][1], kOnes, s);
      s = dot2_bf16(xr[j][2], kOnes, s);
      s = dot2_bf16(xr[j][3], kOnes, s);
    }
    xc.sum = s;
  }
  // (scale | bias << 16) words: the block's table (after one barrier), or the
  // wave's own [RW][32] table, written and read by that wave only (LDS operations
  // of one wave complete in order, so no barrier).
  auto interleave = [&](int p, uint32_t* dst) {
    u32x4 o0, o1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      o0[2 * h] = __builtin_amdgcn_perm(pb[p][h], ps[p][h], 0x05040100u);
      o0[2 * h + 1] = __builtin_amdgcn_perm(pb[p][h], ps[p][h], 0x07060302u);
      o1[2 * h] = __builtin_amdgcn_perm(pb[p][2 + h], ps[p][2 + h], 0x05040100u);
      o1[2 * h + 1] = __builtin_amdgcn_perm(pb[p][2 + h], ps[p][2 + h], 0x07060302u);
    }
    *reinterpret_cast<u32x4*>(dst) = o0;
    *reinterpret_cast<u32x4*>(dst + 4) = o1;
  };
  if constexpr (BS) {
    if (tid < NPC) interleave(0, &sbt[prow][ppc * 8]);
    __syncthreads();
  } else {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int L = lane + 64 * p;
      const int r = L >> 2, pc = L & 3;
      if (r < RW) interleave(p, &sbt[wave][r * 32 + pc * 8]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  float res[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const uint32_t sb = BS ? sbt[rg * RW + r][ks * 32 + (lane >> 1)] : sbt[wave][r * 32 + (lane >> 1)];
    const float s = bf16_lo(sb);
    const float bo = __builtin_fmaf(-magic_offset<4>(), s, bf16_hi(sb));
    res[r] = __builtin_fmaf(s, chunk_dot<4>(wv[r], xc), bo * xc.sum);
    if (r == 0) {
      FMXQ_TL_AFTER(tl[2], res[0]);
      FMXQ_TL_STAMP(tl[2]);
    }
  }
  FMXQ_TL_AFTER(tl[3], res[RW - 1]);
  FMXQ_TL_STAMP(tl[3]);
  const float tot = wave_sum_multi<RW>(res, lane);
  const int idx = lane >> (6 - LV);
  const bool writer = (lane & ((64 >> LV) - 1)) == 0;
  const int64_t n = nbase + idx;
  if constexpr (KS > 1) {
    if (writer) part[rg][ks][idx] = tot;
    __syncthreads();
    if (ks == 0 && writer) {
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < KS; ++k) v += part[rg][k][idx];
      if (n < a.N) a.y[n] = finish_out(v, a.bias, n);
    }
  } else {
    if (writer && n < a.N) a.y[n] = finish_out(tot, a.bias, n);
  }
#ifdef FMXQ_QMV1_TIMELINE
  FMXQ_TL_STAMP(tl[4]);
  if (a.tl_stamps && lane == 0) {
    const uint32_t hw = __builtin_amdgcn_s_getreg((4 << 0) | (0 << 6) | (31 << 11));   // HW_ID
    const uint32_t xcc = __builtin_amdgcn_s_getreg((20 << 0) | (0 << 6) | (3 << 11));  // XCC_ID
    uint64_t* o = a.tl_stamps + 6 * (bx * (KS * RG) + wave);
#pragma unroll
    for (int i = 0; i < 5; ++i) o[i] = tl[i];
    o[5] = ((uint64_t)xcc << 32) | hw;
  }
#endif
}

template <int RW, int KS, int RG>
__global__ __launch_bounds__(KS * RG * 64) void qmv1_slice_kernel(QmmArgs a) {
  qmv1_slice_body<RW, KS, RG>(a, blockIdx.x);
}

// Several products of one x row in one launch (fmxq_quantized_matmul_group): block
// b belongs to matrix i when first[i] <= b < first[i + 1], and runs that matrix's
// block b - first[i].  The matrix index is uniform over the block.
struct SliceGroup {
  QmmArgs m[kSliceGroupMax];
  int64_t first[kSliceGroupMax + 1];
  int n;
};
template <int RW, int KS, int RG>
__global__ __launch_bounds__(KS * RG * 64) void qmv1_slice_group_kernel(SliceGroup g) {
  const int64_t b = blockIdx.x;
  int i = 0;
#pragma unroll
  for (int j = 1; j < kSliceGroupMax; ++j)
    if (j < g.n && b >= g.first[j]) i = j;
  i = __builtin_amdgcn_readfirstlane(i);
  qmv1_slice_body<RW, KS, RG>(g.m[i], b - g.first[i]);
}

template <int RW, int KS, int RG>
static hipError_t launch_qmv1_slice_cfg(const QmmArgs& a, hipStream_t stream) {
  constexpr int64_t rows = RW * RG;
  qmv1_slice_kernel<RW, KS, RG><<<(unsigned)((a.N + rows - 1) / rows), KS * RG * 64, 0, stream>>>(a);
  return hipGetLastError();
}

// Shapes where the slice kernel beats qmv1_kernel or the qmvx GEMV (graphs of
// launches over distinct weight copies): 2048-deep rows (below), 14336-deep rows (8.2 -> 7.7 us for 4096 x 14336) and
// K = 4096 at every height (4.2 -> 3.9 us for 4096 x 4096; 8.1 -> 7.8 us for
// 14336 x 4096 once the scales load as block runs; 28672 x 4096 12.4-12.8 ->
// 12.1 us; the 128256 x 4096 tied head 47.7-48.4 -> 43.7-44.4 us, 85% of HBM).
// The slice kernel's shape for rows of depth K and N outputs: launch(RW, KS, RG)
// with the three as integral constants, or hipErrorNotSupported.
template <class L>
static hipError_t with_slice_shape(int64_t K, int64_t N, L&& launch) {
  using std::integral_constant;
  auto go = [&](auto rw, auto ks, auto rg) { return launch(rw, ks, rg); };
  switch (K / 2048) {
    // One slice (2048-deep rows): 2 rows per wave, 4 waves per block, no cross-slice
    // sum (against the qmvx GEMV: 2048 x 2048 2.89 -> 2.60 us, 512 x 2048 2.54 ->
    // 2.25 us, 8192 x 2048 4.20 -> 4.07 us; 1 or 4 rows per wave, or 2 waves per
    // block, measured in between).
    case 1: return go(integral_constant<int, 2>{}, integral_constant<int, 1>{}, integral_constant<int, 4>{});
    case 4: return go(integral_constant<int, 8>{}, integral_constant<int, 4>{}, integral_constant<int, 1>{});
    case 5: return go(integral_constant<int, 8>{}, integral_constant<int, 5>{}, integral_constant<int, 1>{});
    case 6: return go(integral_constant<int, 8>{}, integral_constant<int, 6>{}, integral_constant<int, 1>{});
    // 14336-deep rows: 16 rows per wave, one 7-slice block per 16 rows, up to 16384
    // outputs (4096 x 14336 7.89-8.01 -> 7.64-7.68 us, 16384 x 14336 23.1-23.7 ->
    // 22.3-22.6 us; 4 rows 8.0-8.1, 4 rows in two row groups 9.1-9.2 us); 8 rows
    // on taller matrices (32768 x 14336: 41.8-41.9 against 42.9-43.2 us).
    case 7:
      if (N > 16384)
        return go(integral_constant<int, 8>{}, integral_constant<int, 7>{}, integral_constant<int, 1>{});
      return go(integral_constant<int, 16>{}, integral_constant<int, 7>{}, integral_constant<int, 1>{});
    case 8: return go(integral_constant<int, 8>{}, integral_constant<int, 8>{}, integral_constant<int, 1>{});
    case 2:
      // 4 rows per wave from 8192 to 32767 outputs (14336 x 4096 7.64-7.98 ->
      // 7.45-7.49 us, the C1 stack at M = 1 1.178 -> 1.165 ms); 8 below and above
      // (4096 x 4096 3.80 against 4.01 us, the 128256-row head 44.0-44.4 against
      // 45.1 us).
      if (N >= 8192 && N < 32768)
        return go(integral_constant<int, 4>{}, integral_constant<int, 2>{}, integral_constant<int, 2>{});
      if (N >= 2048)
        return go(integral_constant<int, 8>{}, integral_constant<int, 2>{}, integral_constant<int, 2>{});
      return go(integral_constant<int, 2>{}, integral_constant<int, 2>{}, integral_constant<int, 2>{});
    default: return hipErrorNotSupported;
  }
}

static bool slice_supported(const QmmArgs& a) {
  return a.M == 1 && a.bits == 4 && a.group_size == 64 && a.K % 2048 == 0 &&
         a.N < (int64_t(1) << 31) && !(reinterpret_cast<uintptr_t>(a.scales) & 15u) &&
         !(reinterpret_cast<uintptr_t>(a.biases) & 15u) && !(reinterpret_cast<uintptr_t>(a.x) & 15u) &&
         !(reinterpret_cast<uintptr_t>(a.w) & 15u);
}

static hipError_t launch_qmv1_slice(const QmmArgs& a, hipStream_t stream) {
  if (!slice_supported(a)) return hipErrorNotSupported;
  return with_slice_shape(a.K, a.N, [&](auto rw, auto ks, auto rg) {
    return launch_qmv1_slice_cfg<decltype(rw)::value, decltype(ks)::value, decltype(rg)::value>(
        a, stream);
  });
}

struct QmvxShape {
  int ks, cpl, rpw, waves;
  int r = 2;  // rows per load group (all rpw rows at once when r == rpw)
};
// The fewest K slices (1, 2 or 4) that keep a lane at <= 2 chunks per row (x in
// registers grows with MM), and more rows per wave for the longest rows, where
// building x costs the most.  cpl 0 means the shape is not handled here.
static QmvxShape pick_qmvx_shape(int64_t nch, int64_t N, int mm, int bits, int64_t m) {
  QmvxShape sh{4, (int)((nch + 255) / 256), 4, 4};
  if (nch <= 64) sh = {1, 1, 4, 4};
  else if (nch <= 128) sh = {2, 1, 4, 4};
  else if (nch <= 256) sh = {4, 1, 4, 4};
  if (nch > 256 && sh.cpl <= 2) sh.rpw = 8;
  if (N <= 2048) sh.rpw = 2;
  // Register budget: MM x CPL x-chunks of 17 VGPRs each.
  const int max_cpl = mm == 1 ? 4 : mm == 2 ? 4 : mm == 4 ? 2 : 1;
  if (sh.cpl > max_cpl) sh.cpl = 0;
  if (sh.rpw * mm > 64) sh.rpw = 64 / mm;
  if (mm == 8 && sh.rpw > 4) sh.rpw = 4;
  // Eight rows of x and long rows: eight K slices (8-wave blocks) keep one chunk
  // per lane.
  if (mm == 8 && nch > 256 && nch <= 512) {
    sh.ks = 8;
    sh.cpl = 1;
    sh.waves = 8;
  }
  // Four x rows, int4 rows of 2049-4096 values, outputs past 2048 rows: 8 rows per
  // wave (M = 4: 14336x4096 15.5 -> 15.1 us, 4096x4096 6.64 -> 6.27 us,
  // 28672x4096 26.8 -> 23.3 us; M = 3 on 14336x4096 14.9 -> 14.5 us).
  if (mm == 4 && bits == 4 && nch > 64 && nch <= 128 && N > 2048) sh.rpw = 8;
  // Two x rows on the same rows, outputs past 4096 rows: 8 rows per wave as well
  // (14336x4096 10.6 -> 10.4 us, 28672x4096 17.3 -> 15.5 us; 4096x4096 lost, 5.04
  // -> 5.2 us, and 4 rows per wave below 2048 outputs at M = 3, 4 lost: 4.0 ->
  // 4.5 us on 1024x4096).
  if (mm == 2 && bits == 4 && nch > 64 && nch <= 128 && N > 4096) sh.rpw = 8;
  // int8, two or four x rows, rows of 2049-4096 values, outputs past 2048 rows: 8
  // rows per wave (M = 2, 14336x4096: 15.6 -> 15.2 us; M = 4: 21.0 -> 20.5 us,
  // 4096x4096 8.37 -> 8.0 us; at M = 1 it did not help, 4096x4096 5.38 -> 5.51 us;
  // eight K slices there lost 40-70%).
  if (bits == 8 && (mm == 2 || mm == 4) && nch > 128 && nch <= 256 && N > 2048) sh.rpw = 8;
  // Two x rows, int4 rows of 8193-16384 values: eight slices of one chunk per
  // lane (4096x14336: 11.1 -> 10.7 us, 14336x14336: 30.3 -> 28.0 us; at four x
  // rows it lost: 4096x14336 15.0 -> 17.0 us).
  if (mm == 2 && bits == 4 && nch > 256 && nch <= 512) {
    sh.ks = 8;
    sh.cpl = 1;
    sh.waves = 8;
  }
  // Three or four x rows on int4 rows of 8193-16384 values with at most 2048
  // outputs: 4 rows per wave rather than 2 (1024x14336 8.4 -> 6.7 us; with 4096
  // outputs 4 rather than 8 lost, 15.2 -> 18.2 us, and so did 4 at two x rows).
  if (mm == 4 && bits == 4 && nch > 256 && nch <= 512 && N <= 2048) sh.rpw = 4;
  // int8 rows up to 16384 values (twice the chunks of int4 at the same K) at
  // M = 1 to 5: eight slices of at most two 9-register x chunks per lane and x
  // row (M = 1, 4096x14336: 20.2 -> 15.9 us; M = 2: 22.8 -> 21.0 us, 14336x14336
  // 73.2 -> 67.5 us; M = 5, 4096x14336: 36.2 -> 33.4 us against the prefill tile, 1024x16384:
  // 23.7 -> 13.0 us; at M = 6, 7, 8 the tile stays faster: 35.1 / 36.3 / 36.6
  // against 36.9 / 40.5 / 48.2 us.  M = 4 against the general GEMV: 4096x14336
  // 35.5 -> 29.4 us, 14336x14336 108.3 -> 97.2 us; M = 3 30.0 -> 29.5 us).
  if (bits == 8 && (mm <= 4 || (mm == 8 && m <= 5)) && nch > 512 && nch <= 1024) {
    sh.ks = 8;
    sh.cpl = 2;
    sh.waves = 8;
  }
  return sh;
}

template <int BITS, int MM, int CPL, int RPW, int KS, int WAVES, int R = 2, int MX = MM>
static hipError_t launch_qmvx_cfg(const QmmArgs& a, hipStream_t stream) {
  constexpr int64_t rows_per_block = (WAVES / KS) * RPW;
  const unsigned blocks = (unsigned)((a.N + rows_per_block - 1) / rows_per_block);
  qmvx_kernel<BITS, MM, CPL, R, RPW, KS, WAVES, MX><<<blocks, WAVES * 64, 0, stream>>>(a);
  return hipGetLastError();
}

template <int BITS, int MM, int CPL, int KS, int WAVES = 4, int MX = MM>
static hipError_t launch_qmvx_rpw(const QmmArgs& a, int rpw, hipStream_t stream, int r = 2) {
  if constexpr (MM == 1 && CPL == 1) {
    if (rpw == 4 && r == 4) return launch_qmvx_cfg<BITS, MM, CPL, 4, KS, WAVES, 4, MX>(a, stream);
  }
  if (rpw == 2) return launch_qmvx_cfg<BITS, MM, CPL, 2, KS, WAVES, 2, MX>(a, stream);
  if constexpr (MM <= 8) {
    if (rpw == 4) return launch_qmvx_cfg<BITS, MM, CPL, 4, KS, WAVES, 2, MX>(a, stream);
  }
  if constexpr (MM <= 4) return launch_qmvx_cfg<BITS, MM, CPL, 8, KS, WAVES, 2, MX>(a, stream);
  return launch_qmvx_cfg<BITS, MM, CPL, 4, KS, WAVES, 2, MX>(a, stream);
}

// The M <= 8 rows of x padded to 1, 2, 4 or 8; shapes whose x chunks would not
// fit in registers use the general kernels.
static int qmvx_mm(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

static bool qmvx_supported(const QmmArgs& a, int bits) {
  if (a.M < 1 || a.M > 8) return false;
  const int64_t nch = a.K / (128 / bits);
  return pick_qmvx_shape(nch, a.N, qmvx_mm(a.M), bits, a.M).cpl > 0;
}

template <int BITS, int MM, int MX = MM>
static hipError_t launch_qmvx_mm(const QmmArgs& a, hipStream_t stream) {
  const QmvxShape sh = pick_qmvx_shape(a.K / (128 / BITS), a.N, MM, BITS, a.M);
  if constexpr (BITS == 8 && (MM <= 4 || (MM == 8 && MX <= 5))) {
    if (sh.ks == 8 && sh.cpl == 2) return launch_qmvx_rpw<BITS, MM, 2, 8, 8, MX>(a, sh.rpw, stream, sh.r);
  }
  if (sh.ks == 8) return launch_qmvx_rpw<BITS, MM, 1, 8, 8, MX>(a, sh.rpw, stream, sh.r);
  if (sh.ks == 1) return launch_qmvx_rpw<BITS, MM, 1, 1, 4, MX>(a, sh.rpw, stream);
  if (sh.ks == 2) {
    if (sh.waves == 8) return launch_qmvx_rpw<BITS, MM, 1, 2, 8, MX>(a, sh.rpw, stream, sh.r);
    return launch_qmvx_rpw<BITS, MM, 1, 2, 4, MX>(a, sh.rpw, stream, sh.r);
  }
  if (sh.cpl == 1) return launch_qmvx_rpw<BITS, MM, 1, 4, 4, MX>(a, sh.rpw, stream);
  if constexpr (MM <= 4) {
    if (sh.cpl == 2) return launch_qmvx_rpw<BITS, MM, 2, 4, 4, MX>(a, sh.rpw, stream);
  }
  if constexpr (MM <= 2) return launch_qmvx_rpw<BITS, MM, 4, 4, 4, MX>(a, sh.rpw, stream);
  return hipErrorInvalidValue;  // excluded by qmvx_supported
}

template <int BITS>
static hipError_t launch_qmvx(const QmmArgs& a, hipStream_t stream) {
  switch (qmvx_mm(a.M)) {
    case 1: return launch_qmvx_mm<BITS, 1>(a, stream);
    case 2: return launch_qmvx_mm<BITS, 2>(a, stream);
    case 4: return launch_qmvx_mm<BITS, 4>(a, stream);
    default:
      if (a.M == 5) return launch_qmvx_mm<BITS, 8, 5>(a, stream);
      if (a.M == 6) return launch_qmvx_mm<BITS, 8, 6>(a, stream);
      if (a.M == 7) return launch_qmvx_mm<BITS, 8, 7>(a, stream);
      return launch_qmvx_mm<BITS, 8>(a, stream);
  }
}

// ---------------------------------------------------------------------------
// General decode GEMV for M <= 4.

template <int BITS, int MM, int R, int CPL, int KS>
__global__ __launch_bounds__(256) void qmv_kernel(QmmArgs a) {
  constexpr int CH = 128 / BITS;
  constexpr int RG = 4 / KS;  // row groups per block
  __shared__ float part[KS > 1 ? RG : 1][KS > 1 ? KS - 1 : 1][R][MM];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = wave / KS, ks = wave % KS;
  const int64_t n0 = ((int64_t)blockIdx.x * RG + rg) * R;
  const int64_t nch = a.K / CH;
  const int64_t c0 = ks * nch / KS, c1 = (ks + 1) * nch / KS;
  const int gshift = __builtin_ctz((unsigned)a.group_size);
  const int chunk_gshift = gshift - __builtin_ctz((unsigned)CH);
  const int64_t wpr = a.K * BITS / 32, gpr = a.K >> gshift;

  // Issue every weight and scale/bias load of this wave first.  Rows past N and
  // chunks past the slice are clamped to valid addresses and masked below.
  u32x4 wv[R][CPL];
  float sv[R][CPL], bv[R][CPL];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t n = n0 + r < a.N ? n0 + r : a.N - 1;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      int64_t c = c0 + lane + 64 * i;
      c = c < c1 ? c : c1 - 1;
      wv[r][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.w + n * wpr) + c);
      const int64_t g = c >> chunk_gshift;
      sv[r][i] = bf16_bits_to_f32(a.scales[n * gpr + g]);
      bv[r][i] = bf16_bits_to_f32(a.biases[n * gpr + g]);
    }
  }
  float acc[R][MM];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[r][m] = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int64_t c = c0 + lane + 64 * i;
    if (c < c1) {
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        XChunk<BITS> xc;
        xc.load(a.x + (int64_t)m * a.ldx, c * CH);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float d = chunk_dot<BITS>(wv[r][i], xc);
          const float boff = __builtin_fmaf(-magic_offset<BITS>(), sv[r][i], bv[r][i]);
          acc[r][m] = __builtin_fmaf(sv[r][i], d, __builtin_fmaf(boff, xc.sum, acc[r][m]));
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[r][m] = wave_sum_dpp(acc[r][m]);
  if constexpr (KS > 1) {
    if (ks > 0 && lane == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MM; ++m) part[rg][ks - 1][r][m] = acc[r][m];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int s = 0; s < KS - 1; ++s) acc[r][m] += part[rg][s][r][m];
  }
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

// K split and chunks per lane: the fewest K slices that keep a wave at no more
// than 2 chunks per row (4 for the longest rows).
struct QmvShape {
  int ks, cpl;
};
static QmvShape pick_qmv_shape(int64_t nch) {
  if (nch <= 64) return {1, 1};
  if (nch <= 128) return {1, 2};
  if (nch <= 256) return {2, 2};
  if (nch <= 512) return {4, 2};
  return {4, (int)((nch + 255) / 256)};
}

template <int BITS, int MM, int R, int CPL, int KS>
static hipError_t launch_qmv_cfg(const QmmArgs& a, hipStream_t stream) {
  constexpr int rows_per_block = (4 / KS) * R;
  const unsigned blocks = (unsigned)((a.N + rows_per_block - 1) / rows_per_block);
  qmv_kernel<BITS, MM, R, CPL, KS><<<blocks, 256, 0, stream>>>(a);
  return hipGetLastError();
}

template <int BITS, int MM, int R>
static hipError_t launch_qmv_r(const QmmArgs& a, const QmvShape& sh, hipStream_t stream) {
  if (sh.ks == 1 && sh.cpl == 1) return launch_qmv_cfg<BITS, MM, R, 1, 1>(a, stream);
  if (sh.ks == 1) return launch_qmv_cfg<BITS, MM, R, 2, 1>(a, stream);
  if (sh.ks == 2) return launch_qmv_cfg<BITS, MM, R, 2, 2>(a, stream);
  if (sh.cpl <= 2) return launch_qmv_cfg<BITS, MM, R, 2, 4>(a, stream);
  if (sh.cpl <= 4) return launch_qmv_cfg<BITS, MM, R, 4, 4>(a, stream);
  return launch_qmv_cfg<BITS, MM, R, 8, 4>(a, stream);
}

template <int BITS, int MM>
static hipError_t launch_qmv_m(const QmmArgs& a, hipStream_t stream) {
  const QmvShape sh = pick_qmv_shape(a.K / (128 / BITS));
  // Two rows per wave share each x chunk; worth it once there are rows to spare.
  const bool two = sh.ks == 1 && a.N >= 8192;
  return two ? launch_qmv_r<BITS, MM, 2>(a, sh, stream) : launch_qmv_r<BITS, MM, 1>(a, sh, stream);
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

bool qmv_supported(const QmmArgs& a) {
  return a.M <= kQmvMaxM || qmvx_supported(a, a.bits);
}

// Several products of one x row in one launch: every matrix M = 1, int4 group 64,
// the same K and x, the slice kernel's alignment; the shape is the one a single
// matrix of all their rows would take (q | k | v of 4096 + 1024 + 1024 rows: 8 rows
// per wave; gate | up of 2 x 14336: 4).  hipErrorNotSupported otherwise.
hipError_t launch_qmv1_slice_group(const QmmArgs* mats, int n, hipStream_t stream) {
  if (n < 1 || n > kSliceGroupMax) return hipErrorNotSupported;
  SliceGroup g{};
  g.n = n;
  int64_t total = 0;
  for (int i = 0; i < n; ++i) {
    const QmmArgs& a = mats[i];
    if (!slice_supported(a) || a.K != mats[0].K || a.x != mats[0].x || a.N < 0)
      return hipErrorNotSupported;
    g.m[i] = a;
    total += a.N;
  }
  if (total >= (int64_t(1) << 31)) return hipErrorNotSupported;
  if (total == 0) return hipSuccess;
  return with_slice_shape(mats[0].K, total, [&](auto rw, auto ks, auto rg) -> hipError_t {
    constexpr int RW = decltype(rw)::value, KS = decltype(ks)::value, RG = decltype(rg)::value;
    constexpr int64_t rows = RW * RG;
    int64_t b = 0;
    for (int i = 0; i < n; ++i) {
      g.first[i] = b;
      b += (g.m[i].N + rows - 1) / rows;
    }
    for (int i = n; i <= kSliceGroupMax; ++i) g.first[i] = b;
    if (b == 0) return hipSuccess;
    qmv1_slice_group_kernel<RW, KS, RG><<<(unsigned)b, KS * RG * 64, 0, stream>>>(g);
    return hipGetLastError();
  });
}

hipError_t launch_qmv(const QmmArgs& a, hipStream_t stream) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  const hipError_t e0 = launch_qmv1_slice(a, stream);
  if (e0 != hipErrorNotSupported) return e0;
  const hipError_t e1 = launch_qmv1(a, stream);
  if (e1 != hipErrorNotSupported) return e1;
  if (qmvx_supported(a, a.bits))
    return a.bits == 4 ? launch_qmvx<4>(a, stream) : launch_qmvx<8>(a, stream);
  return a.bits == 4 ? launch_qmv_bits<4>(a, stream) : launch_qmv_bits<8>(a, stream);
}

// ---------------------------------------------------------------------------
// Gathered GEMV: grid (slots, row blocks).  Each slot reads its own x row and
// the weight slice of its expert.  An out-of-range index writes zeros for that
// slot and raises err_flag instead of reading outside the stacks.

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
  uint16_t* yrow = a.y + (a.yrow ? (int64_t)a.yrow[slot] : slot) * a.N;
  if (e >= a.E || xi >= a.x_batch) {
    if (lane == 0) {
      for (int r = 0; r < R; ++r)
        if (n0 + r < a.N) yrow[n0 + r] = 0;
      atomicOr(a.err_flag, 1u);
    }
    return;
  }
  const int64_t wpr = a.K * BITS / 32, gpr = a.K >> __builtin_ctz((unsigned)a.group_size);
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
