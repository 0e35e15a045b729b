// fmxq_moe_gemm.hip -- grouped int4 (group 64) product over expert segments:
// the gather_qmm calls of a SwitchGLU layer (compute/models/switch_glu.go:107-153;
// mlx_gather_qmm, mlxgo/binding_cgo.go:645-673) once the routing slots are sorted
// by expert.
//
// Slots sorted by expert id form runs; a segment is a piece of one run, the run
// cut every W slots from its start (W = 16 MT), so a segment holds at most 16 MT
// slots of one expert and a run of c slots reads the expert's weights
// ceil(c / W) times (a block of a 32-slot window whose segment has at most 16
// slots walks one 16-row tile only).  sort_slots_kernel (fmxq_moe.hip) writes the segment table
// while it sorts.  Grid: (column tiles, segment bound); blocks past the actual
// segment count return at once.  A block of 4 waves = WC column groups x KS K
// slices computes its segment's rows against 16 NTT WC columns of that expert's
// weights with the skinny-product walk of fmxq_qmvs.hpp (whole-segment weight
// loads through LDS, v_mfma_f32_16x16x32_bf16), so each expert's weights are read
// once per segment whatever the number of slots.  With one K slice (every grid of
// about two blocks per CU or more) the block runs moe_qmvw_kernel: the 4 waves
// share the segment's x rows through an LDS stage that the block fills by DMA
// (qmvs_walk_xlds); smaller grids run moe_qmvs_kernel, each wave loading its own
// x rows.  Without a segment table (few slots), rows of 2048 <= K <= 16384 take
// the GEMV form (moe_qmv1_kernel) instead.
//
// NMAT = 2 fuses the gate and up projections: both walk the same x rows and the
// block writes h = silu(gate) * up with the op chain's bf16 roundings
// (qwen3_forward.go:229-239): g, u rounded to bf16, sigmoid rounded, g * sigmoid
// rounded, times u rounded.  NMAT = 1 writes bf16(acc) to output row yrow[slot]
// (the unsort of switch_glu.go:150-152) or to row slot.
//
// Without a segment table (a.seg null, few slots) segment i is slot i alone, in
// the caller's slot order.
//
// A slot whose expert id is >= E or whose x row is >= x_rows gets a zero output
// row and raises err_flag.
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"
#include "fmxq_qmvs.hpp"
#include "fmxq_qmv_impl.hpp"

namespace fmxq {
namespace {

__device__ __forceinline__ float r16(float v) { return bf16_bits_to_f32(f32_to_bf16_rne(v)); }

// Store a segment's rows.  C layout of a 16x16 tile: register r of lane l is row
// 4 (l / 16) + r, column l % 16.  Row m of tile mt is slot start + 16 mt + m; nb
// is the wave's first column.
template <int MT, int NTT, int NMAT>
__device__ __forceinline__ void store_segment(const MoeArgs& a, int64_t start, int64_t len,
                                              bool bad_e, int64_t nb,
                                              const f32x4 (&acc)[NMAT][MT][NTT]) {
  const int lane = threadIdx.x & 63;
  const int c16 = lane & 15, q = lane >> 4;
  bool raise = false;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 16 * mt + 4 * q + r;
      if (m >= len) continue;
      const int64_t slot = start + m;
      const int64_t xr = a.lhs ? (int64_t)a.lhs[slot] : slot / a.lhs_div;
      const bool bad = bad_e || xr >= a.x_rows;
      raise |= bad;
      const int64_t orow = a.yrow ? (int64_t)a.yrow[slot] : slot;
      uint16_t* yr = a.y + orow * a.N;
#pragma unroll
      for (int t = 0; t < NTT; ++t) {
        const int64_t n = nb + 16 * t + c16;
        if (n >= a.N) continue;
        uint16_t v;
        if (bad) {
          v = 0;
        } else if constexpr (NMAT == 2) {
          const float g = r16(acc[0][mt][t][r]), u = r16(acc[1][mt][t][r]);
          const float sg_ = r16(1.f / (1.f + __expf(-g)));
          v = (uint16_t)f32_to_bf16_rne(r16(r16(g * sg_) * u));
        } else {
          v = (uint16_t)f32_to_bf16_rne(acc[0][mt][t][r]);
        }
        yr[n] = v;
      }
    }
  if (raise) atomicOr(a.err_flag, 1u);
}

template <int MT, int NTT, int WC, int NMAT>
__global__ __launch_bounds__(256) void moe_qmvs_kernel(MoeArgs a) {
  constexpr int SU = 4;
  constexpr int KS = 4 / WC;
  using G = QmvsGeom<NTT, SU>;
  __shared__ __attribute__((aligned(16))) uint8_t stage[4][NMAT * G::STAGE];
  __shared__ float red[KS > 1 ? KS - 1 : 1][WC][NMAT][MT][NTT][4][64];

  const int64_t sg = blockIdx.y;
  if (sg >= (a.seg ? (int64_t)*a.nseg : a.S)) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wc = wave % WC, ks = wave / WC;
  const int c16 = lane & 15, q = lane >> 4;
  const int64_t start = a.seg ? (int64_t)a.seg[2 * sg] : sg;
  const int64_t len = a.seg ? (int64_t)a.seg[2 * sg + 1] : 1;
  const uint32_t e = a.rhs[start];
  const int64_t nb = (int64_t)blockIdx.x * (16 * NTT * WC) + wc * (16 * NTT);
  const bool sh = a.sh_seg && (int64_t)e == a.E;
  const bool bad_e = (int64_t)e >= a.E && !sh;

  // x row of each of this lane's slots (row of the segment's first slot for lanes
  // past its end; a bad slot reads row 0 and is zeroed at the store).
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + c16;
    const int64_t slot = start + (m < len ? m : 0);
    int64_t xr = a.lhs ? (int64_t)a.lhs[slot] : slot / a.lhs_div;
    if (xr >= a.x_rows) xr = 0;
    xrow[mt] = a.x + xr * a.K + q * 16;
  }

  f32x4 acc[NMAT][MT][NTT];
#pragma unroll
  for (int p = 0; p < NMAT; ++p)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < NTT; ++t) acc[p][mt][t] = f32x4{};
  if (!bad_e) {
    const int64_t wpr = a.K / 8, gpr = a.K / 64;
    const uint32_t* w[NMAT];
    const uint16_t* sc[NMAT];
    const uint16_t* bi[NMAT];
#pragma unroll
    for (int p = 0; p < NMAT; ++p) {
      w[p] = sh ? a.sh_w[p] : a.w[p] + (int64_t)e * a.N * wpr;
      sc[p] = sh ? a.sh_s[p] : a.s[p] + (int64_t)e * a.N * gpr;
      bi[p] = sh ? a.sh_b[p] : a.b[p] + (int64_t)e * a.N * gpr;
    }
    const int64_t nst = a.K / (SU * 64);
    const int64_t st0 = ks * nst / KS, st1 = (ks + 1) * nst / KS;
    if (MT == 2 && len <= 16) {
      // Short segment of a 32-slot window: the 16-row walk (the second tile's
      // accumulators stay zero and no row of it is stored).
      const uint16_t* const x1[1] = {xrow[0]};
      f32x4 acc1[NMAT][1][NTT];
#pragma unroll
      for (int p = 0; p < NMAT; ++p)
#pragma unroll
        for (int t = 0; t < NTT; ++t) acc1[p][0][t] = f32x4{};
      qmvs_slice<1, NTT, SU, NMAT, true>(stage[wave], w, sc, bi, nb, a.N, a.K, x1, st0, st1, acc1);
#pragma unroll
      for (int p = 0; p < NMAT; ++p)
#pragma unroll
        for (int t = 0; t < NTT; ++t) acc[p][0][t] = acc1[p][0][t];
    } else {
      qmvs_slice<MT, NTT, SU, NMAT, true>(stage[wave], w, sc, bi, nb, a.N, a.K, xrow, st0, st1, acc);
    }
  }

  if constexpr (KS > 1) {
    if (ks > 0) {
#pragma unroll
      for (int p = 0; p < NMAT; ++p)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int t = 0; t < NTT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[ks - 1][wc][p][mt][t][r][lane] = acc[p][mt][t][r];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int p = 0; p < NMAT; ++p)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < NTT; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int k = 0; k < KS - 1; ++k) acc[p][mt][t][r] += red[k][wc][p][mt][t][r][lane];
  }

  store_segment<MT, NTT, NMAT>(a, start, len, bad_e, nb, acc);
}

#ifndef FMXQ_MOE_DEQ_MIN_MT
#define FMXQ_MOE_DEQ_MIN_MT 2
#endif
// Walks of at least this many 16-row x tiles dequantize the weights (DEQ of
// qmvs_walk_xlds) instead of folding the bias term: the 32-slot segments with
// more than 16 slots.  Measured per layer: configuration 4 at M=256 1529-1541 ->
// 1492 us, at M=32 581-583 -> 575-579 us; configuration 3 at M=512 254-259 ->
// 249-252 us, at M=128 unchanged.
constexpr int kMoeDeqMinMT = FMXQ_MOE_DEQ_MIN_MT;

// Fixed-length (16 or 32 slot) x-in-LDS form of moe_qmvs_kernel for blocks whose
// 4 waves walk the whole K range side by side (16 NTT columns each): the
// segment's x rows go to LDS once per step for all four (qmvs_walk_xlds), so a
// step's texture-unit traffic is the weights plus a quarter of x instead of the
// weights plus all of x per wave.
template <int MT, int NTT, int NMAT, int WV>
__global__ __launch_bounds__(WV * 64) __attribute__((amdgpu_waves_per_eu(MT == 1 && NTT == 1 ? 3 : 2))) void moe_qmvw_kernel(
    MoeArgs a) {
  using G = QmvsGeom<NTT, 4>;
  __shared__ __attribute__((aligned(1024))) uint8_t xs[2][16 * MT * kXStageRow];
  __shared__ __attribute__((aligned(16))) uint8_t stage[WV][NMAT * G::STAGE];

  const int64_t sg = blockIdx.y;
  if (sg >= (a.seg ? (int64_t)*a.nseg : a.S)) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t start = a.seg ? (int64_t)a.seg[2 * sg] : sg;
  const int64_t len = a.seg ? (int64_t)a.seg[2 * sg + 1] : 1;
  const uint32_t e = a.rhs[start];
  const int64_t nb = (int64_t)blockIdx.x * (16 * NTT * WV) + wave * (16 * NTT);
  const bool sh = a.sh_seg && (int64_t)e == a.E;
  const bool bad_e = (int64_t)e >= a.E && !sh;

  f32x4 acc[NMAT][MT][NTT];
#pragma unroll
  for (int p = 0; p < NMAT; ++p)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < NTT; ++t) acc[p][mt][t] = f32x4{};
  if (!bad_e) {
    const int64_t wpr = a.K / 8, gpr = a.K / 64;
    const uint32_t* w[NMAT];
    const uint16_t* sc[NMAT];
    const uint16_t* bi[NMAT];
#pragma unroll
    for (int p = 0; p < NMAT; ++p) {
      w[p] = sh ? a.sh_w[p] : a.w[p] + (int64_t)e * a.N * wpr;
      sc[p] = sh ? a.sh_s[p] : a.s[p] + (int64_t)e * a.N * gpr;
      bi[p] = sh ? a.sh_b[p] : a.b[p] + (int64_t)e * a.N * gpr;
    }
    // moe_xlds_supported keeps x_rows * K * 2 below 2^31.
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a.x, (short)0, (int)(a.x_rows * a.K * 2), 0x00020000);
    // Byte offset of the x chunk lane `lane` fetches for DMA instruction j (see
    // qmvs_walk_xlds): stage row r is slot start + r (the first slot for a row past
    // the segment that shares an issued instruction), a bad x row reads row 0 (its
    // output is zeroed).
    auto x_offsets = [&](uint32_t* xo, int ax) {
      for (int j = 0; j < ax; ++j) {
        const int r = 2 * (wave * ax + j) + (lane >> 5);
        const int c = (lane & 31) ^ (r & 15);
        const int64_t slot = start + (r < len ? r : 0);
        int64_t xr = a.lhs ? (int64_t)a.lhs[slot] : slot / a.lhs_div;
        if (xr >= a.x_rows) xr = 0;
        xo[j] = (uint32_t)(xr * a.K * 2 + c * 16);
      }
    };
    // One matrix with K <= 512 (the down projection of 512-wide experts): a walk
    // of one or two steps, so every load is issued first (qmvs_walk_xall).
    const bool upfront = NMAT == 1 && a.K <= 512;
    if (MT == 2 && len <= 16) {
      // Short segment of a 32-slot window: 16 stage rows, one tile walked.
      uint32_t xo[8 / WV];
      x_offsets(xo, 8 / WV);
      if (upfront) {
        f32x4 acc1[1][NTT];
#pragma unroll
        for (int t = 0; t < NTT; ++t) acc1[0][t] = f32x4{};
        qmvs_walk_xall<1, NTT, WV, 2>(&xs[0][0], stage[wave], xres, xo, wave, w[0], sc[0], bi[0],
                                      nb, a.N, a.K, 0, a.K / 256, acc1);
#pragma unroll
        for (int t = 0; t < NTT; ++t) acc[0][0][t] = acc1[0][t];
      } else {
        qmvs_walk_xlds<1, MT, NTT, NMAT, WV, true>(xs[0], xs[1], stage[wave], xres, xo, wave, len, w, sc,
                                             bi, nb, a.N, a.K, 0, a.K / 256, acc);
      }
    } else {
      uint32_t xo[8 * MT / WV];
      x_offsets(xo, 8 * MT / WV);
      if (upfront)
        qmvs_walk_xall<MT, NTT, WV, 2>(&xs[0][0], stage[wave], xres, xo, wave, w[0], sc[0], bi[0],
                                       nb, a.N, a.K, 0, a.K / 256, acc[0]);
      else
        qmvs_walk_xlds<MT, MT, NTT, NMAT, WV, !(MT >= kMoeDeqMinMT), (MT >= kMoeDeqMinMT)>(
            xs[0], xs[1], stage[wave], xres, xo, wave, len, w, sc, bi, nb, a.N, a.K, 0,
            a.K / 256, acc);
    }
  }
  store_segment<MT, NTT, NMAT>(a, start, len, bad_e, nb, acc);
}

// x through buffer resources needs every byte offset of x below 2^31, and the
// 16-byte DMA a 16-byte aligned base.
static bool moe_xlds_supported(const MoeArgs& a) {
  return a.x_rows > 0 && a.x_rows * a.K * 2 < (int64_t(1) << 31) &&
         (reinterpret_cast<uintptr_t>(a.x) & 15) == 0;
}

template <int MT, int NTT, int NMAT>
static hipError_t launch_wc(const MoeArgs& a, int wc, int64_t max_seg, hipStream_t stream) {
  const int64_t cols = 16 * NTT * wc;
  dim3 grid((unsigned)((a.N + cols - 1) / cols), (unsigned)max_seg);
  // Four waves per block: an 8-wave block (128 columns per x fetch, two blocks
  // per CU) measured slower (configuration 4 at M=256: 1871 -> 1971 us, and again
  // with the dequantizing walk: 1463-1478 -> 1553-1604 us; at M=32 with one-tile
  // segments too: 556-561 -> 620 us), unlike the dense walk's 64-row tiles.
  if (wc == 4 && moe_xlds_supported(a)) moe_qmvw_kernel<MT, NTT, NMAT, 4><<<grid, 256, 0, stream>>>(a);
  else if (wc == 1) moe_qmvs_kernel<MT, NTT, 1, NMAT><<<grid, 256, 0, stream>>>(a);
  else if (wc == 2) moe_qmvs_kernel<MT, NTT, 2, NMAT><<<grid, 256, 0, stream>>>(a);
  else moe_qmvs_kernel<MT, NTT, 4, NMAT><<<grid, 256, 0, stream>>>(a);
  return hipGetLastError();
}


// The few-slot path (no sort: every slot its own segment, in slot order) with
// 2048 <= K <= 16384: the decode GEMV form of the same product.  With a segment
// table it takes segments of up to MM slots and leaves longer ones.  Grid
// (row blocks of RW, segments); a block is KS waves splitting K, lane l owning
// 16-byte chunk c0 + l of its slice for all RW rows of each of the NMAT matrices.
// Each packed word is unpacked once and dotted with the segment's x rows (v_dot2
// on exponent-trick pairs, then s d + (b - 128 s) sum(x) per chunk, as in the
// dense GEMV, fmxq_qmv.hip).  The slices meet in LDS and wave 0 stores RW output
// columns per slot (silu(g) * u with the op chain's roundings for NMAT = 2).
// Segments longer than MM are left to the MFMA walk above.
template <int NMAT, int RW, int KS, int MM, bool SH>
__global__ __launch_bounds__(KS * 64) void moe_qmv1_kernel(MoeArgs a) {
  constexpr int V = NMAT * RW * MM;  // partials per lane: index (p RW + r) MM + m
  constexpr int LV = __builtin_ctz(V);
  static_assert((V & (V - 1)) == 0 && V <= 64, "partials per lane");
  __shared__ float part[KS][V];
  const int lane = threadIdx.x & 63;
  const int ks = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t sg = blockIdx.y;
  int64_t start = sg, len = 1;
  if (a.seg) {
    if (sg >= (int64_t)*a.nseg) return;
    start = a.seg[2 * sg];
    len = a.seg[2 * sg + 1];
    if (len > MM) return;
  }
  const int64_t nbase = (int64_t)blockIdx.x * RW;
  // SH: segments past the S slots (sh_T of them, no segment table) are the shared
  // expert on x row sg - S, written to row sg.
  const bool shs = SH && sg >= a.S;
  const uint32_t* wp[NMAT];
  const uint16_t* sp[NMAT];
  const uint16_t* bp[NMAT];
#pragma unroll
  for (int p = 0; p < NMAT; ++p) {
    wp[p] = shs ? a.sh_w[p] : a.w[p];
    sp[p] = shs ? a.sh_s[p] : a.s[p];
    bp[p] = shs ? a.sh_b[p] : a.b[p];
  }
  int64_t xr[MM], orow[MM];
  bool rbad[MM];
#pragma unroll
  for (int m = 0; m < MM; ++m) {
    const int64_t slot = start + (m < len ? m : 0);
    // Slot counts stay below 2^31 (checked by the callers): a 32-bit division.
    const int64_t r = shs ? sg - a.S
                          : a.lhs ? (int64_t)a.lhs[slot]
                                  : (int64_t)((uint32_t)slot / (uint32_t)a.lhs_div);
    rbad[m] = r >= a.x_rows;
    xr[m] = rbad[m] ? 0 : r;
    orow[m] = a.yrow ? (int64_t)a.yrow[slot] : slot;
  }
  const int nch = (int)(a.K / 32);
  const int c0 = ks * nch / KS, c1 = (ks + 1) * nch / KS;
  const int c = c0 + lane;
  const bool live = c < c1;
  const int cc = live ? c : c0;
  const int g = cc >> 1;  // group of the chunk (64 values = 2 chunks)
  const int64_t wpr = a.K / 8, gpr = a.K / 64;
  XChunk<4> xc[MM];
  auto load_x = [&]() {
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      xc[m].load(a.x + xr[m] * a.K, (int64_t)cc * 32);
      if (!live) xc[m].sum = 0.f;
    }
  };
  // One-wave blocks request x before the expert id is read, so x arrives while
  // the id's round trip and the weight requests go on (configuration 3 at M = 1
  // and 16, with the same order in the down/combine kernel: 10.1 -> 9.7 us and
  // 56.4 -> 53.4 us per layer).  Blocks of several K slices keep x after the
  // weights (configuration 4 at M = 1 measured no gain from it).
  if constexpr (KS == 1) {
    load_x();
    __builtin_amdgcn_sched_barrier(0);
  }
  const uint32_t e = shs ? 0u : a.rhs[start];
  if (!shs && (int64_t)e >= a.E) {
    if (ks == 0) {
#pragma unroll
      for (int m = 0; m < MM; ++m)
        if (m < len && lane < RW && nbase + lane < a.N) a.y[orow[m] * a.N + nbase + lane] = 0;
      if (lane == 0) atomicOr(a.err_flag, 1u);
    }
    return;
  }
  u32x4 wv[NMAT][RW];
  uint32_t sv[NMAT][RW], bv[NMAT][RW];
  // The expert's matrices through buffer resources (each below 2^31 bytes,
  // moe_qmvs_supported): the lane's offset is fixed (its chunk) and each row's is
  // one wave-uniform scalar, so no per-row vector address math.  Rows in 32 bits,
  // clamped on the scalar unit; rows past N re-read row N-1 and are not stored.
  const int nb32 = __builtin_amdgcn_readfirstlane((int)nbase);
  const int nlast = (int)a.N - 1;
  __amdgpu_buffer_rsrc_t wres[NMAT], sres[NMAT], bres[NMAT];
#pragma unroll
  for (int p = 0; p < NMAT; ++p) {
    const int64_t erow = (int64_t)e * a.N;
    wres[p] = __builtin_amdgcn_make_buffer_rsrc((void*)(wp[p] + erow * wpr), (short)0,
                                                (int)(a.N * wpr * 4), 0x00020000);
    sres[p] = __builtin_amdgcn_make_buffer_rsrc((void*)(sp[p] + erow * gpr), (short)0,
                                                (int)(a.N * gpr * 2), 0x00020000);
    bres[p] = __builtin_amdgcn_make_buffer_rsrc((void*)(bp[p] + erow * gpr), (short)0,
                                                (int)(a.N * gpr * 2), 0x00020000);
  }
#pragma unroll
  for (int p = 0; p < NMAT; ++p)
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int n = __builtin_amdgcn_readfirstlane(min(nb32 + r, nlast));
      wv[p][r] = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(wres[p], cc * 16, n * (int)wpr * 4, 2));
      sv[p][r] = __builtin_amdgcn_raw_buffer_load_b16(sres[p], g * 2, n * (int)gpr * 2, 0);
      bv[p][r] = __builtin_amdgcn_raw_buffer_load_b16(bres[p], g * 2, n * (int)gpr * 2, 0);
    }
  // The weight requests go out before x is read and paired.
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (KS != 1) load_x();
  float res[V];
#pragma unroll
  for (int p = 0; p < NMAT; ++p)
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const float sc = bf16_bits_to_f32(sv[p][r]);
      const float bo = __builtin_fmaf(-magic_offset<4>(), sc, bf16_bits_to_f32(bv[p][r]));
      if constexpr (MM == 1) {
        const float t = __builtin_fmaf(sc, chunk_dot<4>(wv[p][r], xc[0]), bo * xc[0].sum);
        res[p * RW + r] = live ? t : 0.f;
      } else {
        uint32_t pk[16];
        unpack_chunk(wv[p][r], pk);
#pragma unroll
        for (int m = 0; m < MM; ++m) {
          const float t = __builtin_fmaf(sc, dot_pairs<4>(pk, xc[m]), bo * xc[m].sum);
          res[(p * RW + r) * MM + m] = live ? t : 0.f;
        }
      }
    }
  const float tot = wave_sum_multi<V>(res, lane);
  if ((lane & ((64 >> LV) - 1)) == 0) part[ks][lane >> (6 - LV)] = tot;
  __syncthreads();
  if (ks == 0 && lane < RW * MM) {
    const int r = lane / MM, m = lane % MM;
    const int64_t n = nbase + r;
    int64_t o = orow[0];
    bool bad = rbad[0];
#pragma unroll
    for (int mm = 1; mm < MM; ++mm)
      if (m == mm) {
        o = orow[mm];
        bad = rbad[mm];
      }
    if (m < len && n < a.N) {
      float acc[NMAT];
#pragma unroll
      for (int p = 0; p < NMAT; ++p) {
        acc[p] = 0.f;
#pragma unroll
        for (int k = 0; k < KS; ++k) acc[p] += part[k][(p * RW + r) * MM + m];
      }
      uint16_t v;
      if (bad) {
        v = 0;
      } else if constexpr (NMAT == 2) {
        const float gg = r16(acc[0]), u = r16(acc[1]);
        const float sg_ = r16(1.f / (1.f + __expf(-gg)));
        v = (uint16_t)f32_to_bf16_rne(r16(r16(gg * sg_) * u));
      } else {
        v = (uint16_t)f32_to_bf16_rne(acc[0]);
      }
      a.y[o * a.N + n] = v;
      if (bad) atomicOr(a.err_flag, 1u);
    }
  }
}

template <int NMAT, int KS, int MM, int RW = 4>
static hipError_t launch_qmv1_ks(const MoeArgs& a, int64_t segs, hipStream_t stream) {
  dim3 grid((unsigned)((a.N + RW - 1) / RW), (unsigned)segs);
  if (a.sh_T > 0)
    moe_qmv1_kernel<NMAT, RW, KS, MM, true><<<grid, KS * 64, 0, stream>>>(a);
  else
    moe_qmv1_kernel<NMAT, RW, KS, MM, false><<<grid, KS * 64, 0, stream>>>(a);
  return hipGetLastError();
}

template <int NMAT, int MM>
static hipError_t launch_qmv1_nmat(const MoeArgs& a, int64_t segs, hipStream_t stream) {
  const int64_t nch = a.K / 32;
  // Rows up to 4096 values: 2 rows per block of 1-2 waves, so the few-slot grid
  // has enough waves (configuration 3 at M = 1, K = 2048: 8 rows 13.4 us, 4 rows
  // 12.1, 2 rows 11.5, 1 row 12.3 us per layer).  With 64 or more segments the
  // grid is large anyway, and 8 rows per wave load each x chunk for 4x the
  // weights (configuration 3 at M = 16, 160 slots: 72.0 -> 67.7 us per layer; 4
  // rows 68.8, 16 rows 71-73 us at 244 VGPRs).  Longer rows keep 4 rows over
  // 4-8 waves (configuration 4 at M = 1, K = 7168: 2 or 8 rows were slower).
  if (nch <= 64)
    return segs >= 64 ? launch_qmv1_ks<NMAT, 1, MM, 8>(a, segs, stream)
                      : launch_qmv1_ks<NMAT, 1, MM, 2>(a, segs, stream);
  if (nch <= 128) return launch_qmv1_ks<NMAT, 2, MM, 2>(a, segs, stream);
  if (nch <= 256) return launch_qmv1_ks<NMAT, 4, MM>(a, segs, stream);
  return launch_qmv1_ks<NMAT, 8, MM>(a, segs, stream);
}

// moe_down_combine_kernel: the few-slot down projection fused with the top-k
// combine (qwen3next_forward.go:519-524, deepseekv3_forward.go:436-440).  Block
// (row tile of RW output columns, token t), one wave per slot j of the token:
//   - wave j computes e_j = bf16(h[t k + j] . deq(Wd[e_j])^T) for the tile's rows
//     in the GEMV form of moe_qmv1_kernel (lane -> 16-byte chunk of 32 values,
//     LPR lanes per row, RW / (64 / LPR) passes of 64 / LPR rows), then
//     p_j = bf16(e_j * w[t, j]) into LDS;
//   - the first RW threads sum p_j in slot order in fp32 and finish as
//     moe_combine_kernel: bf16, then the shared term (sigmoid-gated or plain).
// A bad expert id gives p_j = 0 and raises the flag, as the unfused path's zero
// row does.
struct DownCombineArgs {
  const uint16_t* h;         // [T k, I] silu(gate) * up rows in slot order
  const uint32_t* inds;      // [T k] expert of each slot
  const uint32_t* w;         // [E, D, I/8]
  const uint16_t* s;         // [E, D, I/64]
  const uint16_t* b;
  const uint16_t* weights;   // [T, k] bf16 router weights
  const uint16_t* shared;    // [T, D] or null
  const uint16_t* sgate;     // [T] or null
  uint16_t* out;             // [T, D]
  int64_t T, k, E, D, I;
  uint32_t* err_flag;
  // The shared expert's down matrix [D, I/8] (and scales, biases), or null: wave k
  // of each block computes that expert's output for the token from h row T k + t.
  const uint32_t* sh_w = nullptr;
  const uint16_t* sh_s = nullptr;
  const uint16_t* sh_b = nullptr;
};

template <int RW, int LPR, int CPL, bool SH>
__global__ __launch_bounds__(1024) void moe_down_combine_kernel(DownCombineArgs a) {
  constexpr int RPP = 64 / LPR, PASSES = RW / RPP;
  static_assert(RW % RPP == 0, "rows per pass");
  __shared__ float part[SH ? 17 : 16][RW];
  const int lane = threadIdx.x & 63;
  const int j = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t = blockIdx.y, n0 = (int64_t)blockIdx.x * RW;
  // SH: wave k is the shared expert, h row T k + t, its own matrices.
  const bool shw = SH && j == a.k;
  const int64_t slot = shw ? a.T * a.k + t : t * a.k + j;
  const int rsub = lane / LPR, cl = lane % LPR;
  // What does not depend on the expert id is requested before the id is read: the
  // h row, the routing weight and the combine's shared term and gate, so that no
  // memory round trip is left for the end (configuration 3 at M = 1 and 16: 9.7
  // -> 9.5 us and 53.5 -> 51.8 us per layer against loading the last three at the
  // combine).
  XChunk<4> xc[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) xc[i].load(a.h + slot * a.I, (int64_t)(cl + LPR * i) * 32);
  // The shared expert's output is its bf16 product (no routing weight).
  const float wj = shw ? 1.f : bf16_bits_to_f32(a.weights[slot]);
  float shv = 0.f, sgv = 1.f;
  if (threadIdx.x < RW && n0 + threadIdx.x < a.D) {
    if (!SH && a.shared) shv = bf16_bits_to_f32(a.shared[t * a.D + n0 + threadIdx.x]);
    if (a.sgate) sgv = r16(1.f / (1.f + __expf(-bf16_bits_to_f32(a.sgate[t]))));
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t e = shw ? 0u : a.inds[slot];
  const bool bad = !shw && (int64_t)e >= a.E;
  const uint32_t* wm = shw ? a.sh_w : a.w;
  const uint16_t* sm = shw ? a.sh_s : a.s;
  const uint16_t* bm = shw ? a.sh_b : a.b;
  const int64_t wpr = a.I / 8, gpr = a.I / 64;
  float res[PASSES];
#pragma unroll
  for (int p = 0; p < PASSES; ++p) res[p] = 0.f;
  if (!bad && RPP == 1) {
    // One row per pass (whole-wave rows): plain loads, rows past D re-read row D - 1
    // (not stored).  Buffer loads measured slower here (configuration 4 at M = 1:
    // 55.4 -> 57.4 us).
    u32x4 wv[PASSES][CPL];
    uint32_t sv[PASSES][CPL], bv[PASSES][CPL];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      int64_t n = n0 + p * RPP + rsub;
      n = n < a.D ? n : a.D - 1;
      const int64_t row = (int64_t)e * a.D + n;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = cl + LPR * i;
        wv[p][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wm + row * wpr) + c);
        sv[p][i] = sm[row * gpr + (c >> 1)];
        bv[p][i] = bm[row * gpr + (c >> 1)];
      }
    }
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const float sc = bf16_bits_to_f32(sv[p][i]);
        const float bo = __builtin_fmaf(-magic_offset<4>(), sc, bf16_bits_to_f32(bv[p][i]));
        res[p] += __builtin_fmaf(sc, chunk_dot<4>(wv[p][i], xc[i]), bo * xc[i].sum);
      }
  } else if (!bad) {
    // Several rows per pass: the expert's three arrays through buffer resources
    // (each below 2^31 bytes, moe_down_combine_supported).  A lane's byte offsets
    // are set once and step by a wave-uniform stride per pass, which saves the
    // per-pass 64-bit row addressing (configuration 3 at M = 16: 67.6 -> 65.4 us);
    // rows past D fall outside the resource and read zeros (not stored).
    const int64_t erow = (int64_t)e * a.D;
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(wm + erow * wpr), (short)0, (int)(a.D * wpr * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(sm + erow * gpr), (short)0, (int)(a.D * gpr * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(bm + erow * gpr), (short)0, (int)(a.D * gpr * 2), 0x00020000);
    const int r0 = (int)(n0 + rsub);
    const int wstep = RPP * (int)wpr * 4, sstep = RPP * (int)gpr * 2;
    u32x4 wv[PASSES][CPL];
    uint32_t sv[PASSES][CPL], bv[PASSES][CPL];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = cl + LPR * i;
        const int wo = r0 * (int)wpr * 4 + c * 16 + p * wstep;
        const int so = r0 * (int)gpr * 2 + (c >> 1) * 2 + p * sstep;
        wv[p][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wres, wo, 0, 2));
        sv[p][i] = __builtin_amdgcn_raw_buffer_load_b16(sres, so, 0, 0);
        bv[p][i] = __builtin_amdgcn_raw_buffer_load_b16(bres, so, 0, 0);
      }
    }
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const float sc = bf16_bits_to_f32(sv[p][i]);
        const float bo = __builtin_fmaf(-magic_offset<4>(), sc, bf16_bits_to_f32(bv[p][i]));
        res[p] += __builtin_fmaf(sc, chunk_dot<4>(wv[p][i], xc[i]), bo * xc[i].sum);
      }
  }
  // Row totals: butterfly within each group of LPR lanes.
#pragma unroll
  for (int p = 0; p < PASSES; ++p)
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) res[p] += __shfl_xor(res[p], off, 64);
  if (cl == 0) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) part[j][p * RPP + rsub] = bad ? 0.f : r16(r16(res[p]) * wj);
  }
  if (bad && lane == 0) atomicOr(a.err_flag, 1u);
  __syncthreads();
  if (threadIdx.x < RW) {
    const int r = threadIdx.x;
    const int64_t n = n0 + r;
    if (n < a.D) {
      float acc = 0.f;
      for (int jj = 0; jj < a.k; ++jj) acc += part[jj][r];
      acc = r16(acc);
      if (SH || a.shared) {
        float sh = SH ? part[SH ? a.k : 0][r] : shv;
        if (a.sgate) sh = r16(sgv * sh);
        acc = r16(acc + sh);
      }
      a.out[t * a.D + n] = (uint16_t)f32_to_bf16_rne(acc);
    }
  }
}

template <int RW, int LPR, int CPL>
static hipError_t launch_down_combine_cfg(const DownCombineArgs& a, hipStream_t stream) {
  dim3 grid((unsigned)((a.D + RW - 1) / RW), (unsigned)a.T);
  if (a.sh_w)
    moe_down_combine_kernel<RW, LPR, CPL, true><<<grid, (unsigned)((a.k + 1) * 64), 0, stream>>>(a);
  else
    moe_down_combine_kernel<RW, LPR, CPL, false><<<grid, (unsigned)(a.k * 64), 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace

bool moe_down_combine_supported(int64_t T, int64_t k, int64_t D, int64_t I, int bits,
                                int group_size) {
  // One expert's down matrix (plus a row tile past its end) stays below 2^30 bytes:
  // the kernel addresses it through a buffer resource with 32-bit offsets.
  return bits == 4 && group_size == 64 && k >= 1 && k <= 16 && T >= 1 && T <= 65535 &&
         D >= 1 && (I == 512 || I == 1024 || I == 2048 || I == 4096 || I == 8192) &&
         (D + 64) * (I / 2) < (int64_t(1) << 30);
}

hipError_t launch_moe_down_combine(const uint16_t* h, const uint32_t* inds, const uint32_t* w,
                                   const uint16_t* s, const uint16_t* b, const uint16_t* weights,
                                   const uint16_t* shared, const uint16_t* sgate, uint16_t* out,
                                   int64_t T, int64_t k, int64_t E, int64_t D, int64_t I,
                                   uint32_t* err_flag, hipStream_t stream, const uint32_t* sh_w,
                                   const uint16_t* sh_s, const uint16_t* sh_b) {
  if (!moe_down_combine_supported(T, k, D, I, 4, 64) || (sh_w && (k > 15 || !sh_s || !sh_b)))
    return hipErrorInvalidValue;
  DownCombineArgs a{h, inds, w, s, b, weights, shared, sgate, out, T, k, E, D, I, err_flag};
  a.sh_w = sh_w;
  a.sh_s = sh_s;
  a.sh_b = sh_b;
  // Row tiles of 8 (I = 512) and 4 (I = 2048) columns: more blocks for the
  // one-token grids (configuration 3 at M = 1 11.5 -> 10.5-10.8 us with 8 rows
  // against 16, and 10.2-10.3 against 10.6-10.9 us with 4; configuration 4 at
  // M = 1 61.3 -> 58.3-58.9 us with 4 against 8, and 48-50 against 54-57 us with
  // 4 against 2).
  // From 8 tokens the grid is large, and 16-row tiles load each h row for 2x the
  // weights (configuration 3 at M = 16, whole layer: 8-row tiles 67.7 us, 32-row
  // 59.4-59.8 us, 16-row 58.5-58.7 us; 64 rows 60.9-61.2 us, and 32-row tiles of
  // 8 lanes x 2 chunks per row 59.6 us).
  switch (I) {
    case 512:
      return T >= 8 ? launch_down_combine_cfg<16, 16, 1>(a, stream)
                    : launch_down_combine_cfg<8, 16, 1>(a, stream);
    case 1024: return launch_down_combine_cfg<16, 32, 1>(a, stream);
    case 2048: return launch_down_combine_cfg<4, 64, 1>(a, stream);
    // Longer rows keep fewer rows per block so that a 16-wave block (16 slots)
    // fits its registers without spilling.
    case 4096: return launch_down_combine_cfg<4, 64, 2>(a, stream);
    default: return launch_down_combine_cfg<1, 64, 4>(a, stream);
  }
}

// One expert's weights go through a buffer resource: below 2^31 bytes.
bool moe_qmvs_supported(int64_t N, int64_t K, int bits, int group_size) {
  return bits == 4 && group_size == 64 && K % 256 == 0 && N >= 1 &&
         N * (K / 2) < (int64_t(1) << 31);
}

// 32-slot windows (two 16-row tiles per block) once slots average 4 per expert:
// fewer re-reads of long runs.  Below that the 16-slot form wins: its kernels hold
// fewer registers, so more blocks share a CU.  Measured with the shared-x walk:
// 16-slot windows everywhere, configuration 4 at M=256 1699 -> 1825 us and
// configuration 3 at M=512 346 -> 365 us; 32-slot windows everywhere,
// configuration 3 at M=16 79 -> 83 us.
int moe_window(int64_t S, int64_t E) { return S >= 4 * E ? 32 : 16; }

int64_t moe_max_segments(int64_t S, int64_t E, int window) {
  const int64_t runs = S < E + 1 ? S : E + 1;
  const int64_t b = runs + (S + window - 1) / window;
  return b < S ? b : S;
}

hipError_t launch_moe_qmvs(const MoeArgs& a, int nmat, int window, int64_t max_seg,
                           hipStream_t stream) {
  if (a.S <= 0 || a.N <= 0 || max_seg <= 0) return hipSuccess;
  if (!moe_qmvs_supported(a.N, a.K, 4, 64) || (window != 16 && window != 32) ||
      (nmat != 1 && nmat != 2))
    return hipErrorInvalidValue;
  // Without a segment table (the few-slot path: every slot its own segment), rows
  // of 2048..16384 values take the GEMV form (all lanes busy with 64-chunk
  // slices).  Sorted batches run every segment, one-slot ones included, on the
  // MFMA walk: with x shared through LDS a one-slot segment DMAs a single x row
  // pair, and the walk measured as fast as a separate GEMV launch for those
  // segments or faster (configuration 3 at M=16 86 -> 81 us, at M=128 248 -> 239
  // us), without the GEMV grid's blocks for every other segment.
  MoeArgs b = a;
  const bool gemv = a.K >= 2048 && a.K <= 16384 && !a.seg;
  // Shared-expert segments exist in the GEMV form, without an output row map, and
  // as id E of a segment table.
  const bool sh_ops = a.sh_w[0] && a.sh_s[0] && a.sh_b[0] &&
                      (nmat == 1 || (a.sh_w[1] && a.sh_s[1] && a.sh_b[1]));
  if (a.sh_T > 0 && (!gemv || a.yrow || !sh_ops)) return hipErrorInvalidValue;
  if (a.sh_seg && (!a.seg || a.sh_T > 0 || !sh_ops)) return hipErrorInvalidValue;
  if (gemv)
    return nmat == 2 ? launch_qmv1_nmat<2, 1>(a, a.S + a.sh_T, stream)
                     : launch_qmv1_nmat<1, 1>(a, a.S + a.sh_T, stream);
  // K slices per block; the remaining waves of the block take further column
  // groups.  One slice: the four waves walk the same K range and share the
  // segment's x rows through LDS (moe_qmvw_kernel; measured against about four
  // 4-unit steps per wave in up to 4 slices: configuration 4 at M=256 2537 -> 1874
  // us, at M=32 715 -> 661 us; configuration 3 at M=512 494 -> 374 us).  With few
  // segments (decode, a shared expert) the column tiles narrow (one 16-column tile
  // per wave, then more K slices while every slice keeps a step) until the grid has
  // about two blocks per CU.
  const int64_t nst = a.K / 256;
  int ks = 1;
  int ntt = nmat == 2 ? 1 : 2;
  auto blocks = [&](int ks_, int ntt_) {
    const int64_t cols = 16 * ntt_ * (4 / ks_);
    return (a.N + cols - 1) / cols * max_seg;
  };
  constexpr int64_t kMinBlocks = 512;
  if (blocks(ks, ntt) < kMinBlocks) ntt = 1;
  while (blocks(ks, ntt) < kMinBlocks && ks < 4 && 2 * ks <= nst) ks *= 2;
  const int wc = 4 / ks;
  if (nmat == 2)
    return window == 16 ? launch_wc<1, 1, 2>(b, wc, max_seg, stream)
                        : launch_wc<2, 1, 2>(b, wc, max_seg, stream);
  if (ntt == 1)
    return window == 16 ? launch_wc<1, 1, 1>(b, wc, max_seg, stream)
                        : launch_wc<2, 1, 1>(b, wc, max_seg, stream);
  return window == 16 ? launch_wc<1, 2, 1>(b, wc, max_seg, stream)
                      : launch_wc<2, 2, 1>(b, wc, max_seg, stream);
}

}  // namespace fmxq
