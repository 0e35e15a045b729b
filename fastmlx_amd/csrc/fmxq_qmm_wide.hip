// fmxq_qmm_wide.hip -- MFMA GEMM with the dequantization in registers, for
// quantized_matmul at prefill sizes (qmm_use_wide: M >= 384 rows of x, or
// M >= 128 for outputs at least twice the depth).
//
// Replaces the GEMM of mlx_quantized_matmul (mlxgo/binding_cgo.go:636-643) for
// x [M, K] with M = batch * seq rows: prefill through compute/models/quant.go:91-101
// from compute/models/llama.go:403-428.
//
// Tile: 256 rows of x by 256 weight rows (outputs), 64-deep K steps, 4 waves (one
// per SIMD).  Wave w owns the outputs n0 + 64 w .. + 64 of all 256 x rows:
//   - its packed weights go from global memory straight into registers (one
//     16-byte load per lane and 32-row group per step for 4-bit, two for 8-bit),
//     are dequantized there, w = bf16(fma(s, q, b)) (the exact s q + b rounded
//     once), and are the A operand of v_mfma_f32_32x32x16_bf16 without passing
//     through LDS; no two waves dequantize the same weights, and every weight is
//     dequantized once per 256 rows of x;
//   - x goes global -> LDS with buffer_load ... lds (16 bytes a lane) into one of
//     four stages, three steps ahead, and every wave reads all 256 rows of the
//     stage as the B operand.
// Lane L takes weight row L % 32 of a 32-row group and, in sub-step s, the K
// chunk (8 values) 4 (L / 32) + s of the step: the lane's four chunks of a step
// are one contiguous 16 bytes of packed words, and the x fragments are read in
// the same chunk order, so every product still pairs x[k] with w[k].
//
// Work per block: `dp` whole tiles, then (stream-K) a run of sk_len 64-deep
// iterations of the remaining tiles, cut at tile boundaries into pieces that are
// taken highest first.  A piece that ends its tile and does not start it
// (FINAL) waits for the pieces of the same tile from lower-numbered blocks
// (CONTRIB), each of which wrote its fp32 partial to the block's slot and bumped
// the tile's counter; the final piece adds the partials in block order, writes y
// and clears the counter.  Blocks only wait on lower-numbered blocks, and those
// write their partial first thing in their stream-K run, so the wait ends
// whatever the order in which the hardware dispatches blocks.
#include <type_traits>

#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"
#include "fmxq_mfma_frag.hpp"

namespace fmxq {
namespace {

typedef __attribute__((address_space(3))) void lds_t;

constexpr int kT = 256;                 // weight rows (outputs) of a tile
constexpr int kS = 64;                  // K values per step
constexpr int kWideWaves = 8;  // two waves per SIMD

// 16-byte chunk c of x row r sits at chunk position c ^ swz(r) of the row's 128
// LDS bytes: 8 consecutive rows at one chunk hit 8 distinct positions, and rows
// r and r + 8 differ in the lowest position bit (16 rows per 256 bytes).
__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// s_waitcnt with vmcnt = vm and lgkmcnt = lgkm (gfx9 encoding, expcnt left alone).
__device__ __forceinline__ constexpr int wait_enc(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8);
}

template <int BITS, int WAVES, int BM>
struct WideCfg {
  static constexpr int T = WAVES * 64;           // threads
  static constexpr int JT = 8 / WAVES;           // 32-row weight groups per wave (2 or 1)
  static constexpr int RT = BM / 32;             // 32-row x groups of a tile
  static constexpr int XI = BM / (8 * WAVES);    // x DMA instructions per wave and step
  static constexpr int STAGE = BM * kS * 2;      // bytes of one x stage
  static constexpr int LB = kS * BITS / 16;      // bytes of a lane's half row per step (16 or 32)
  static constexpr int NLD = LB / 16;            // 16-byte weight loads per lane and row group
  static constexpr int NV = XI + JT * NLD;       // vector memory instructions per step and wave
  static constexpr int NV0 = NV + 2;             // ... in the first step of each four (scales, biases)
};

enum Role { kFull = 0, kContrib = 1, kFinal = 2 };

template <int BITS, int WAVES, int BM>
__global__ __launch_bounds__(WAVES * 64, 1) void qmm_wide_kernel(WideArgs wa) {
  using C = WideCfg<BITS, WAVES, BM>;
  static_assert(WAVES == 8, "the output staging gives each of 8 waves 4 rows of a 32-row group");
  constexpr int T = C::T, JT = C::JT, RT = C::RT, XI = C::XI, NLD = C::NLD, NV = C::NV,
                NV0 = C::NV0, kStage = C::STAGE;
  // Four x stages, each its own LDS object so the compiler can tell the DMA
  // into one stage from the fragment reads of another (an LDS read it cannot
  // tell apart from a DMA target waits for every DMA in flight).
  __shared__ __attribute__((aligned(1024))) uint8_t xs0[kStage];
  __shared__ __attribute__((aligned(1024))) uint8_t xs1[kStage];
  __shared__ __attribute__((aligned(1024))) uint8_t xs2[kStage];
  __shared__ __attribute__((aligned(1024))) uint8_t xs3[kStage];
  auto stage = [&](int st) -> uint8_t* { return st == 0 ? xs0 : st == 1 ? xs1 : st == 2 ? xs2 : xs3; };
  __shared__ uint32_t s_flag;
  const QmmArgs& a = wa.q;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31, h = lane >> 5;
  const int P = gridDim.x, b = blockIdx.x;
  const int wcol = 32 * JT * wave;                      // first output of this wave in the tile

  const int64_t wpr = a.K * BITS / 32;                 // packed words per weight row
  const int64_t gpr = a.K / kS;                        // groups (of 64) per row
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.w, (short)0, (int)(a.N * wpr * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.scales, (short)0, (int)(a.N * gpr * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.biases, (short)0, (int)(a.N * gpr * 2), 0x00020000);

  // x DMA: instruction i of this wave fills tile rows 8 (XI wave + i) .. + 8 of a
  // stage; lane L lands at row + L / 8, chunk position L % 8, so it fetches
  // chunk (L % 8) ^ swz(row).
  uint32_t xdo[XI];
#pragma unroll
  for (int i = 0; i < XI; ++i) {
    const int row = 8 * (XI * wave + i) + (lane >> 3);
    xdo[i] = (uint32_t)(row * a.ldx * 2 + (((lane & 7) ^ swz(row)) << 4));
  }
  // x fragment of sub-step s: row r32 of each 32-row group, chunk 4 h + s.
  uint32_t xfo[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) xfo[s] = r32 * 128 + (((4 * h + s) ^ swz(r32)) << 4);

  f32x16 acc[JT][RT];
  bf16x8 af0[JT][4], af1[JT][4];   // A operands of two consecutive steps
  bf16x8 xf0[RT], xf1[RT];         // B operands of two consecutive sub-steps
  u32x4 wq[4][JT][NLD];            // packed weights, one set per step in flight
  // Scales and biases of four steps (one group each), words {s(0,1), s(2,3),
  // b(0,1), b(2,3)}: lane L holds those of weight row wcol + L (JT = 2) or of
  // row wcol + L % 32 (JT = 1).  sbA serves the current four steps, sbB is loaded
  // for the next four.
  uint32_t sbA[4], sbB[4];

  // Work items of this block: dp whole tiles (dealt to the XCDs so that each
  // one's resident blocks hold neighbouring tiles), then the stream-K pieces.
  const int64_t sk0 = (int64_t)b * wa.sk_len;
  const int64_t sk1 = sk0 + wa.sk_len < wa.sk_iters ? sk0 + wa.sk_len : wa.sk_iters;
  int64_t hi = sk1;
  int item = 0;
  for (;;) {
    int64_t tile;
    int kb, ke, role, first = 0;
    if (item < wa.dp) {
      const int bx = (P & 7) == 0 ? (b & 7) * (P >> 3) + (b >> 3) : b;
      tile = (int64_t)item * P + bx;
      kb = 0;
      ke = wa.nk;
      role = kFull;
      ++item;
    } else if (wa.sk_len > 0 && hi > sk0) {
      const int64_t r = (hi - 1) / wa.nk, ts = r * wa.nk;
      const int64_t lo = sk0 > ts ? sk0 : ts;
      tile = (int64_t)wa.dp * P + r;
      kb = (int)(lo - ts);
      ke = (int)(hi - ts);
      role = (kb == 0 && ke == wa.nk) ? kFull : (ke == wa.nk ? kFinal : kContrib);
      first = (int)(ts / wa.sk_len);  // first block of the tile (stream-K numbering)
      hi = lo;
    } else {
      break;
    }
    const int64_t m0 = (tile % wa.tm) * BM, n0 = (tile / wa.tm) * kT;

    // x rows of this tile through a buffer resource: rows past M read as zero.
    const int64_t rows_here = a.M - m0 < BM ? a.M - m0 : BM;
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.x + m0 * a.ldx), (short)0, (int)(rows_here * a.ldx * 2), 0x00020000);
    // Weight rows of this lane (rows past N load row N - 1; not stored).
    uint32_t wvo[JT];
#pragma unroll
    for (int j = 0; j < JT; ++j) {
      int64_t n = n0 + wcol + 32 * j + r32;
      if (n > a.N - 1) n = a.N - 1;
      wvo[j] = (uint32_t)(n * wpr * 4 + h * C::LB);
    }
    int64_t n_sb = n0 + wcol + (JT == 2 ? lane : r32);
    if (n_sb > a.N - 1) n_sb = a.N - 1;
    const uint32_t sbo = (uint32_t)(n_sb * gpr * 2);
    // Scales and biases of steps k .. k + 3 (8-byte aligned: gpr and k are
    // multiples of 4).
    auto load_sb = [&](uint32_t (&sb)[4], int k) {
      k = k < ke - 4 ? k : ke - 4;
      const u32x2 sv = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(sres, (int)sbo, k * 2, 0));
      const u32x2 bv = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(bres, (int)sbo, k * 2, 0));
      sb[0] = sv[0];
      sb[1] = sv[1];
      sb[2] = bv[0];
      sb[3] = bv[1];
    };

    // Loads of step k: the packed weights first, then the x DMA, so a wait for
    // the weights does not also wait for the DMA issued with them.
    // Steps past the piece issue nothing, so no DMA is still landing in a stage
    // when the epilogue reuses the stages; the last pass of four steps counts
    // its waits without them (below).
    auto issue = [&](int k, int st, int set) {
      if (k >= ke) return;
      const int woff = k * (kS * BITS / 8);
#pragma unroll
      for (int j = 0; j < JT; ++j)
#pragma unroll
        for (int l = 0; l < NLD; ++l)
          wq[set][j][l] = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(wres, (int)wvo[j] + 16 * l, woff, 0));
      const int xoff = k * kS * 2;
#pragma unroll
      for (int i = 0; i < XI; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            xres, (lds_t*)(stage(st) + 8 * (XI * wave + i) * 128), 16, (int)xdo[i], xoff, 0, 0);
    };
    // The scale and bias of step offset o (0..3) of sb as fp32 for each row group
    // of the lane.  With two row groups lane L holds row L's, and
    // v_permlane32_swap on two copies gives rows 0..31 to both halves of the wave
    // (row group 0) and rows 32..63 to both halves (row group 1).
    struct SB {
      float s[JT], b[JT];
    };
    auto scale_bias = [&](const uint32_t (&sb)[4], int o) {
      const uint32_t sw = sb[o >> 1], bw = sb[2 + (o >> 1)];
      const uint32_t sf = (o & 1) ? (sw & 0xffff0000u) : (sw << 16);
      const uint32_t bf = (o & 1) ? (bw & 0xffff0000u) : (bw << 16);
      SB r;
      if constexpr (JT == 2) {
        const auto sp = __builtin_amdgcn_permlane32_swap(sf, sf, false, false);
        const auto bp = __builtin_amdgcn_permlane32_swap(bf, bf, false, false);
        r.s[0] = __uint_as_float(sp[0]);
        r.s[1] = __uint_as_float(sp[1]);
        r.b[0] = __uint_as_float(bp[0]);
        r.b[1] = __uint_as_float(bp[1]);
      } else {
        r.s[0] = __uint_as_float(sf);
        r.b[0] = __uint_as_float(bf);
      }
      return r;
    };
    // Dequantize sub-step s of weight set `set` (every row group) into af[.][s].
    auto dequant = [&](bf16x8 (&af)[JT][4], int set, const SB& sb, int s) {
#pragma unroll
      for (int j = 0; j < JT; ++j) {
        if constexpr (BITS == 4) {
          af[j][s] = deq_frag4(wq[set][j][0][s], sb.s[j], sb.s[j] * 0.0625f, sb.b[j]);
        } else {
          const u32x4 v = wq[set][j][s >> 1];
          af[j][s] = deq_frag8(v[(s & 1) * 2], v[(s & 1) * 2 + 1], sb.s[j], sb.b[j]);
        }
      }
    };
    auto read_x = [&](bf16x8 (&xf)[RT], int st, int s) {
#pragma unroll
      for (int i = 0; i < RT; ++i)
        xf[i] = *reinterpret_cast<const bf16x8*>(stage(st) + xfo[s] + i * 4096);
    };
    auto mfmas = [&](const bf16x8 (&af)[JT][4], const bf16x8 (&xf)[RT], int s) {
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < JT; ++j)
          acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[j][s], xf[i], acc[j][i], 0, 0, 0);
    };

#pragma unroll
    for (int j = 0; j < JT; ++j)
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[j][i][r] = 0.f;

    // Prologue: steps kb .. kb + 2 in flight, step kb dequantized and its first
    // x fragments read.
    load_sb(sbA, kb);
    issue(kb, 0, 0);
    issue(kb + 1, 1, 1);
    issue(kb + 2, 2, 2);
    __builtin_amdgcn_s_waitcnt(wait_enc(XI + 2 * NV, 15));  // step kb's weights
    {
      const SB sb0 = scale_bias(sbA, 0);
#pragma unroll
      for (int s = 0; s < 4; ++s) dequant(af0, 0, sb0, s);
    }
    __builtin_amdgcn_s_waitcnt(wait_enc(2 * NV, 15));  // step kb's x
    __builtin_amdgcn_s_barrier();
    read_x(xf0, 0, 0);

    // Step k (stage / weight set j = (k - kb) % 4): wait for step k + 1's loads,
    // issue step k + 3's, dequantize step k + 1 across the sub-steps, run the
    // MFMAs.  The barrier sits before the last sub-step's MFMAs: every wave has
    // then read its last fragments of stage j (the next step's DMA refills it)
    // and waited for its share of stage j + 1 (read right after it).
    auto step = [&](int k, auto jc, auto tc, bf16x8 (&ac)[JT][4], bf16x8 (&an)[JT][4]) {
      constexpr int j = decltype(jc)::value;
      // Outstanding: the loads of steps k + 1 (issued two steps back) and k + 2.
      // Wait for step k + 1's weights (its x DMA and step k + 2's loads may stay
      // in flight); its x is waited for before the barrier.  In the piece's last
      // pass (tail) steps k + 2, k + 3 past the end issued nothing, so fewer
      // loads may stay in flight: after step k + 1's x come only step ke - 4's
      // loads (j = 1), or none (j >= 2).
      constexpr bool tail = decltype(tc)::value;
      constexpr int nv_prev = j == 1 ? NV0 : NV, nv_cur = j == 0 ? NV0 : NV;
      constexpr int wait_w = !tail || j <= 1 ? XI + nv_prev : j == 2 ? XI : 0;
      constexpr int wait_x = !tail || j == 0 ? nv_prev + nv_cur : j == 1 ? nv_prev : 0;
      __builtin_amdgcn_s_waitcnt(wait_enc(wait_w, 15));
      if constexpr (j == 0) load_sb(sbB, k + 4);
      issue(k + 3, (j + 3) & 3, (j + 3) & 3);
      const int dn = (j + 1) & 3;
      const SB sb = scale_bias(j == 3 ? sbB : sbA, (j + 1) & 3);
      read_x(xf1, j, 1);
      mfmas(ac, xf0, 0);
      dequant(an, dn, sb, 0);
      read_x(xf0, j, 2);
      mfmas(ac, xf1, 1);
      dequant(an, dn, sb, 1);
      read_x(xf1, j, 3);
      mfmas(ac, xf0, 2);
      dequant(an, dn, sb, 2);
      // Per MFMA: the next sub-step's fragment reads (and in sub-step 0 this
      // step's loads) and a share of the dequantization's VALU work, so it runs
      // under the MFMAs instead of between them.  Before the barrier, step
      // k + 1's x DMA (issued two steps back) must have landed.
#pragma unroll
      for (int t = 0; t < 3 * RT * JT; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        if (t < NV + 2) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
        if ((t % (RT * JT)) < RT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        __builtin_amdgcn_sched_group_barrier(0x002, 3 * 8 / RT, 0);   // VALU
      }
      __builtin_amdgcn_s_waitcnt(wait_enc(wait_x, 0));
      __builtin_amdgcn_s_barrier();
      read_x(xf0, (j + 1) & 3, 0);
      mfmas(ac, xf1, 3);
      dequant(an, dn, sb, 3);
#pragma unroll
      for (int t = 0; t < RT * JT; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (t < RT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3 * 8 / RT, 0);
      }
    };
    // Piece lengths are multiples of 4 steps (qmm_wide_plan), so the stages and
    // weight sets rotate with a period of one loop pass.
    auto pass = [&](int k, auto tc) {
      step(k, std::integral_constant<int, 0>{}, tc, af0, af1);
      step(k + 1, std::integral_constant<int, 1>{}, tc, af1, af0);
      step(k + 2, std::integral_constant<int, 2>{}, tc, af0, af1);
      step(k + 3, std::integral_constant<int, 3>{}, tc, af1, af0);
#pragma unroll
      for (int q = 0; q < 4; ++q) sbA[q] = sbB[q];
    };
    int k = kb;
    for (; k + 4 < ke; k += 4) pass(k, std::false_type{});
    pass(k, std::true_type{});
    __builtin_amdgcn_s_waitcnt(wait_enc(0, 15));

    // Partial slots hold a tile's fp32 sums in register order: 16-byte piece
    // (j, i, g) of thread t at ((j 8 + i) 4 + g) T + t, so every store and load
    // instruction of a wave covers 1 KiB.
    auto piece = [&](int j, int i, int g) { return ((((j * RT + i) * 4 + g) * T) + tid) * 16; };
    if (role == kContrib) {
      // fp32 partial to this block's slot with agent-coherent stores (sc1), then
      // bump the tile's counter.
      const __amdgpu_buffer_rsrc_t pres = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(a.ws + (int64_t)b * BM * kT), (short)0, BM * kT * 4, 0x00020000);
#pragma unroll
      for (int j = 0; j < JT; ++j)
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const f32x4 v = {acc[j][i][4 * g], acc[j][i][4 * g + 1], acc[j][i][4 * g + 2],
                             acc[j][i][4 * g + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), pres, piece(j, i, g),
                                                   0, 16 /* sc1 */);
          }
      __builtin_amdgcn_s_waitcnt(wait_enc(0, 15));
      __syncthreads();
      if (tid == 0)
        __hip_atomic_fetch_add(a.tile_count + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      continue;
    }
    int c_lo = 0, c_hi = 0;  // partial slots to add (FINAL)
    if (role == kFinal) {
      const uint32_t need = (uint32_t)(b - first);
      if (tid == 0) {
        uint32_t spins = 0, ok = 1;
        while (__hip_atomic_load(a.tile_count + tile, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
               need) {
          __builtin_amdgcn_s_sleep(2);
          if (++spins > (1u << 24)) {  // a bound on the wait: flag it and go on
            ok = 0;
            break;
          }
        }
        s_flag = ok;
        if (!ok) atomicOr(wa.err, 2u);
        __hip_atomic_store(a.tile_count + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (s_flag) {
        c_lo = first;
        c_hi = b;
      }
    }
    // y = bf16(acc), then the optional additive bias as a second bf16 add (the
    // qlinear-then-add chain, compute/models/quant.go:105-111).  The tile goes
    // out through LDS one 32-row group at a time, so that every store instruction
    // writes whole 512-byte row segments (a lane's own outputs are 4 values on
    // each of 32 rows).  Lane values: x row m0 + 32 i + r32, outputs
    // n0 + wcol + 32 j + 8 g + 4 h .. + 3.  Chunk rows are 512 bytes of 16-byte
    // units, unit u of row r at position u ^ r.  The stages are free: every wave
    // has drained its DMA (vmcnt(0) above), and the barrier orders the other
    // waves' last fragment reads and DMA before the first chunk write.
    __builtin_amdgcn_s_waitcnt(wait_enc(0, 0));
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      // Partials of the FINAL piece, one row group at a time (a whole slot's
      // loads at once would not fit the registers beside the accumulators).
      for (int c = c_lo; c < c_hi; ++c) {
        const __amdgpu_buffer_rsrc_t pres = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(a.ws + (int64_t)c * BM * kT), (short)0, BM * kT * 4, 0x00020000);
        f32x4 part[JT][4];
#pragma unroll
        for (int j = 0; j < JT; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            part[j][g] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(pres, piece(j, i, g), 0, 16 /* sc1 */));
#pragma unroll
        for (int j = 0; j < JT; ++j)
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[j][i][4 * g + e] += part[j][g][e];
      }
      uint8_t* chunk = stage(i & 1);
#pragma unroll
      for (int j = 0; j < JT; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int u = wcol / 8 + 4 * j + g;
          *reinterpret_cast<u32x2*>(chunk + r32 * 512 + ((u ^ r32) << 4) + 8 * h) =
              u32x2{pack_bf16x2(acc[j][i][4 * g], acc[j][i][4 * g + 1]),
                    pack_bf16x2(acc[j][i][4 * g + 2], acc[j][i][4 * g + 3])};
        }
      __syncthreads();
      // Rows 4 wave + 2 q + h of the chunk, lane r32 taking outputs n0 + 8 r32 ..
      // + 7.  (The next write to this buffer comes after the next chunk's
      // barrier, which every wave reaches only after these reads.)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int R = 4 * (wave & 7) + 2 * q + h;
        u32x4 v = *reinterpret_cast<const u32x4*>(chunk + R * 512 + ((r32 ^ R) << 4));
        const int64_t m = m0 + 32 * i + R, n = n0 + 8 * r32;
        if (m < a.M && n < a.N) {
          if (a.bias) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              v[e] = pack_bf16x2(bf16_lo(v[e]) + bf16_bits_to_f32(a.bias[n + 2 * e]),
                                 bf16_hi(v[e]) + bf16_bits_to_f32(a.bias[n + 2 * e + 1]));
          }
          *reinterpret_cast<u32x4*>(a.y + m * a.ldy + n) = v;
        }
      }
    }
    // The next item's DMA refills the stages: every wave has read its rows.
    __syncthreads();
  }
}

}  // namespace

WidePlan qmm_wide_plan(int64_t M, int64_t N, int64_t K, int cus) {
  WidePlan p{};
  // 256-row x tiles while they fill half the chip (stream-K then cuts each tile
  // in at most two); otherwise 128-row tiles, which double the tiles (each
  // weight is dequantized twice as often) rather than cut every tile's K range
  // into more pieces.
  const int64_t tn = (N + kT - 1) / kT;
  p.bm = 2 * ((M + 255) / 256) * tn >= cus ? 256 : 128;

  p.tm = (int)((M + p.bm - 1) / p.bm);
  const int64_t tiles = (int64_t)p.tm * tn;
  p.nk = (int)(K / kS);
  p.blocks = cus;
  p.dp = (int)(tiles / cus);
  // Tiles filling at least 7/8 of the CUs but not all of them: one whole tile
  // per block, no stream-K.  Pieces of tiles * nk / cus steps would cut nearly
  // every tile in two, each cut costing a partial's round trip and a wait
  // (14336x4096 at M = 512, 224 tiles on 256 CUs: 4-bit 73-77 -> 63-67 us, 8-bit
  // 92-95 -> 73 us).
  if (p.dp == 0 && tiles * 8 >= (int64_t)cus * 7) {
    p.dp = 1;
    p.blocks = (int)tiles;
    p.sk_iters = 0;
    p.sk_len = 0;
    p.tiles = tiles;
    p.ws_floats = 0;
    return p;
  }
  const int64_t rest = tiles % cus;
  p.sk_iters = rest * p.nk;
  p.sk_len = 0;
  if (rest > 0) {
    int64_t len = (p.sk_iters + cus - 1) / cus;
    if (len < kWideMinPiece) len = kWideMinPiece < p.nk ? kWideMinPiece : p.nk;
    len = (len + 3) & ~(int64_t)3;  // whole passes of four steps (nk is a multiple of 4)
    p.sk_len = (int)len;
    if (p.dp == 0) p.blocks = (int)((p.sk_iters + len - 1) / len);
  }
  p.tiles = tiles;
  p.ws_floats = p.sk_len > 0 ? (int64_t)p.blocks * p.bm * kT : 0;
  return p;
}

bool qmm_wide_supported(const QmmArgs& a) {
  return a.M >= 1 && a.N >= 1 && a.K % (4 * kS) == 0 && a.K > 0 && a.ldx % 8 == 0 &&
         // 16-byte output stores of 8 outputs
         a.N % 8 == 0 && a.ldy % 8 == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 &&
         (a.bits == 4 || a.bits == 8) && a.group_size == kS && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(a.w) & 15) == 0 &&
         // buffer resources count bytes in 32 bits: x per tile, w / scales / biases whole
         kT * a.ldx * 2 < ((int64_t)1 << 31) && a.N * (a.K * a.bits / 8) < ((int64_t)1 << 31) &&
         a.N * (a.K / a.group_size) * 2 < ((int64_t)1 << 31);
}

hipError_t launch_qmm_wide(const QmmArgs& a, const WidePlan& p, uint32_t* err, hipStream_t stream) {
  if (!qmm_wide_supported(a) || p.blocks < 1 || (p.bm != 128 && p.bm != 256))
    return hipErrorInvalidValue;
  if (p.sk_len > 0 && (!a.ws || !a.tile_count || !err)) return hipErrorInvalidValue;
  WideArgs wa{a, p.tm, p.nk, p.dp, p.sk_len, p.sk_iters, err};
  constexpr int W = kWideWaves;
  const dim3 grid((unsigned)p.blocks), block(W * 64);
  if (p.bm == 256) {
    if (a.bits == 4) qmm_wide_kernel<4, W, 256><<<grid, block, 0, stream>>>(wa);
    else qmm_wide_kernel<8, W, 256><<<grid, block, 0, stream>>>(wa);
  } else {
    if (a.bits == 4) qmm_wide_kernel<4, W, 128><<<grid, block, 0, stream>>>(wa);
    else qmm_wide_kernel<8, W, 128><<<grid, block, 0, stream>>>(wa);
  }
  return hipGetLastError();
}

}  // namespace fmxq
