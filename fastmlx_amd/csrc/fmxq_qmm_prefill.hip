// fmxq_qmm_prefill.hip -- MFMA GEMM for quantized_matmul at verify and prefill sizes (M > 32,
// and the 5 <= M <= 32 shapes no GEMV kernel takes).
//
// Replaces the GEMM side of mlx_quantized_matmul (mlxgo/binding_cgo.go:636-643)
// for x [M, K] with M = batch * seq rows (prefill at batch_generator.go:258).
//
// Block tile BM x BN over 64-deep K steps, 8 waves in a WM x WN grid (two waves
// per SIMD), each wave owning a (BM/WM) x (BN/WN) patch of
// v_mfma_f32_32x32x16_bf16 tiles.  Per step the block
//   - copies the x tile (BM rows x 128 bytes) global -> LDS with buffer_load ...
//     lds (no VGPR staging), two steps ahead, into one of three x stages;
//   - loads the packed weight tile two steps ahead into registers and, one step
//     later, dequantizes it into one of two bf16 weight stages in LDS:
//     w = bf16(s * q + b), for 4-bit one v_cvt_f32_ubyteN and one fma per value
//     (the exact s*q + b rounded once to fp32);
//   - runs its MFMAs from LDS in four k16 sub-steps, fragments read one
//     sub-step ahead.
// One barrier per step.  Before it each wave waits only for the loads issued one
// step earlier, so this step's loads stay in flight across it; the barrier sits
// before the last sub-step's MFMAs so those overlap the next step's first
// fragment reads.
//
// LDS rows are 128 bytes (64 bf16 along K) with 16-byte chunk c of row r stored
// at position c ^ swz(r): 32 consecutive rows read at one chunk hit distinct
// banks both as 8 rows per 128 bytes and as 16 rows per 256 bytes.
//
// The MFMA A operand is the weight fragment and B the x fragment, so a lane
// holds 4 consecutive output columns of one row and stores them as 8 bytes.
#include "fmxq_common.hpp"
#include "fmxq_internal.hpp"

namespace fmxq {
namespace {

typedef __attribute__((address_space(3))) void lds_t;

constexpr int kStepK = 64;

__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding, expcnt left alone).
#define FMXQ_WAIT_VM_LGKM0(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4))

// One 4-bit word (values q0..q7, least significant first) -> bf16 pairs
// (w0,w1) (w2,w3) (w4,w5) (w6,w7) of w = bf16(fma(s, q, b)): the exact s*q + b
// rounded once to fp32, then to bf16.  The nibbles are split into two byte
// vectors (q0 q2 q4 q6 and q1 q3 q5 q7) and converted with v_cvt_f32_ubyteN
// (written out: the compiler turns the byte extracts into bfe + ubyte0);
// each fma writes a fresh register, where v_dot2c (which accumulates into its
// destination) would need a copy of the shared addend before every use.
template <int K>
__device__ __forceinline__ float ubyte_to_f32(uint32_t v) {
  float f;
  if constexpr (K == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(v));
  else if constexpr (K == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(v));
  else if constexpr (K == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(v));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(v));
  return f;
}
__device__ __forceinline__ void dequant_word4(uint32_t w, float s, float b, uint32_t* out) {
  const uint32_t e = w & 0x0F0F0F0Fu, o = (w >> 4) & 0x0F0F0F0Fu;
  out[0] = pack_bf16x2(__builtin_fmaf(s, ubyte_to_f32<0>(e), b), __builtin_fmaf(s, ubyte_to_f32<0>(o), b));
  out[1] = pack_bf16x2(__builtin_fmaf(s, ubyte_to_f32<1>(e), b), __builtin_fmaf(s, ubyte_to_f32<1>(o), b));
  out[2] = pack_bf16x2(__builtin_fmaf(s, ubyte_to_f32<2>(e), b), __builtin_fmaf(s, ubyte_to_f32<2>(o), b));
  out[3] = pack_bf16x2(__builtin_fmaf(s, ubyte_to_f32<3>(e), b), __builtin_fmaf(s, ubyte_to_f32<3>(o), b));
}
// Two 8-bit words (values e0..e7) -> 4 bf16 pairs of w = s*q + b.
__device__ __forceinline__ void dequant_words8(uint32_t w0, uint32_t w1, float s, float b,
                                               uint32_t* out) {
  out[0] = pack_bf16x2(__builtin_fmaf(s, (float)(w0 & 0xffu), b),
                       __builtin_fmaf(s, (float)((w0 >> 8) & 0xffu), b));
  out[1] = pack_bf16x2(__builtin_fmaf(s, (float)((w0 >> 16) & 0xffu), b),
                       __builtin_fmaf(s, (float)(w0 >> 24), b));
  out[2] = pack_bf16x2(__builtin_fmaf(s, (float)(w1 & 0xffu), b),
                       __builtin_fmaf(s, (float)((w1 >> 8) & 0xffu), b));
  out[3] = pack_bf16x2(__builtin_fmaf(s, (float)((w1 >> 16) & 0xffu), b),
                       __builtin_fmaf(s, (float)(w1 >> 24), b));
}

template <int BITS, int BM, int BN, int WM, int WN>
struct PrefillTile {
  static constexpr int T = WM * WN * 64;                 // threads
  static constexpr int WTM = BM / WM, WTN = BN / WN;     // wave patch
  static constexpr int TM = WTM / 32, TN = WTN / 32;     // 32x32 tiles per wave
  // A weight unit is UW words (16 or 8 bytes) of one row; each thread owns BU
  // units per step.
  static constexpr int UW = (BN * (kStepK * BITS / 128) >= T) ? 4 : 2;
  static constexpr int CHU = UW * 32 / BITS;             // values per unit
  static constexpr int UPR = kStepK / CHU;               // units per row
  static constexpr int BU = BN * UPR / T;
  static constexpr int NWD = BITS == 4 ? UW : UW / 2;    // 16-byte chunks per unit
  static constexpr int AI = BM * 128 / 1024 / (T / 64);  // x DMA instructions per wave
  static constexpr int NV = AI + 3 * BU;                 // loads each thread issues per step
  static_assert(WM * WN == 8, "8 waves");
  static_assert(BU >= 1 && BN * UPR == BU * T, "weight units");
  static_assert(AI >= 1 && AI * (T / 64) * 1024 == BM * 128, "x DMA split");
  static_assert(TM >= 1 && TN >= 1, "wave patch");
  static_assert(3 * BM * 128 + 2 * BN * 128 <= 160 * 1024, "LDS budget");
};

template <int BITS, int BM, int BN, int WM, int WN, bool GR = false>
__global__ __launch_bounds__(WM * WN * 64, 1) void qmm_prefill_kernel(QmmArgs a) {
  using P = PrefillTile<BITS, BM, BN, WM, WN>;
  constexpr int T = P::T, TM = P::TM, TN = P::TN, UW = P::UW, BU = P::BU, AI = P::AI;
  constexpr int NWD = P::NWD;
  // Three x stages and two weight stages, each its own LDS object so the
  // compiler can tell reads of one stage from the DMA into another.
  __shared__ __attribute__((aligned(1024))) uint8_t xs0[BM * 128];
  __shared__ __attribute__((aligned(1024))) uint8_t xs1[BM * 128];
  __shared__ __attribute__((aligned(1024))) uint8_t xs2[BM * 128];
  __shared__ __attribute__((aligned(1024))) uint8_t ws0[BN * 128];
  __shared__ __attribute__((aligned(1024))) uint8_t ws1[BN * 128];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;

  // Block -> tile and K range.  Blocks [0, full) take whole tiles; they are dealt
  // to the 8 XCDs round robin, so consecutive tiles (M fastest) go to one XCD and
  // its resident blocks share weight rows through its L2.  With a.splits > 1 the
  // last a.split_tail tiles are cut into a.splits K ranges, one block each, which
  // write fp32 partials to a.ws for prefill_fixup_kernel (they are dispatched
  // last, so a part-full last wave of whole tiles becomes a full wave of parts).
  const int64_t wpr = a.K * BITS / 32;
  const int gshift = __builtin_ctz((unsigned)a.group_size);
  const int64_t gpr = a.K >> gshift;
  const int nk_all = (int)(a.K / kStepK);
  int64_t t = blockIdx.x, full = 0, m0 = 0, n0 = 0;
  int part = -1;
  // Grouped form: one work-list tile (slots g_start .. + g_len of expert g_e) by
  // one N tile.
  int64_t g_start = 0, g_len = 0, g_e = 0;
  if constexpr (GR) {
    const int64_t tile = blockIdx.y;
    if (tile >= (int64_t)*a.g_ntile) return;
    g_start = a.g_tiles[2 * tile];
    g_len = a.g_tiles[2 * tile + 1];
    g_e = a.g_rhs[g_start];
    n0 = (int64_t)blockIdx.x * BN;
  } else {
    const int nt_m = (int)((a.M + BM - 1) / BM);
    const int64_t tiles = (int64_t)nt_m * ((a.N + BN - 1) / BN);
    full = tiles - (a.splits > 1 ? a.split_tail : 0);
    if (t < full) {
      if ((full & 7) == 0) t = (t & 7) * (full >> 3) + (t >> 3);
    } else {
      const int64_t r = t - full;
      t = full + r / a.splits;
      part = (int)(r % a.splits);
    }
    m0 = (int64_t)(t % nt_m) * BM;
    n0 = (int64_t)(t / nt_m) * BN;
  }
  const int kb = part < 0 ? 0 : (int)((int64_t)part * nk_all / a.splits);  // first step
  const int nk = part < 0 ? nk_all : (int)((int64_t)(part + 1) * nk_all / a.splits) - kb;

  // x rows through a buffer resource: rows past M (or a grouped slot's row past
  // g_xrows) read as zero.
  const int64_t rows_here = GR ? a.g_xrows : (a.M - m0 < BM ? a.M - m0 : BM);
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.x + m0 * a.ldx), (short)0, (int)(rows_here * a.ldx * 2), 0x00020000);
  // DMA instruction j of this wave fills rows 8 (wave AI + j) .. +8 of a stage:
  // lane L lands at row + L/8, position L%8, so it fetches chunk (L%8) ^ swz(row).
  // Grouped: the row is tile slot g_start + row (slots past the tile repeat its
  // first), whose x row comes from g_rows.
  uint32_t aoff[AI];
#pragma unroll
  for (int j = 0; j < AI; ++j) {
    const int row = 8 * (wave * AI + j) + (lane >> 3);
    const int c = (lane & 7) ^ swz(row);
    if constexpr (GR) {
      const int64_t slot = g_start + (row < g_len ? row : 0);
      const int64_t xr = a.g_rows ? (int64_t)a.g_rows[slot] : slot;
      aoff[j] = (uint32_t)((xr < a.g_xrows ? xr : a.g_xrows) * a.ldx * 2 + c * 16);
    } else {
      aoff[j] = (uint32_t)((row * a.ldx + c * 8) * 2);
    }
  }

  // Weights, scales and biases through buffer resources: a thread's offset is
  // fixed and each step adds one wave-uniform offset (no per-step 64-bit address
  // arithmetic).  qmm_prefill_supported keeps every byte offset below 2^31.
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.w + g_e * a.N * wpr), (short)0, (int)(a.N * wpr * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.scales + g_e * a.N * gpr), (short)0, (int)(a.N * gpr * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.biases + g_e * a.N * gpr), (short)0, (int)(a.N * gpr * 2), 0x00020000);
  uint32_t wvo[BU], svo[BU];
  int u_row[BU], u_idx[BU];
#pragma unroll
  for (int i = 0; i < BU; ++i) {
    const int q = tid + T * i;
    u_row[i] = q / P::UPR;
    u_idx[i] = q % P::UPR;
    int64_t n = n0 + u_row[i];
    if (n > a.N - 1) n = a.N - 1;  // rows past N load row N-1; their outputs are not stored
    wvo[i] = (uint32_t)((n * wpr + u_idx[i] * UW) * 4);
    // Group of the unit: (64 kt + u_idx CHU) >> gshift.  A 64-deep step lies in one
    // group when group_size >= 64; with group_size 32 the unit's half is fixed.
    const int gadd = a.group_size == 32 ? (u_idx[i] * P::CHU) >> 5 : 0;
    svo[i] = (uint32_t)((n * gpr + gadd) * 2);
  }

  typedef uint32_t uvec __attribute__((ext_vector_type(UW)));
  auto issue_x = [&](int kt, uint8_t* xs) {
    kt = kb + (kt < nk ? kt : nk - 1);
    const int soff = kt * kStepK * 2;
#pragma unroll
    for (int j = 0; j < AI; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (lds_t*)(xs + (wave * AI + j) * 1024), 16,
                                               (int)aoff[j], soff, 0, 0);
  };
  auto load_w = [&](int kt, uvec* wq, uint32_t* sq, uint32_t* bq) {
    kt = kb + (kt < nk ? kt : nk - 1);
    const int wso = kt * (kStepK * BITS / 8);          // bytes of packed words per step
    const int sso = ((kt * kStepK) >> gshift) * 2;     // first group of the step
#pragma unroll
    for (int i = 0; i < BU; ++i) {
      if constexpr (UW == 2)
        wq[i] = __builtin_bit_cast(uvec, __builtin_amdgcn_raw_buffer_load_b64(wres, (int)wvo[i],
                                                                              wso, 2 /* nt */));
      else
        wq[i] = __builtin_bit_cast(uvec, __builtin_amdgcn_raw_buffer_load_b128(wres, (int)wvo[i],
                                                                               wso, 2 /* nt */));
      sq[i] = __builtin_amdgcn_raw_buffer_load_b16(sres, (int)svo[i], sso, 0);
      bq[i] = __builtin_amdgcn_raw_buffer_load_b16(bres, (int)svo[i], sso, 0);
    }
  };
  // Dequantize chunk v of every unit of this thread into weight stage ws.
  auto store_chunk = [&](uint8_t* ws, const uvec* wq, const uint32_t* sq, const uint32_t* bq, int v) {
#pragma unroll
    for (int i = 0; i < BU; ++i) {
      const int r = u_row[i];
      uint32_t d[4];
      if constexpr (BITS == 4) {
        dequant_word4(wq[i][v], bf16_bits_to_f32(sq[i]), bf16_bits_to_f32(bq[i]), d);
      } else {
        dequant_words8(wq[i][2 * v], wq[i][2 * v + 1], bf16_bits_to_f32(sq[i]),
                       bf16_bits_to_f32(bq[i]), d);
      }
      const int ch = u_idx[i] * NWD + v;
      *reinterpret_cast<u32x4*>(ws + r * 128 + ((ch ^ swz(r)) << 4)) = u32x4{d[0], d[1], d[2], d[3]};
    }
  };

  // Fragment offsets: row (lane % 32) of each 32-row tile, chunk 2 s + lane / 32.
  const int fr = lane & 31, fh = lane >> 5;
  uint32_t xro[4], wro[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int rx = wm * P::WTM + fr, rw = wn * P::WTN + fr;
    xro[s] = rx * 128 + (((2 * s + fh) ^ swz(rx)) << 4);
    wro[s] = rw * 128 + (((2 * s + fh) ^ swz(rw)) << 4);
  }

  // acc[i][j]: lane l holds output row 32 i + l % 32 of the wave patch and, in
  // register r, column 32 j + 8 (r / 4) + 4 (l / 32) + r % 4.
  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  auto read_frags = [&](const uint8_t* xs, const uint8_t* ws, int s, bf16x8* xf, bf16x8* wf) {
#pragma unroll
    for (int i = 0; i < TM; ++i) xf[i] = *reinterpret_cast<const bf16x8*>(xs + xro[s] + i * 32 * 128);
#pragma unroll
    for (int j = 0; j < TN; ++j) wf[j] = *reinterpret_cast<const bf16x8*>(ws + wro[s] + j * 32 * 128);
  };
  auto mfmas = [&](const bf16x8* xf, const bf16x8* wf) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j], xf[i], acc[i][j], 0, 0, 0);
  };

  uvec w0[BU], w1[BU];
  uint32_t s0[BU], s1[BU], b0[BU], b1[BU];
  bf16x8 xf0[TM], wf0[TN], xf1[TM], wf1[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) xf1[i] = bf16x8{};
#pragma unroll
  for (int j = 0; j < TN; ++j) wf1[j] = bf16x8{};

  auto dequant_part = [&](uint8_t* ws, const uvec* wq, const uint32_t* sq, const uint32_t* bq,
                          int part) {
#pragma unroll
    for (int v = 0; v < NWD; ++v)
      if (v * 3 / NWD == part) store_chunk(ws, wq, sq, bq, v);
  };
  // Step kt reads x stage kt%3 and weight stage kt%2.  It loads the weights of
  // step kt+2 into register set kt%2, DMAs the x of step kt+2 into stage
  // (kt+2)%3 and dequantizes the weights of step kt+1 (register set (kt+1)%2,
  // loaded one step earlier) into weight stage (kt+1)%2 across sub-steps 0..2.
  // The first step's "previous" MFMAs run on zero fragments.  sched_barrier
  // keeps each sub-step's fragment reads ahead of the MFMAs they feed.
  auto step = [&](const uint8_t* xr, const uint8_t* wr, uint8_t* xn, uint8_t* wn_, int kt,
                  uvec* wl, uint32_t* sl, uint32_t* bl, const uvec* wd_in,
                  const uint32_t* sd_in, const uint32_t* bd_in) {
    read_frags(xr, wr, 0, xf0, wf0);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(xf1, wf1);
    load_w(kt + 2, wl, sl, bl);
    issue_x(kt + 2, xn);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(xr, wr, 1, xf1, wf1);
    __builtin_amdgcn_sched_barrier(0);
    // The empty asm keeps arithmetic on the weights loaded one step earlier from
    // being hoisted up to their loads, which would wait for them too early.
    uvec wd[BU];
    uint32_t sd[BU], bd[BU];
#pragma unroll
    for (int i = 0; i < BU; ++i) {
      wd[i] = wd_in[i];
      sd[i] = sd_in[i];
      bd[i] = bd_in[i];
      asm volatile("" : "+v"(wd[i]), "+v"(sd[i]), "+v"(bd[i]));
    }
    mfmas(xf0, wf0);
    dequant_part(wn_, wd, sd, bd, 0);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(xr, wr, 2, xf0, wf0);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(xf1, wf1);
    dequant_part(wn_, wd, sd, bd, 1);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(xr, wr, 3, xf1, wf1);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(xf0, wf0);
    dequant_part(wn_, wd, sd, bd, 2);
    FMXQ_WAIT_VM_LGKM0(P::NV);
    __builtin_amdgcn_s_barrier();
  };

  issue_x(0, xs0);
  issue_x(1, xs1);
  load_w(0, w0, s0, b0);
  load_w(1, w1, s1, b1);
  FMXQ_WAIT_VM_LGKM0(0);
#pragma unroll
  for (int v = 0; v < NWD; ++v) store_chunk(ws0, w0, s0, b0, v);
  FMXQ_WAIT_VM_LGKM0(0);
  __builtin_amdgcn_s_barrier();

  // Six steps per iteration so every stage and register set is a fixed name.
#define FMXQ_STEP(j)                                                                         \
  step((j) % 3 == 0 ? xs0 : (j) % 3 == 1 ? xs1 : xs2, (j) % 2 ? ws1 : ws0,                   \
       ((j) + 2) % 3 == 0 ? xs0 : ((j) + 2) % 3 == 1 ? xs1 : xs2, (j) % 2 ? ws0 : ws1, kt + (j), \
       (j) % 2 ? w1 : w0, (j) % 2 ? s1 : s0, (j) % 2 ? b1 : b0, (j) % 2 ? w0 : w1,             \
       (j) % 2 ? s0 : s1, (j) % 2 ? b0 : b1)
  int kt = 0;
  for (; kt + 6 <= nk; kt += 6) {
    FMXQ_STEP(0); FMXQ_STEP(1); FMXQ_STEP(2); FMXQ_STEP(3); FMXQ_STEP(4); FMXQ_STEP(5);
  }
  switch (nk - kt) {
    case 5: FMXQ_STEP(0); FMXQ_STEP(1); FMXQ_STEP(2); FMXQ_STEP(3); FMXQ_STEP(4); break;
    case 4: FMXQ_STEP(0); FMXQ_STEP(1); FMXQ_STEP(2); FMXQ_STEP(3); break;
    case 3: FMXQ_STEP(0); FMXQ_STEP(1); FMXQ_STEP(2); break;
    case 2: FMXQ_STEP(0); FMXQ_STEP(1); break;
    case 1: FMXQ_STEP(0); break;
    default: break;
  }
#undef FMXQ_STEP
  mfmas(xf1, wf1);

  if (part >= 0) {
    // fp32 partial of this K range into slot ((t - full) * splits + part) of the
    // workspace, BM x BN row-major; the fixup kernel sums the parts of a tile.
    float* wsp = a.ws + ((t - full) * a.splits + part) * (int64_t)(BM * BN);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int r = wm * P::WTM + fr + 32 * i;
          const int c = wn * P::WTN + j * 32 + 8 * g + 4 * fh;
          *reinterpret_cast<f32x4*>(wsp + r * BN + c) =
              f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                    acc[i][j][4 * g + 3]};
        }
    return;
  }

  // Epilogue: bf16 (round to nearest even), then the optional additive bias as a
  // second bf16 add (the qlinear-then-add chain, compute/models/quant.go:105-111).
  const bool fast = ((a.ldy & 3) == 0) && ((reinterpret_cast<uintptr_t>(a.y) & 7) == 0);
  const int64_t m_l = m0 + wm * P::WTM + fr;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    int64_t m = m_l + i * 32;
    bool zero = false;
    if constexpr (GR) {
      if (m >= g_len) continue;
      const int64_t slot = g_start + m;
      const int64_t xr = a.g_rows ? (int64_t)a.g_rows[slot] : slot;
      zero = xr >= a.g_xrows;
      if (zero && fh == 0 && n0 + wn * P::WTN == 0) atomicOr(a.g_flag, 1u);
      m = a.g_yrow ? (int64_t)a.g_yrow[slot] : slot;
    } else {
      if (m >= a.M) continue;
    }
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t n = n0 + wn * P::WTN + j * 32 + 8 * g + 4 * fh;
        if (n >= a.N) continue;
        uint32_t p0 = zero ? 0u : pack_bf16x2(acc[i][j][4 * g], acc[i][j][4 * g + 1]);
        uint32_t p1 = zero ? 0u : pack_bf16x2(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
        if (a.bias && !zero) {
          float bv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) bv[e] = n + e < a.N ? bf16_bits_to_f32(a.bias[n + e]) : 0.f;
          p0 = pack_bf16x2(bf16_lo(p0) + bv[0], bf16_hi(p0) + bv[1]);
          p1 = pack_bf16x2(bf16_lo(p1) + bv[2], bf16_hi(p1) + bv[3]);
        }
        uint16_t* dst = a.y + m * a.ldy + n;
        if (fast && n + 3 < a.N) {
          *reinterpret_cast<u32x2*>(dst) = u32x2{p0, p1};
        } else {
          const uint16_t v[4] = {(uint16_t)p0, (uint16_t)(p0 >> 16), (uint16_t)p1,
                                 (uint16_t)(p1 >> 16)};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n + e < a.N) dst[e] = v[e];
        }
      }
  }
}

// Sums the a.splits fp32 partials of each split tile and stores it like the
// main epilogue (bf16, then the optional bias add rounded again).  One thread per
// 4 consecutive columns of a tile row.
template <int BM, int BN>
__global__ __launch_bounds__(256) void prefill_fixup_kernel(QmmArgs a) {
  const int nt_m = (int)((a.M + BM - 1) / BM);
  const int64_t tiles = (int64_t)nt_m * ((a.N + BN - 1) / BN);
  const int64_t full = tiles - a.split_tail;
  constexpr int Q = BM * BN / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.split_tail * Q) return;
  const int64_t tt = idx / Q;
  const int e = (int)(idx % Q) * 4;
  const int64_t t = full + tt;
  const int64_t m = (t % nt_m) * BM + e / BN, n = (t / nt_m) * BN + e % BN;
  if (m >= a.M || n >= a.N) return;
  // Every part is loaded before the first add (one round trip, not one per
  // part); the sum runs in part order.
  f32x4 part[kPrefillMaxSplits];
#pragma unroll
  for (int sp = 0; sp < kPrefillMaxSplits; ++sp)
    if (sp < a.splits)
      part[sp] = *reinterpret_cast<const f32x4*>(a.ws + (tt * a.splits + sp) * (int64_t)(BM * BN) + e);
  f32x4 v = {};
#pragma unroll
  for (int sp = 0; sp < kPrefillMaxSplits; ++sp)
    if (sp < a.splits) v += part[sp];
  uint32_t p0 = pack_bf16x2(v[0], v[1]), p1 = pack_bf16x2(v[2], v[3]);
  if (a.bias) {
    float bv[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) bv[k] = n + k < a.N ? bf16_bits_to_f32(a.bias[n + k]) : 0.f;
    p0 = pack_bf16x2(bf16_lo(p0) + bv[0], bf16_hi(p0) + bv[1]);
    p1 = pack_bf16x2(bf16_lo(p1) + bv[2], bf16_hi(p1) + bv[3]);
  }
  uint16_t* dst = a.y + m * a.ldy + n;
  const bool fast = ((a.ldy & 3) == 0) && ((reinterpret_cast<uintptr_t>(a.y) & 7) == 0);
  if (fast && n + 3 < a.N) {
    *reinterpret_cast<u32x2*>(dst) = u32x2{p0, p1};
  } else {
    const uint16_t w[4] = {(uint16_t)p0, (uint16_t)(p0 >> 16), (uint16_t)p1, (uint16_t)(p1 >> 16)};
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (n + k < a.N) dst[k] = w[k];
  }
}

template <int BITS, int BM, int BN, int WM, int WN>
hipError_t launch_tile(const QmmArgs& a, hipStream_t stream) {
  const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  const int64_t blocks = a.splits > 1 ? tiles + a.split_tail * (a.splits - 1) : tiles;
  qmm_prefill_kernel<BITS, BM, BN, WM, WN><<<(unsigned)blocks, WM * WN * 64, 0, stream>>>(a);
  if (a.splits > 1) {
    const int64_t threads = a.split_tail * (BM * BN / 4);
    prefill_fixup_kernel<BM, BN><<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(a);
  }
  return hipGetLastError();
}

struct TileShape {
  int bm, bn;
};
TileShape prefill_tile(const QmmArgs& a) {
  // Up to 64 rows of x (verify batches, and the skinny shapes no GEMV kernel
  // takes): 64 x 128 tiles.  Fewer rows of a tile are wasted on rows past M, and
  // split tiles write a quarter of the fp32 partials of a 128 x 256 tile.
  if (a.M <= 64) return {64, 128};
  if (a.bits == 8 || a.M > 128) return {256, 128};
  return {128, 256};
}

}  // namespace

PrefillPlan qmm_prefill_plan(const QmmArgs& a, int cus) {
  const TileShape ts = prefill_tile(a);
  const int64_t tiles = ((a.M + ts.bm - 1) / ts.bm) * ((a.N + ts.bn - 1) / ts.bn);
  const int64_t nk = a.K / kStepK;
  // Tiles of a part-full last wave (or all tiles, when they do not fill the chip
  // once) are split along K while the parts still fill at most one wave and keep
  // at least 8 steps each.
  const int64_t tail = tiles < cus ? tiles : tiles % cus;
  int splits = 1;
  if (tail > 0 && tail * 2 <= cus)
    while (splits < kPrefillMaxSplits && tail * splits * 2 <= cus && nk / (splits * 2) >= 8)
      splits *= 2;
  if (splits == 1) return {1, 0, 0};
  return {splits, tail, tail * splits * ts.bm * ts.bn};
}

bool qmm_prefill_supported(const QmmArgs& a) {
  return a.M >= 1 && a.K % kStepK == 0 && a.K > 0 && a.ldx % 8 == 0 &&
         (a.bits == 4 || a.bits == 8) && a.group_size >= 32 &&
         (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(a.w) & 15) == 0 &&
         // the buffer resources (x per block; w, scales, biases whole) count bytes
         // in 32 bits
         256 * a.ldx * 2 < ((int64_t)1 << 31) && a.N < ((int64_t)1 << 31) / 256 &&
         a.N * (a.K * a.bits / 8) < ((int64_t)1 << 31) &&
         a.N * (a.K / a.group_size) * 2 < ((int64_t)1 << 31);
}

bool qmm_grouped_supported(int64_t N, int64_t K, int64_t x_rows, int bits, int group_size) {
  return bits == 4 && group_size >= 32 && K % kStepK == 0 && K > 0 && N > 0 &&
         x_rows * K * 2 < ((int64_t)1 << 31) && N * (K / 2) < ((int64_t)1 << 31) &&
         N * (K / group_size) * 2 < ((int64_t)1 << 31);
}

hipError_t launch_qmm_grouped(const QmmArgs& a, int64_t max_tiles, hipStream_t stream) {
  if (max_tiles <= 0) return hipSuccess;
  if (!qmm_grouped_supported(a.N, a.K, a.g_xrows, a.bits, a.group_size) || !a.g_tiles ||
      !a.g_ntile || !a.g_rhs || !a.g_flag || a.ldx % 8 != 0 ||
      (reinterpret_cast<uintptr_t>(a.x) & 15) || (reinterpret_cast<uintptr_t>(a.w) & 15))
    return hipErrorInvalidValue;
  static_assert(kGroupedTileRows == 128, "grouped tile height");
  constexpr int BM = 128, BN = 256;
  dim3 grid((unsigned)((a.N + BN - 1) / BN), (unsigned)max_tiles);
  qmm_prefill_kernel<4, BM, BN, 2, 4, true><<<grid, 512, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_qmm_prefill(const QmmArgs& a, hipStream_t stream) {
  if (!qmm_prefill_supported(a)) return hipErrorInvalidValue;
  if (a.splits > 1 && (!a.ws || a.split_tail < 1 || a.splits > kPrefillMaxSplits))
    return hipErrorInvalidValue;
  // 128 x 256 tiles for 64 < M <= 128 (4-bit; the 8-bit form of that tile spills).
  const TileShape ts = prefill_tile(a);
  if (ts.bm == 64)
    return a.bits == 8 ? launch_tile<8, 64, 128, 2, 4>(a, stream)
                       : launch_tile<4, 64, 128, 2, 4>(a, stream);
  if (a.bits == 8) return launch_tile<8, 256, 128, 4, 2>(a, stream);
  if (ts.bm == 256) return launch_tile<4, 256, 128, 4, 2>(a, stream);
  return launch_tile<4, 128, 256, 2, 4>(a, stream);
}

}  // namespace fmxq
