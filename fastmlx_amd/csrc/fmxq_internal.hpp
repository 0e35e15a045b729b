// fmxq_internal.hpp -- launchers shared between the kernel files and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fmxq {

// Arguments common to every dense quantized product y = x . deq(W)^T.
struct QmmArgs {
  const uint16_t* x;        // [M, K] bf16 (row stride ldx elements)
  const uint32_t* w;        // [N, K*bits/32]
  const uint16_t* scales;   // [N, K/group]
  const uint16_t* biases;   // [N, K/group]
  const uint16_t* bias;     // optional additive bias [N] (qlinearBias), may be null
  uint16_t* y;              // [M, N] bf16 (row stride ldy elements)
  int64_t M, N, K;
  int64_t ldx, ldy;
  int group_size, bits;
  // Split-K state (MFMA GEMM only): splits > 1 adds fp32 partial tiles into ws
  // [M, N] (all zero between calls) and counts finished splits per output tile
  // in tile_count (all zero between calls); the last split of a tile writes y
  // and restores both to zero.
  float* ws = nullptr;
  uint32_t* tile_count = nullptr;
  int splits = 1;
  // Prefill GEMM only: the last split_tail output tiles are computed in `splits`
  // K ranges whose fp32 partials go to ws (no zero state) and are summed by a
  // second kernel.
  int64_t split_tail = 0;
  // Grouped prefill GEMM only (expert-sorted slots): tile t of the work list is
  // slots [g_tiles[2t], + g_tiles[2t+1]) of one expert g_rhs[start] (its weights at
  // w/scales/biases + expert * N rows); slot s reads x row g_rows[s] (s itself
  // without g_rows) and writes y row g_yrow[s] (s itself without g_yrow).  x has
  // g_xrows rows; a slot whose x row is past them gets a zero row and raises g_flag.
  const uint32_t* g_tiles = nullptr;
  const uint32_t* g_ntile = nullptr;
  const uint32_t* g_rhs = nullptr;
  const uint32_t* g_rows = nullptr;
  const uint32_t* g_yrow = nullptr;
  int64_t g_xrows = 0;
  uint32_t* g_flag = nullptr;
#ifdef FMXQ_QMV1_TIMELINE
  // Time-line diagnostic build only (fastmlx_amd/diag/qmv1_timeline.hip):
  // qmv1_slice_kernel stores six words per wave here when non-null.
  uint64_t* tl_stamps = nullptr;
#endif
};

// Gathered product over `batch` items of Mx rows:
//   y[i] = x[xi(i)] . deq(W[rhs[i]])^T,  xi(i) = lhs ? lhs[i] : i / lhs_div.
// A slot is one (item, row) pair; slot s = item * Mx + row is output row s.
struct GatherArgs {
  const uint16_t* x;        // [x_batch, Mx, K]
  const uint32_t* w;        // [E, N, K*bits/32]
  const uint16_t* scales;   // [E, N, K/group]
  const uint16_t* biases;   // [E, N, K/group]
  const uint32_t* lhs;      // [batch] or null
  const uint32_t* rhs;      // [batch]
  uint16_t* y;              // [batch, Mx, N]
  int64_t batch, x_batch, lhs_div, Mx, N, K, E;
  int group_size, bits;
  uint32_t* err_flag;       // set to 1 by a kernel that meets an out-of-range index
  const uint32_t* yrow = nullptr;  // optional output row of each slot (Mx == 1): the
                                   // unsort of switchGLUCore fused into the store
};

// idx (optional, [rows]) maps output row r to table row idx[r] < table_rows;
// rows whose index is out of range are zeroed and raise *err_flag.
hipError_t launch_dequantize(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                             uint16_t* out, int64_t rows, int64_t K, int group_size, int bits,
                             hipStream_t stream, const uint32_t* idx = nullptr,
                             int64_t table_rows = 0, uint32_t* err_flag = nullptr);

// Broadcast index materialization for gather_qmm's MLX batch semantics
// (fmx_index.hip).  out[i] for i over the row-major output batch shape
// shape[0..ndim) reads src at offset sum_d coord_d * stride_d (stride 0 on
// broadcast axes) and converts it to uint32: src == nullptr yields the offset
// itself (an implicit arange); negative or >= 2^32 values become 0xffffffff so
// the consumer's range check rejects them.  elem_bytes is 1, 2, 4 or 8.
constexpr int kMaxIndexDims = 8;
struct IndexMap {
  int ndim;
  int elem_bytes;
  bool is_signed;
  int64_t shape[kMaxIndexDims];
  int64_t stride[kMaxIndexDims];
};
hipError_t launch_broadcast_index(const void* src, const IndexMap& m, uint32_t* out, int64_t n,
                                  hipStream_t stream);

// Bandwidth-bound decode GEMV without MFMA: every M <= kQmvMaxM (int4 group 64
// at M = 3, 4 with 4096 or more outputs takes the MFMA walk instead), and M <= 8
// where the x rows fit in registers (qmv_supported).
constexpr int kQmvMaxM = 4;
bool qmv_supported(const QmmArgs& a);
hipError_t launch_qmv(const QmmArgs& a, hipStream_t stream);
// At most this many products of one x row in one grouped launch.
constexpr int kSliceGroupMax = 4;
hipError_t launch_qmv1_slice_group(const QmmArgs* mats, int n, hipStream_t stream);

// MFMA GEMV for 5 <= M <= 32 (fmxq_skinny.hip): qmvs for int4 group 64 with K a
// multiple of 256 and aligned operands, qmv_mfma for the other int4 (group_size
// >= 64) and int8 (group_size >= 32) cases.
constexpr int kSkinnyMaxM = 32;
bool qmvs_supported(const QmmArgs& a);
hipError_t launch_qmvs(const QmmArgs& a, hipStream_t stream);
bool qmv_mfma_supported(const QmmArgs& a);
hipError_t launch_qmv_mfma(const QmmArgs& a, hipStream_t stream);
// int4 / int8 group-64 product for M <= kQmvwMaxM with x shared through LDS by the waves
// of a block and K split over blocks (fmxq_skinny.hip, qmvw_kernel).
constexpr int kQmvwMaxM = 64;
struct QmvwPlan {
  int mt, ntt, wv, parts, d;
  int64_t ws_floats;  // fp32 partials when parts > 1
};
bool qmvw_supported(const QmmArgs& a);
QmvwPlan qmvw_plan(const QmmArgs& a, int cus);
hipError_t launch_qmvw(const QmmArgs& a, const QmvwPlan& p, hipStream_t stream);

// MFMA GEMM for larger M.  qmm_plan() reports the split-K factor and the
// workspace launch_qmm() will need for these sizes.
struct QmmPlan {
  int splits;
  int64_t ws_floats;     // M * N when splits > 1
  int64_t tile_counters; // output tiles when splits > 1
};
QmmPlan qmm_plan(int64_t M, int64_t N, int64_t K);
hipError_t launch_qmm(const QmmArgs& a, hipStream_t stream);

// Prefill GEMM (fmxq_qmm_prefill.hip): K a multiple of 64, x rows 16-byte
// aligned, 4- or 8-bit with group_size >= 32.  It takes every M > 32, and the
// 5 <= M <= 32 shapes the int4 skinny kernel (qmvs) does not.
constexpr int64_t kPrefillMinM = 32;
// Most K parts a split tile is cut into (each writes fp32 partials).
constexpr int kPrefillMaxSplits = 16;
bool qmm_prefill_supported(const QmmArgs& a);
// K split of the tiles of a part-full last wave on `cus` compute units (one block
// per CU): splits 1 means none; otherwise ws_floats of workspace for split_tail.
struct PrefillPlan {
  int splits;
  int64_t tail;
  int64_t ws_floats;
};
PrefillPlan qmm_prefill_plan(const QmmArgs& a, int cus);
hipError_t launch_qmm_prefill(const QmmArgs& a, hipStream_t stream);
// Wide GEMM (fmxq_qmm_wide.hip): 256 (or 128) x 256 tiles, weights dequantized in
// registers, stream-K over the tiles that do not fill a whole wave of blocks.
// The plan deals `dp` whole tiles to each of `blocks` blocks, then sk_len
// iterations (64-deep K steps) of the remaining sk_iters; pieces that do not end
// their tile leave fp32 partials in ws (ws_floats, one bm x 256 slot per block)
// and bump tile_count (tiles counters, zero between calls; the kernel clears
// them again).
// quantized_matmul takes the wide GEMM (where qmm_wide_supported) from
// kWideMinM rows of x, and from kWideMinMWide rows for outputs at least twice
// the depth (N >= 2K: the gate/up shapes).  Measured against the prefill GEMM
// (4-bit / 8-bit, us): 14336x4096 at M = 128 48-50 / 51-53 -> 36-38 / 38.5, at
// M = 256 58-62 / 58 -> 46-50 / 56, at M = 512 77-79 / 82 -> 63-67 / 73;
// 4096x14336 at M = 384 91 / 93 -> 70 / 86, at M = 512 93-94 / 96 -> 77.5 / 85,
// at M = 640 153 / 157 -> 110 / 132.  Below M = 384 the deep shape stays on the
// prefill GEMM (M = 256: 54 against 54-62 us).
constexpr int64_t kWideMinM = 384;
constexpr int64_t kWideMinMWide = 128;
inline bool qmm_use_wide(int64_t M, int64_t N, int64_t K) {
  return M >= kWideMinM || (M >= kWideMinMWide && N >= 2 * K);
}
constexpr int kWideMinPiece = 16;
struct WidePlan {
  int bm, tm, nk, dp, sk_len, blocks;
  int64_t sk_iters, tiles, ws_floats;
};
struct WideArgs {
  QmmArgs q;
  int tm, nk, dp, sk_len;
  int64_t sk_iters;
  uint32_t* err;  // raised (bit 2) when a wait for another block's partial gives up
};
WidePlan qmm_wide_plan(int64_t M, int64_t N, int64_t K, int cus);
bool qmm_wide_supported(const QmmArgs& a);
hipError_t launch_qmm_wide(const QmmArgs& a, const WidePlan& p, uint32_t* err, hipStream_t stream);
// Grouped form (QmmArgs::g_*): grid = N tiles x max_tiles work-list entries.
constexpr int kGroupedTileRows = 128;
bool qmm_grouped_supported(int64_t N, int64_t K, int64_t x_rows, int bits, int group_size);
hipError_t launch_qmm_grouped(const QmmArgs& a, int64_t max_tiles, hipStream_t stream);

hipError_t launch_gather_qmv(const GatherArgs& a, hipStream_t stream);

// MoE pieces around gather_qmm (fmxq_moe.hip).  The sort orders the S slots by
// expert id (ids >= E last); lhs_sorted[pos] = lhs ? lhs[s] : s / lhs_div for the
// slot s moved to pos.  With seg non-null it also writes the segment table of the
// sorted order ((start, len) pairs, each run of one id cut every `window` slots
// from its start) and the segment count to *nseg.  With sh_T > 0, sh_T slots of a
// shared expert (id E, x row t for slot S + t) follow the routed ones, and
// out-of-range routed ids are stored as E + 1.
hipError_t launch_sort_slots(const uint32_t* inds, int64_t S, int64_t lhs_div, int64_t E,
                             uint32_t* order, uint32_t* rhs_sorted, uint32_t* lhs_sorted,
                             hipStream_t stream, const uint32_t* lhs = nullptr,
                             uint32_t* seg = nullptr, uint32_t* nseg = nullptr, int window = 16,
                             uint32_t* tiles = nullptr, uint32_t* ntile = nullptr,
                             int long_min = 0, int tile_rows = 0, int64_t sh_T = 0);
hipError_t launch_silu_mul_tiles(const uint16_t* g, const uint16_t* u, uint16_t* h,
                                 const uint32_t* tiles, const uint32_t* ntile, int64_t max_tiles,
                                 int64_t tile_rows, int64_t n, hipStream_t stream);
hipError_t launch_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* h, int64_t n,
                           hipStream_t stream);
hipError_t launch_moe_combine(const uint16_t* y, const uint16_t* w, const uint16_t* shared,
                              const uint16_t* sgate, uint16_t* out, int64_t T, int64_t topk,
                              int64_t D, hipStream_t stream);

// MoE routers (fmxq_route.hip).  logits [T, E] (bf16 when in_bf16, else fp32);
// bias [E] fp32 or null (group router only); inds [T, k] uint32; weights [T, k]
// (bf16 when out_bf16, else fp32).  group selects the DeepSeek group-limited
// sigmoid router, otherwise the softmax router.
constexpr int64_t kRouteMaxExperts = 1024;
struct RouteArgs {
  const void* logits;
  const float* bias;
  uint32_t* inds;
  void* weights;
  int64_t T, E;
  int k, n_group, topk_group;
  float scale;
  bool norm, in_bf16, out_bf16;
};
hipError_t launch_route(const RouteArgs& a, bool group, hipStream_t stream);

// Weight ingest (fmx_ingest.hip): dst = -8 * src elementwise in the source dtype
// (kind 0 bf16, 1 f16, 2 f32).
hipError_t launch_scale_neg8(const void* src, void* dst, int64_t n, int kind, hipStream_t stream);

// dst = src with axes d1 and d2 of the row-major view [A, d1, B, d2, C] swapped:
// dst [A, d2, B, d1, C].  elem_bytes is 1, 2, 4 or 8 (fmx_ingest.hip).
hipError_t launch_swap_axes(const void* src, void* dst, int64_t A, int64_t d1, int64_t B,
                            int64_t d2, int64_t C, int elem_bytes, hipStream_t stream);

// MLX affine quantization of bf16 w [rows, K] into packed words wq [rows,
// K*bits/32] and bf16 scales / biases [rows, K/group_size] (fmxq_quantize.hip).
// The caller checks bits in {4, 8}, group_size in {32, 64, 128} and
// K % group_size == 0.
hipError_t launch_quantize(const uint16_t* w, uint32_t* wq, uint16_t* scales, uint16_t* biases,
                           int64_t rows, int64_t K, int group_size, int bits,
                           hipStream_t stream);

// Grouped int4 (group 64, K a multiple of 256) product over expert segments of
// a sorted slot order (fmxq_moe_gemm.hip).  w/s/b hold NMAT stacks [E, N, .]
// (gate and up for NMAT = 2, which writes silu(gate) * up); slot s reads x row
// lhs ? lhs[s] : s and writes output row yrow ? yrow[s] : s.
struct MoeArgs {
  const uint16_t* x;        // [x_rows, K]
  const uint32_t* lhs;      // [S] or null
  const uint32_t* w[2];
  const uint16_t* s[2];
  const uint16_t* b[2];
  const uint32_t* rhs;      // [S] expert of each slot (sorted when seg is set)
  const uint32_t* seg;      // (start, len) pairs, or null: segment i is slot i alone
  const uint32_t* nseg;     // segment count (device); S when seg is null
  uint16_t* y;              // [rows, N]
  const uint32_t* yrow;     // [S] or null
  int64_t S, N, K, E, x_rows;
  uint32_t* err_flag;
  int64_t lhs_div = 1;      // x row of slot s is lhs[s], or s / lhs_div without lhs
  // Few-slot GEMV form only (no segment table, no yrow): sh_T more segments after
  // the S slots, segment S + t the shared expert (sh_w / sh_s / sh_b, one [N, .]
  // matrix each) on x row t, written to output row S + t.
  const uint32_t* sh_w[2] = {nullptr, nullptr};
  const uint16_t* sh_s[2] = {nullptr, nullptr};
  const uint16_t* sh_b[2] = {nullptr, nullptr};
  int64_t sh_T = 0;
  // Segment-table form only: expert id E names the shared expert (sh_w / sh_s /
  // sh_b), ids above E are out of range (launch_sort_slots with sh_T > 0).
  bool sh_seg = false;
};
// Slot counts up to which the MoE products skip the sort: every slot is its own
// segment (a sort saves weight reads only when slots share an expert).
constexpr int64_t kMoeUnsortedMaxSlots = 16;
// SwitchGLU with the top-k combine (fmxq_switch_glu_combine) stays unsorted, with
// the combine fused into the down projection, up to 256 slots routed over at least
// twice as many experts: few slots then share an expert, and skipping the sort
// and combine launches outweighs the re-reads (configuration 3 at M = 16, 160
// slots over 512 experts: 77.5 -> 72.5 us).  Where many slots share experts
// (configuration 4 at M = 32, 256 slots over 256 experts, Zipf routing) the
// re-reads double the time, so those batches sort.
constexpr int64_t kMoeUnsortedCombineMaxSlots = 256;
inline bool moe_combine_unsorted(int64_t S, int64_t E) {
  return S <= kMoeUnsortedMaxSlots || (S <= kMoeUnsortedCombineMaxSlots && 2 * S <= E);
}
bool moe_qmvs_supported(int64_t N, int64_t K, int bits, int group_size);
int moe_window(int64_t S, int64_t E);
int64_t moe_max_segments(int64_t S, int64_t E, int window);
hipError_t launch_moe_qmvs(const MoeArgs& a, int nmat, int window, int64_t max_seg,
                           hipStream_t stream);

// Few-slot down projection fused with the top-k combine (one block per row
// tile and token, one wave per slot): out [T, D] from the h rows [T k, I].
bool moe_down_combine_supported(int64_t T, int64_t k, int64_t D, int64_t I, int bits,
                                int group_size);
// With sh_w (the shared expert's down matrix [D, I*bits/32] and its scales and
// biases), one more wave per block computes that expert's down product for the
// token from h row T k + t and adds it (sigmoid-gated by sgate) in place of the
// precomputed `shared` rows; then k <= 15.
hipError_t launch_moe_down_combine(const uint16_t* h, const uint32_t* inds, const uint32_t* w,
                                   const uint16_t* s, const uint16_t* b, const uint16_t* weights,
                                   const uint16_t* shared, const uint16_t* sgate, uint16_t* out,
                                   int64_t T, int64_t k, int64_t E, int64_t D, int64_t I,
                                   uint32_t* err_flag, hipStream_t stream,
                                   const uint32_t* sh_w = nullptr, const uint16_t* sh_s = nullptr,
                                   const uint16_t* sh_b = nullptr);
// Fill n uint32 words with v (a kernel, so it can sit in a captured graph).
hipError_t launch_fill_u32(uint32_t* p, uint32_t v, int64_t n, hipStream_t stream);

// Grouped MFMA gather for expert-sorted batches (int4 group_size >= 64, int8 >= 32).
constexpr int64_t kGroupedMinSlots = 32;
bool gather_mfma_supported(const GatherArgs& a);
hipError_t launch_gather_mfma(const GatherArgs& a, hipStream_t stream);

}  // namespace fmxq
