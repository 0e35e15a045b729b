// fmxq_capi.cpp -- extern "C" entry points of libfmxq.so (declared in include/fmxq.h).
//
// Validation happens here, before anything is enqueued: a failing call returns a
// nonzero fmxq_status with a message and leaves the stream untouched, the
// contract mlxgo relies on when it frees the result handle on rc != 0
// (mlxgo/binding_cgo.go:636-643).  Dispatch by M:
//   M <= 8 (x rows fit in registers) -> decode GEMV (fmxq_qmv.hip), no MFMA
//   M <= 32                          -> MFMA GEMV (fmxq_skinny.hip)
//   otherwise                        -> LDS-dequant MFMA GEMM (fmxq_qmm.hip)
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/fmxq.h"
#include "fmxq_host.hpp"
#include "fmxq_internal.hpp"

namespace fmxq {

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return FMXQ_OK;
  return fail(FMXQ_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}


}  // namespace fmxq

using fmxq::check_quant;
using fmxq::device_flag;
using fmxq::fail;
using fmxq::hip_status;

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Split-K workspace of the MFMA GEMM, one per (device, stream) so that calls on
// different streams never share it.  Both arrays are zero between calls: the
// kernel's last split per tile restores them.  Growth needs hipMalloc, which is
// refused while the stream is being captured into a graph.
struct SplitWs {
  float* ws = nullptr;
  int64_t ws_floats = 0;
  uint32_t* counters = nullptr;
  int64_t n_counters = 0;
  float* pf = nullptr;  // K-split partials (overwritten by every call, no zero state)
  int64_t pf_floats = 0;
};
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, SplitWs> g_ws;

// Device buffers replaced by larger ones.  A graph captured earlier may still
// hold them, so they are kept alive (growth is monotonic, at most doubling the
// footprint) rather than freed.  The list has its own lock: the split-K and the
// SwitchGLU scratch grow under different locks.
std::mutex g_retired_mu;
std::vector<void*> g_retired;
void retire(void* p) {
  if (!p) return;
  std::lock_guard<std::mutex> lk(g_retired_mu);
  g_retired.push_back(p);
}

int split_workspace(hipStream_t s, const fmxq::QmmPlan& plan, float** ws, uint32_t** cnt) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(FMXQ_ERR_DEVICE, "hipGetDevice failed");
  std::lock_guard<std::mutex> lk(g_ws_mu);
  SplitWs& w = g_ws[{dev, s}];
  if (w.ws_floats < plan.ws_floats || w.n_counters < plan.tile_counters) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
      return fail(FMXQ_ERR_INVALID_ARGUMENT,
                  "quantized_matmul: split-K workspace must grow to %lld floats during graph "
                  "capture; run the same shape once outside capture first",
                  (long long)plan.ws_floats);
    if (int rc = hip_status(hipStreamSynchronize(s), "split-K workspace: synchronize")) return rc;
    const int64_t nf = std::max(plan.ws_floats, w.ws_floats);
    const int64_t nc = std::max(plan.tile_counters, w.n_counters);
    float* nws = nullptr;
    uint32_t* ncnt = nullptr;
    if (int rc = hip_status(hipMalloc(&nws, nf * sizeof(float)), "split-K workspace: hipMalloc"))
      return rc;
    if (int rc = hip_status(hipMalloc(&ncnt, nc * sizeof(uint32_t)), "split-K counters: hipMalloc")) {
      (void)hipFree(nws);
      return rc;
    }
    if (int rc = hip_status(hipMemset(nws, 0, nf * sizeof(float)), "split-K workspace: clear")) return rc;
    if (int rc = hip_status(hipMemset(ncnt, 0, nc * sizeof(uint32_t)), "split-K counters: clear"))
      return rc;
    retire(w.ws);
    retire(w.counters);
    w.ws = nws;
    w.ws_floats = nf;
    w.counters = ncnt;
    w.n_counters = nc;
  }
  *ws = w.ws;
  *cnt = w.counters;
  return FMXQ_OK;
}

int prefill_workspace(hipStream_t s, int64_t floats, float** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(FMXQ_ERR_DEVICE, "hipGetDevice failed");
  std::lock_guard<std::mutex> lk(g_ws_mu);
  SplitWs& w = g_ws[{dev, s}];
  if (w.pf_floats < floats) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
      return fail(FMXQ_ERR_INVALID_ARGUMENT,
                  "quantized_matmul: prefill workspace must grow to %lld floats during graph "
                  "capture; run the same shape once outside capture first",
                  (long long)floats);
    if (int rc = hip_status(hipStreamSynchronize(s), "prefill workspace: synchronize")) return rc;
    float* p = nullptr;
    if (int rc = hip_status(hipMalloc(&p, floats * sizeof(float)), "prefill workspace: hipMalloc"))
      return rc;
    retire(w.pf);
    w.pf = p;
    w.pf_floats = floats;
  }
  *out = w.pf;
  return FMXQ_OK;
}

// Compute units of the current device (blocks of the prefill GEMM resident at once).
int device_cus(int* out) {
  static std::mutex mu;
  static std::map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(FMXQ_ERR_DEVICE, "hipGetDevice failed");
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find(dev);
  if (it == cache.end()) {
    int n = 0;
    if (int rc = hip_status(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev),
                            "hipDeviceGetAttribute"))
      return rc;
    it = cache.emplace(dev, n > 0 ? n : 1).first;
  }
  *out = it->second;
  return FMXQ_OK;
}

// Per-(device, stream) scratch for the SwitchGLU intermediates, grown on demand
// (never while the stream is being captured) and, like the split-K workspace,
// never freed while a captured graph may still point at it.
// Slot 1 holds the expert rows between a SwitchGLU and its combine
// (fmxq_switch_glu_combine), while slot 0 serves the SwitchGLU itself.
std::mutex g_arena_mu;
std::map<std::tuple<int, hipStream_t, int>, std::pair<void*, size_t>> g_arena;
// Words of a zero-id buffer (fmxq_moe_layer, arena slot 3) already filled.
std::map<const void*, int64_t> g_zero_filled;

int stream_arena(hipStream_t s, size_t bytes, void** out, const char* op, int slot = 0) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(FMXQ_ERR_DEVICE, "hipGetDevice failed");
  std::lock_guard<std::mutex> lk(g_arena_mu);
  auto& a = g_arena[{dev, s, slot}];
  if (a.second < bytes) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
      return fail(FMXQ_ERR_INVALID_ARGUMENT,
                  "%s: scratch must grow to %zu bytes during graph capture; run the same shape "
                  "once outside capture first", op, bytes);
    void* p = nullptr;
    if (int rc = hip_status(hipMalloc(&p, bytes), "switch_glu scratch: hipMalloc")) return rc;
    retire(a.first);
    a = {p, bytes};
  }
  *out = a.first;
  return FMXQ_OK;
}

// Where a SwitchGLU call's scratch comes from: the per-(device, stream) arena,
// grown with hipMalloc, or (fmxq_switch_glu_noalloc) the device's fixed
// __device__ buffer, which is never grown: a call needing more is refused before
// anything is enqueued.
struct ScratchSource {
  void* fixed = nullptr;
  size_t fixed_bytes = 0;
  int get(hipStream_t s, size_t bytes, void** out, const char* op) const {
    if (!fixed) return stream_arena(s, bytes, out, op);
    if (bytes > fixed_bytes)
      return fail(FMXQ_ERR_SHAPE,
                  "%s: this call needs %zu bytes of scratch, more than the %zu bytes the "
                  "allocation-free entry point holds; use fmxq_switch_glu or fewer slots",
                  op, bytes, fixed_bytes);
    *out = fixed;
    return FMXQ_OK;
  }
};

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

// Counting sort in one block keeps two (E + 1)-entry tables in LDS.
constexpr int64_t kSortMaxExperts = 16384;
// Segments run along the grid's y axis.
constexpr int64_t kMaxSegmentsGrid = 65535;

// Scratch of the segmented MoE product in the stream arena: the sorted order,
// ids and x rows of S slots, the segment table and count, and (SwitchGLU) the
// h rows of the sorted slots.
// With max_tiles > 0 also the grouped GEMM's work list and count and (gu_cols > 0)
// the gate and up rows of its tiles.
struct MoeScratch {
  uint32_t *order, *rhs, *lhs, *seg, *nseg;
  uint16_t* h;
  uint32_t *tiles = nullptr, *ntile = nullptr;
  uint16_t *g = nullptr, *u = nullptr;
};
int moe_scratch(hipStream_t s, int64_t S, int64_t h_cols, int64_t max_seg, MoeScratch* m,
                const char* op, int64_t max_tiles = 0, int64_t gu_cols = 0,
                const ScratchSource& src = ScratchSource()) {
  const size_t ib = align_up((size_t)S * sizeof(uint32_t));
  const size_t sb = align_up((size_t)max_seg * 2 * sizeof(uint32_t));
  const size_t hb = align_up((size_t)S * h_cols * sizeof(uint16_t));
  const size_t tb = align_up((size_t)max_tiles * 2 * sizeof(uint32_t));
  const size_t gb = align_up((size_t)S * gu_cols * sizeof(uint16_t));
  void* arena = nullptr;
  if (int rc = src.get(s, 3 * ib + sb + 256 + hb + tb + 256 + 2 * gb, &arena, op)) return rc;
  char* p = static_cast<char*>(arena);
  m->order = reinterpret_cast<uint32_t*>(p);
  m->rhs = reinterpret_cast<uint32_t*>(p + ib);
  m->lhs = reinterpret_cast<uint32_t*>(p + 2 * ib);
  m->seg = reinterpret_cast<uint32_t*>(p + 3 * ib);
  m->nseg = reinterpret_cast<uint32_t*>(p + 3 * ib + sb);
  m->h = h_cols ? reinterpret_cast<uint16_t*>(p + 3 * ib + sb + 256) : nullptr;
  char* q = p + 3 * ib + sb + 256 + hb;
  if (max_tiles > 0) {
    m->tiles = reinterpret_cast<uint32_t*>(q);
    m->ntile = reinterpret_cast<uint32_t*>(q + tb);
    if (gu_cols > 0) {
      m->g = reinterpret_cast<uint16_t*>(q + tb + 256);
      m->u = reinterpret_cast<uint16_t*>(q + tb + 256 + gb);
    }
  }
  return FMXQ_OK;
}

// Expert runs of at least this many slots go to the grouped GEMM (tiles of
// kGroupedTileRows slots); shorter runs stay on the segment kernels.  Only batches
// of kGroupedMinSlots or more use it: a grouped block walks all of K, so a few
// tiles (one 256-slot run: 2 tiles x N/256 blocks) leave the chip idle where the
// window walk spreads the same run over many blocks.  Batches averaging fewer
// than kGroupedMinAvgRun slots per expert skip it too: the gate, up and down
// passes and the silu pass are launched whatever the routing, and with runs that
// short they rarely find a tile (configuration 3 at M = 512, 10 slots per expert:
// 252-256 -> 248-250 us per layer).
constexpr int64_t kGroupedMinRun = 256;
constexpr int64_t kGroupedMinSlots = 4096;
constexpr int64_t kGroupedMinAvgRun = 16;
int64_t grouped_max_tiles(int64_t S, int64_t E) {
  if (S < kGroupedMinSlots || S < kGroupedMinAvgRun * E) return 0;
  const int64_t runs = S / kGroupedMinRun < E ? S / kGroupedMinRun : E;
  const int64_t bound = runs == 0 ? 0 : runs + S / fmxq::kGroupedTileRows + 1;
  return bound <= kMaxSegmentsGrid ? bound : 0;  // the work list runs along the grid's y axis
}
// A grouped-GEMM pass over the work list of sorted slots (see QmmArgs::g_*).
fmxq::QmmArgs grouped_args(const uint16_t* x, const uint32_t* w, const uint16_t* sc,
                           const uint16_t* bi, uint16_t* y, int64_t N, int64_t K, int bits,
                           int group_size, const MoeScratch& m, const uint32_t* rows,
                           const uint32_t* yrow, int64_t x_rows, uint32_t* flag) {
  fmxq::QmmArgs a{x, w, sc, bi, nullptr, y, 0, N, K, K, N, group_size, bits};
  a.g_tiles = m.tiles;
  a.g_ntile = m.ntile;
  a.g_rhs = m.rhs;
  a.g_rows = rows;
  a.g_yrow = yrow;
  a.g_xrows = x_rows;
  a.g_flag = flag;
  return a;
}

int qmm_common(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
               const uint16_t* biases, const uint16_t* bias, uint16_t* y, int64_t M, int64_t N,
               int64_t K, bool transpose, int group_size, int bits, void* stream,
               const char* op) {
  if (int rc = check_quant(group_size, bits, K, transpose, op)) return rc;
  if (M < 0 || N < 0) return fail(FMXQ_ERR_SHAPE, "%s: negative size M=%lld N=%lld", op,
                                  (long long)M, (long long)N);
  if (M == 0 || N == 0) return FMXQ_OK;
  if (!x || !w || !scales || !biases || !y)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null operand", op);
  if (!aligned16(x) || !aligned16(w))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: x and w must be 16-byte aligned", op);
  fmxq::QmmArgs a{x, w, scales, biases, bias, y, M, N, K, K, N, group_size, bits};
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Prefill sizes: the wide GEMM (256 x 256 tiles, weights dequantized in
  // registers, stream-K over the tiles past the last whole wave of blocks).
  if (fmxq::qmm_use_wide(M, N, K) && fmxq::qmm_wide_supported(a)) {
    int cus = 0;
    if (int rc = device_cus(&cus)) return rc;
    const fmxq::WidePlan wp = fmxq::qmm_wide_plan(M, N, K, cus);
    uint32_t* flag = nullptr;
    if (wp.sk_len > 0) {
      if (int rc = prefill_workspace(s, wp.ws_floats, &a.ws)) return rc;
      float* unused = nullptr;
      if (int rc = split_workspace(s, fmxq::QmmPlan{2, 0, wp.tiles}, &unused, &a.tile_count))
        return rc;
      if (int rc = device_flag(s, &flag)) return rc;
    }
    return hip_status(fmxq::launch_qmm_wide(a, wp, flag, s), op);
  }
  // qmvw, x shared through LDS and K split over blocks.  int4 group 64 at
  // 9 <= M <= 64, at M <= 16 only for wide outputs or long rows, where it beats
  // qmvs.  int8 group 64 (dequantizing walk) from M = 9 on every shape, and from
  // M = 2 / 3 / 8 on long rows / wide / 4096-row outputs, where it beats the dot2
  // GEMV (us, dot2 -> walk: 4096x14336 M = 2 21.1 -> 17.1, M = 5 33.4 -> 17.6;
  // 14336x4096 M = 3 21.0 -> 18.2, M = 5 24.4 -> 18.5 (M = 2 15.4 against 18.1
  // stays); 4096x4096 M = 8 13.0 -> 9.3 (M = 5 9.4 against 9.3 stays); narrower
  // outputs keep the GEMV up to M = 8: 1024x4096 M = 8 5.8 against 6.9) and the
  // prefill GEMM's 64-row tile (M = 9-16 on 4096x4096 16.5-17.3 -> 9.4-9.6).
  const bool walk4 = bits == 4 && M > 8 && (M > 16 || N >= 8192 || K >= 8192);
  const bool walk8 = bits == 8 && (M >= 9 || (M >= 2 && K >= 8192) || (M >= 3 && N >= 8192) ||
                                   (M >= 8 && N >= 4096));
  if ((walk4 || walk8) && M <= fmxq::kQmvwMaxM && fmxq::qmvw_supported(a)) {
    int cus = 0;
    if (int rc = device_cus(&cus)) return rc;
    const fmxq::QmvwPlan qp = fmxq::qmvw_plan(a, cus);
    if (qp.parts > 1) {
      if (int rc = prefill_workspace(s, qp.ws_floats, &a.ws)) return rc;
      a.splits = qp.parts;
    }
    return hip_status(fmxq::launch_qmvw(a, qp, s), op);
  }
  // M <= 2: dot2 GEMV.  M = 3, 4: qmvs on outputs of 4096 rows or more (C1 stack,
  // 224 products, whose 1024-row k and v stay on the dot2 GEMV: M = 3 2.11 ->
  // 1.92 ms, M = 4 2.12 -> 1.97 ms; at M = 2 it lost, 1.56 -> 1.86 ms), the dot2
  // GEMV otherwise.  Other M <= 32: qmvs, except that narrow outputs (N < 2048)
  // at M <= 8 stay on the dot2 GEMV, which is quicker there.
  const bool skinny = (M > fmxq::kQmvMaxM || (M >= 3 && N >= 4096)) && M <= fmxq::kSkinnyMaxM &&
                      fmxq::qmvs_supported(a) && !(M <= 8 && N < 2048 && fmxq::qmv_supported(a));
  if (skinny) return hip_status(fmxq::launch_qmvs(a, s), op);
  // 5 <= M <= 32 shapes qmvs does not take (int8, other group sizes) run on the
  // prefill GEMM's 64-row tile; M <= 4 stays on the dot2 GEMV, and so do int8
  // products where the x rows fit in registers: M <= 6 on any output width, M = 7
  // and 8 up to 4096 rows (int8 M = 5 against the prefill tile: 4096x4096 16.0 ->
  // 9.6 us, 14336x4096 35.7 -> 25.0 us, 28672x4096 60.3 -> 46.2 us; M = 8 at
  // 14336x4096 36.1 against 37.3 us stays on the tile).
  const bool small_gemm =
      M > fmxq::kQmvMaxM && M <= fmxq::kSkinnyMaxM && !fmxq::qmvs_supported(a) &&
      fmxq::qmm_prefill_supported(a) &&
      !(bits == 8 && (M <= 6 || (M <= 8 && N <= 4096)) && fmxq::qmv_supported(a));
  if (!small_gemm && fmxq::qmv_supported(a)) return hip_status(fmxq::launch_qmv(a, s), op);
  if (!small_gemm && M <= fmxq::kSkinnyMaxM && fmxq::qmv_mfma_supported(a))
    return hip_status(fmxq::launch_qmv_mfma(a, s), op);
  if (fmxq::qmm_prefill_supported(a)) {
    int cus = 0;
    if (int rc = device_cus(&cus)) return rc;
    const fmxq::PrefillPlan pp = fmxq::qmm_prefill_plan(a, cus);
    if (pp.splits > 1) {
      if (int rc = prefill_workspace(s, pp.ws_floats, &a.ws)) return rc;
      a.splits = pp.splits;
      a.split_tail = pp.tail;
    }
    return hip_status(fmxq::launch_qmm_prefill(a, s), op);
  }
  const fmxq::QmmPlan plan = fmxq::qmm_plan(M, N, K);
  if (plan.splits > 1) {
    if (int rc = split_workspace(s, plan, &a.ws, &a.tile_count)) return rc;
    a.splits = plan.splits;
  }
  return hip_status(fmxq::launch_qmm(a, s), op);
}

}  // namespace

extern "C" {

int fmxq_version(void) { return 100; }

int fmxq_dequantize(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                    uint16_t* out, int64_t rows, int64_t K, int group_size, int bits,
                    void* stream) {
  if (int rc = check_quant(group_size, bits, K, true, "dequantize")) return rc;
  if (rows < 0) return fail(FMXQ_ERR_SHAPE, "dequantize: negative rows");
  if (rows == 0) return FMXQ_OK;
  if (!w || !scales || !biases || !out)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "dequantize: null operand");
  if (!aligned16(w) || !aligned16(out))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "dequantize: w and out must be 16-byte aligned");
  return hip_status(fmxq::launch_dequantize(w, scales, biases, out, rows, K, group_size, bits,
                                            static_cast<hipStream_t>(stream)),
                    "dequantize");
}

int fmxq_quantize(const uint16_t* w, uint32_t* wq, uint16_t* scales, uint16_t* biases,
                  int64_t rows, int64_t K, int group_size, int bits, void* stream) {
  if (int rc = check_quant(group_size, bits, K, true, "quantize")) return rc;
  if (rows < 0) return fail(FMXQ_ERR_SHAPE, "quantize: negative rows");
  if (rows == 0) return FMXQ_OK;
  if (!w || !wq || !scales || !biases)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "quantize: null operand");
  if (!aligned16(w) || !aligned16(wq))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "quantize: w and wq must be 16-byte aligned");
  return hip_status(fmxq::launch_quantize(w, wq, scales, biases, rows, K, group_size, bits,
                                          static_cast<hipStream_t>(stream)),
                    "quantize");
}

int fmxq_dequantize_rows(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                         const uint32_t* idx, uint16_t* out, int64_t n_idx, int64_t table_rows,
                         int64_t K, int group_size, int bits, void* stream) {
  const char* op = "dequantize_rows";
  if (int rc = check_quant(group_size, bits, K, true, op)) return rc;
  if (n_idx < 0 || table_rows < 0) return fail(FMXQ_ERR_SHAPE, "%s: negative size", op);
  if (n_idx == 0) return FMXQ_OK;
  if (table_rows == 0)
    return fail(FMXQ_ERR_SHAPE, "%s: %lld lookups into an empty table", op, (long long)n_idx);
  if (!w || !scales || !biases || !idx || !out)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null operand", op);
  if (!aligned16(w) || !aligned16(out))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: w and out must be 16-byte aligned", op);
  uint32_t* flag = nullptr;
  if (int rc = device_flag(static_cast<hipStream_t>(stream), &flag)) return rc;
  return hip_status(fmxq::launch_dequantize(w, scales, biases, out, n_idx, K, group_size, bits,
                                            static_cast<hipStream_t>(stream), idx, table_rows,
                                            flag),
                    op);
}

int fmxq_quantized_matmul(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                          const uint16_t* biases, uint16_t* y, int64_t M, int64_t N,
                          int64_t K, bool transpose, int group_size, int bits, void* stream) {
  return qmm_common(x, w, scales, biases, nullptr, y, M, N, K, transpose, group_size, bits,
                    stream, "quantized_matmul");
}

int fmxq_quantized_matmul_group(const uint16_t* x, int n, const uint32_t* const* w,
                                const uint16_t* const* scales, const uint16_t* const* biases,
                                uint16_t* const* y, const int64_t* N, int64_t M, int64_t K,
                                bool transpose, int group_size, int bits, void* stream) {
  const char* op = "quantized_matmul_group";
  if (n < 1 || n > fmxq::kSliceGroupMax)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: n=%d outside 1..%d", op, n, fmxq::kSliceGroupMax);
  if (!w || !scales || !biases || !y || !N)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null operand array", op);
  if (int rc = check_quant(group_size, bits, K, transpose, op)) return rc;
  if (M < 0) return fail(FMXQ_ERR_SHAPE, "%s: negative size M=%lld", op, (long long)M);
  fmxq::QmmArgs mats[fmxq::kSliceGroupMax];
  for (int i = 0; i < n; ++i) {
    if (N[i] < 0)
      return fail(FMXQ_ERR_SHAPE, "%s: negative size N[%d]=%lld", op, i, (long long)N[i]);
    if (M > 0 && N[i] > 0) {
      if (!x || !w[i] || !scales[i] || !biases[i] || !y[i])
        return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null operand of product %d", op, i);
      if (!aligned16(x) || !aligned16(w[i]))
        return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: x and w[%d] must be 16-byte aligned", op, i);
    }
    mats[i] = fmxq::QmmArgs{x, w[i], scales[i], biases[i], nullptr, y[i], M, N[i], K, K, N[i],
                            group_size, bits};
  }
  if (M == 0) return FMXQ_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t e = fmxq::launch_qmv1_slice_group(mats, n, s);
  if (e != hipErrorNotSupported) return hip_status(e, op);
  // Shapes the grouped launch does not take: one product at a time.
  for (int i = 0; i < n; ++i)
    if (int rc = qmm_common(x, w[i], scales[i], biases[i], nullptr, y[i], M, N[i], K, transpose,
                            group_size, bits, stream, op))
      return rc;
  return FMXQ_OK;
}

int fmxq_quantized_matmul_bias(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                               const uint16_t* biases, const uint16_t* bias, uint16_t* y,
                               int64_t M, int64_t N, int64_t K, bool transpose,
                               int group_size, int bits, void* stream) {
  return qmm_common(x, w, scales, biases, bias, y, M, N, K, transpose, group_size, bits, stream,
                    "quantized_matmul_bias");
}

int fmxq_gather_qmm(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                    const uint16_t* biases, const uint32_t* lhs_indices,
                    const uint32_t* rhs_indices, uint16_t* y, int64_t batch, int64_t x_batch,
                    int64_t lhs_div, int64_t Mx, int64_t N, int64_t K, int64_t E,
                    bool transpose, int group_size, int bits, bool sorted_indices,
                    void* stream) {
  // sorted_indices only picks the kernel: the grouped MFMA kernel for sorted
  // batches, the per-slot GEMV otherwise.  Both give the same values for a slot.
  const char* op = "gather_qmm";
  if (int rc = check_quant(group_size, bits, K, transpose, op)) return rc;
  if (batch < 0 || x_batch < 0 || Mx < 0 || N < 0 || E < 0)
    return fail(FMXQ_ERR_SHAPE, "%s: negative size", op);
  if (batch == 0 || Mx == 0 || N == 0) return FMXQ_OK;
  if (E == 0 || x_batch == 0)
    return fail(FMXQ_ERR_SHAPE, "%s: %lld output items but E=%lld x_batch=%lld", op,
                (long long)batch, (long long)E, (long long)x_batch);
  if (!lhs_indices && lhs_div <= 0)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: lhs_div must be >= 1 without lhs_indices", op);
  if (!lhs_indices && (batch - 1) / lhs_div >= x_batch)
    return fail(FMXQ_ERR_SHAPE, "%s: batch=%lld / lhs_div=%lld exceeds x_batch=%lld", op,
                (long long)batch, (long long)lhs_div, (long long)x_batch);
  if (!x || !w || !scales || !biases || !rhs_indices || !y)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null operand", op);
  if (!aligned16(x) || !aligned16(w))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: x and w must be 16-byte aligned", op);
  if (batch * Mx > 0x7fffffffLL)
    return fail(FMXQ_ERR_SHAPE, "%s: batch*Mx=%lld too large", op, (long long)(batch * Mx));
  uint32_t* flag = nullptr;
  if (int rc = device_flag(static_cast<hipStream_t>(stream), &flag)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (Mx == 1 && E <= kSortMaxExperts && fmxq::moe_qmvs_supported(N, K, bits, group_size) &&
      aligned16(scales) && aligned16(biases)) {
    // Items sorted by expert, then one grouped product per expert segment; the
    // sort's order maps each sorted item back to its output row.
    if (batch <= fmxq::kMoeUnsortedMaxSlots) {
      // A few items: each is its own segment, written to its own output row.
      fmxq::MoeArgs a{x, lhs_indices, {w, nullptr}, {scales, nullptr}, {biases, nullptr},
                      rhs_indices, nullptr, nullptr, y, nullptr, batch, N, K, E, x_batch, flag,
                      lhs_div};
      return hip_status(fmxq::launch_moe_qmvs(a, 1, 16, batch, s), op);
    }
    const int window = fmxq::moe_window(batch, E);
    const int64_t max_seg = fmxq::moe_max_segments(batch, E, window);
    if (max_seg <= kMaxSegmentsGrid) {
      MoeScratch m;
      const int64_t max_tiles = fmxq::qmm_grouped_supported(N, K, x_batch, bits, group_size)
                                    ? grouped_max_tiles(batch, E)
                                    : 0;
      if (int rc = moe_scratch(s, batch, 0, max_seg, &m, op, max_tiles)) return rc;
      if (int rc = hip_status(fmxq::launch_sort_slots(rhs_indices, batch, lhs_div, E, m.order,
                                                      m.rhs, m.lhs, s, lhs_indices, m.seg,
                                                      m.nseg, window, m.tiles, m.ntile,
                                                      (int)kGroupedMinRun,
                                                      fmxq::kGroupedTileRows),
                              "gather_qmm: sort"))
        return rc;
      fmxq::MoeArgs a{x, m.lhs, {w, nullptr}, {scales, nullptr}, {biases, nullptr}, m.rhs,
                      m.seg, m.nseg, y, m.order, batch, N, K, E, x_batch, flag};
      if (int rc = hip_status(fmxq::launch_moe_qmvs(a, 1, window, max_seg, s), op)) return rc;
      if (!max_tiles) return FMXQ_OK;
      const fmxq::QmmArgs gq = grouped_args(x, w, scales, biases, y, N, K, bits, group_size, m,
                                            m.lhs, m.order, x_batch, flag);
      return hip_status(fmxq::launch_qmm_grouped(gq, max_tiles, s), op);
    }
  }
  fmxq::GatherArgs a{x,      w,     scales,  biases, lhs_indices, rhs_indices, y,
                     batch,  x_batch, lhs_div, Mx,   N,           K,           E,
                     group_size, bits, flag};
  if (sorted_indices && batch * Mx >= fmxq::kGroupedMinSlots && fmxq::gather_mfma_supported(a))
    return hip_status(fmxq::launch_gather_mfma(a, s), op);
  return hip_status(fmxq::launch_gather_qmv(a, s), op);
}

int fmxq_device_error(void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* own = nullptr;
  uint32_t* graph = nullptr;
  if (int rc = fmxq::device_flags_to_check(s, &own, &graph)) return rc;
  if (int rc = hip_status(hipStreamSynchronize(s), "device_error: synchronize")) return rc;
  uint32_t v = 0;
  for (uint32_t* flag : {own, graph}) {
    uint32_t w = 0;
    if (int rc = hip_status(hipMemcpy(&w, flag, sizeof(w), hipMemcpyDeviceToHost),
                            "device_error: read flag"))
      return rc;
    if (w == 0) continue;
    if (int rc = hip_status(hipMemset(flag, 0, sizeof(uint32_t)), "device_error: clear flag"))
      return rc;
    v |= w;
  }
  if (v == 0) return FMXQ_OK;
  if (v & 2u)
    return fail(FMXQ_ERR_DEVICE,
                "quantized_matmul: a block of the wide GEMM gave up waiting for another "
                "block's partial sums (outputs of that tile are incomplete)");
  return fail(FMXQ_ERR_INDEX, "gather_qmm: an index was out of range (outputs zeroed)");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// SwitchGLU MoE expert MLP and its combine.

namespace {

int gather_dispatch(const fmxq::GatherArgs& a, bool sorted, hipStream_t s) {
  if (sorted && a.batch * a.Mx >= fmxq::kGroupedMinSlots && fmxq::gather_mfma_supported(a))
    return hip_status(fmxq::launch_gather_mfma(a, s), "switch_glu: gather");
  return hip_status(fmxq::launch_gather_qmv(a, s), "switch_glu: gather");
}

}  // namespace

namespace {

int switch_glu_impl(const uint16_t* x, const uint32_t* inds, const uint32_t* w_gate,
                    const uint16_t* s_gate, const uint16_t* b_gate, const uint32_t* w_up,
                    const uint16_t* s_up, const uint16_t* b_up, const uint32_t* w_down,
                    const uint16_t* s_down, const uint16_t* b_down, uint16_t* out, int64_t T,
                    int64_t topk, int64_t E, int64_t D, int64_t I, int group_size, int bits,
                    void* stream, const ScratchSource& src, const char* op) {
  if (int rc = check_quant(group_size, bits, D, true, op)) return rc;
  if (int rc = check_quant(group_size, bits, I, true, op)) return rc;
  if (T < 0 || topk < 1 || E < 1)
    return fail(FMXQ_ERR_SHAPE, "%s: need T >= 0, top_k >= 1, E >= 1 (got %lld %lld %lld)", op,
                (long long)T, (long long)topk, (long long)E);
  const int64_t S = T * topk;
  if (S == 0) return FMXQ_OK;
  if (!x || !inds || !w_gate || !s_gate || !b_gate || !w_up || !s_up || !b_up || !w_down ||
      !s_down || !b_down || !out)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null operand", op);
  if (!aligned16(x) || !aligned16(w_gate) || !aligned16(w_up) || !aligned16(w_down) ||
      !aligned16(out))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: x, weights and out must be 16-byte aligned", op);
  if (S > 0x7fffffffLL) return fail(FMXQ_ERR_SHAPE, "%s: too many slots", op);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* flag = nullptr;
  if (int rc = device_flag(static_cast<hipStream_t>(stream), &flag)) return rc;
  const int window = fmxq::moe_window(S, E);
  const int64_t max_seg = fmxq::moe_max_segments(S, E, window);
  if (E <= kSortMaxExperts && max_seg <= kMaxSegmentsGrid &&
      fmxq::moe_qmvs_supported(I, D, bits, group_size) &&
      fmxq::moe_qmvs_supported(D, I, bits, group_size) && aligned16(s_gate) &&
      aligned16(b_gate) && aligned16(s_up) && aligned16(b_up) && aligned16(s_down) &&
      aligned16(b_down)) {
    // Sorted slots (for every slot count: the order cannot change a value, each
    // slot being its own product row), then gate and up fused with silu * up into
    // h in sorted order, then down written to each slot's own output row.  A few
    // slots skip the sort: each is its own segment, h stays in slot order.
    MoeScratch m;
    if (S <= fmxq::kMoeUnsortedMaxSlots) {
      if (int rc = moe_scratch(s, S, I, 1, &m, op, 0, 0, src)) return rc;
      fmxq::MoeArgs gu{x, nullptr, {w_gate, w_up}, {s_gate, s_up}, {b_gate, b_up}, inds, nullptr,
                       nullptr, m.h, nullptr, S, I, D, E, T, flag, topk};
      if (int rc = hip_status(fmxq::launch_moe_qmvs(gu, 2, 16, S, s), "switch_glu: gate/up"))
        return rc;
      fmxq::MoeArgs dn{m.h, nullptr, {w_down, nullptr}, {s_down, nullptr}, {b_down, nullptr},
                       inds, nullptr, nullptr, out, nullptr, S, D, I, E, S, flag, 1};
      return hip_status(fmxq::launch_moe_qmvs(dn, 1, 16, S, s), "switch_glu: down");
    }
    // Long expert runs (>= kGroupedMinRun slots) go to the grouped GEMM: gate and
    // up into g and u, silu * up into their h rows, then down.
    const int64_t max_tiles =
        fmxq::qmm_grouped_supported(I, D, T, bits, group_size) &&
                fmxq::qmm_grouped_supported(D, I, S, bits, group_size)
            ? grouped_max_tiles(S, E)
            : 0;
    if (int rc = moe_scratch(s, S, I, max_seg, &m, op, max_tiles, max_tiles ? I : 0, src))
      return rc;
    if (int rc = hip_status(fmxq::launch_sort_slots(inds, S, topk, E, m.order, m.rhs, m.lhs, s,
                                                    nullptr, m.seg, m.nseg, window, m.tiles,
                                                    m.ntile, (int)kGroupedMinRun,
                                                    fmxq::kGroupedTileRows),
                            "switch_glu: sort"))
      return rc;
    fmxq::MoeArgs gu{x, m.lhs, {w_gate, w_up}, {s_gate, s_up}, {b_gate, b_up}, m.rhs, m.seg,
                     m.nseg, m.h, nullptr, S, I, D, E, T, flag};
    if (int rc = hip_status(fmxq::launch_moe_qmvs(gu, 2, window, max_seg, s),
                            "switch_glu: gate/up"))
      return rc;
    if (max_tiles) {
      const fmxq::QmmArgs gg = grouped_args(x, w_gate, s_gate, b_gate, m.g, I, D, bits,
                                            group_size, m, m.lhs, nullptr, T, flag);
      if (int rc = hip_status(fmxq::launch_qmm_grouped(gg, max_tiles, s), "switch_glu: gate"))
        return rc;
      const fmxq::QmmArgs gup = grouped_args(x, w_up, s_up, b_up, m.u, I, D, bits, group_size,
                                             m, m.lhs, nullptr, T, flag);
      if (int rc = hip_status(fmxq::launch_qmm_grouped(gup, max_tiles, s), "switch_glu: up"))
        return rc;
      if (int rc = hip_status(fmxq::launch_silu_mul_tiles(m.g, m.u, m.h, m.tiles, m.ntile,
                                                          max_tiles, fmxq::kGroupedTileRows, I,
                                                          s),
                              "switch_glu: silu"))
        return rc;
    }
    fmxq::MoeArgs dn{m.h, nullptr, {w_down, nullptr}, {s_down, nullptr}, {b_down, nullptr},
                     m.rhs, m.seg, m.nseg, out, m.order, S, D, I, E, S, flag};
    if (int rc = hip_status(fmxq::launch_moe_qmvs(dn, 1, window, max_seg, s), "switch_glu: down"))
      return rc;
    if (!max_tiles) return FMXQ_OK;
    const fmxq::QmmArgs gd = grouped_args(m.h, w_down, s_down, b_down, out, D, I, bits,
                                          group_size, m, nullptr, m.order, S, flag);
    return hip_status(fmxq::launch_qmm_grouped(gd, max_tiles, s), "switch_glu: down");
  }
  // The reference sorts once routing reaches 64 slots (switch_glu.go:119-124).
  const bool sort = S >= 64 && E <= kSortMaxExperts;
  const size_t hbytes = align_up((size_t)S * I * sizeof(uint16_t));
  const size_t ibytes = align_up((size_t)S * sizeof(uint32_t));
  void* arena = nullptr;
  if (int rc = src.get(s, 2 * hbytes + (sort ? 3 * ibytes : 0), &arena, op)) return rc;
  uint16_t* gbuf = static_cast<uint16_t*>(arena);
  uint16_t* ubuf = reinterpret_cast<uint16_t*>(static_cast<char*>(arena) + hbytes);
  uint32_t* order = reinterpret_cast<uint32_t*>(static_cast<char*>(arena) + 2 * hbytes);
  uint32_t* rhs_s = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(order) + ibytes);
  uint32_t* lhs_s = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(rhs_s) + ibytes);

  fmxq::GatherArgs g{x, w_gate, s_gate, b_gate, nullptr, inds, gbuf, S, T, topk, 1, I, D, E,
                     group_size, bits, flag};
  if (sort) {
    if (int rc = hip_status(fmxq::launch_sort_slots(inds, S, topk, E, order, rhs_s, lhs_s, s),
                            "switch_glu: sort"))
      return rc;
    g.lhs = lhs_s;
    g.rhs = rhs_s;
    g.lhs_div = 1;
  }
  if (int rc = gather_dispatch(g, sort, s)) return rc;
  fmxq::GatherArgs u = g;
  u.w = w_up;
  u.scales = s_up;
  u.biases = b_up;
  u.y = ubuf;
  if (int rc = gather_dispatch(u, sort, s)) return rc;
  if (int rc = hip_status(fmxq::launch_silu_mul(gbuf, ubuf, gbuf, S * I, s), "switch_glu: silu"))
    return rc;
  fmxq::GatherArgs d{gbuf, w_down, s_down, b_down, nullptr, sort ? rhs_s : inds, out, S, S, 1,
                     1, D, I, E, group_size, bits, flag};
  if (sort) d.yrow = order;
  return gather_dispatch(d, sort, s);
}

}  // namespace

extern "C" int fmxq_switch_glu(const uint16_t* x, const uint32_t* inds, const uint32_t* w_gate,
                               const uint16_t* s_gate, const uint16_t* b_gate,
                               const uint32_t* w_up, const uint16_t* s_up, const uint16_t* b_up,
                               const uint32_t* w_down, const uint16_t* s_down,
                               const uint16_t* b_down, uint16_t* out, int64_t T, int64_t topk,
                               int64_t E, int64_t D, int64_t I, int group_size, int bits,
                               void* stream) {
  return switch_glu_impl(x, inds, w_gate, s_gate, b_gate, w_up, s_up, b_up, w_down, s_down,
                         b_down, out, T, topk, E, D, I, group_size, bits, stream,
                         ScratchSource(), "switch_glu");
}

extern "C" int fmxq_switch_glu_noalloc(const uint16_t* x, const uint32_t* inds,
                                       const uint32_t* w_gate, const uint16_t* s_gate,
                                       const uint16_t* b_gate, const uint32_t* w_up,
                                       const uint16_t* s_up, const uint16_t* b_up,
                                       const uint32_t* w_down, const uint16_t* s_down,
                                       const uint16_t* b_down, uint16_t* out, int64_t T,
                                       int64_t topk, int64_t E, int64_t D, int64_t I,
                                       int group_size, int bits, void* stream) {
  ScratchSource src;
  if (int rc = fmxq::noalloc_scratch(&src.fixed)) return rc;
  src.fixed_bytes = FMXQ_NOALLOC_SCRATCH_BYTES;
  return switch_glu_impl(x, inds, w_gate, s_gate, b_gate, w_up, s_up, b_up, w_down, s_down,
                         b_down, out, T, topk, E, D, I, group_size, bits, stream, src,
                         "switch_glu_noalloc");
}

extern "C" int fmxq_switch_glu_combine(
    const uint16_t* x, const uint32_t* inds, const uint32_t* w_gate, const uint16_t* s_gate,
    const uint16_t* b_gate, const uint32_t* w_up, const uint16_t* s_up, const uint16_t* b_up,
    const uint32_t* w_down, const uint16_t* s_down, const uint16_t* b_down,
    const uint16_t* weights, const uint16_t* shared, const uint16_t* shared_gate, uint16_t* out,
    int64_t T, int64_t topk, int64_t E, int64_t D, int64_t I, int group_size, int bits,
    void* stream) {
  const char* op = "switch_glu_combine";
  if (int rc = check_quant(group_size, bits, D, true, op)) return rc;
  if (int rc = check_quant(group_size, bits, I, true, op)) return rc;
  if (T < 0 || topk < 1 || E < 1 || D % 2 != 0)
    return fail(FMXQ_ERR_SHAPE, "%s: need T >= 0, top_k >= 1, E >= 1 and an even D", op);
  const int64_t S = T * topk;
  if (S == 0) return FMXQ_OK;
  if (!x || !inds || !w_gate || !s_gate || !b_gate || !w_up || !s_up || !b_up || !w_down ||
      !s_down || !b_down || !weights || !out)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null operand", op);
  if (shared_gate && !shared)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: shared_gate without shared", op);
  if (!aligned16(x) || !aligned16(w_gate) || !aligned16(w_up) || !aligned16(w_down))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: x and weights must be 16-byte aligned", op);
  if (S > 0x7fffffffLL) return fail(FMXQ_ERR_SHAPE, "%s: too many slots", op);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Decode-sized batches, and batches whose slots rarely share an expert: gate and
  // up into h (no sort), then one kernel for the down projection and the combine.
  if (fmxq::moe_combine_unsorted(S, E) &&
      fmxq::moe_down_combine_supported(T, topk, D, I, bits, group_size) &&
      fmxq::moe_qmvs_supported(I, D, bits, group_size) && aligned16(s_gate) &&
      aligned16(b_gate) && aligned16(s_up) && aligned16(b_up)) {
    uint32_t* flag = nullptr;
    if (int rc = device_flag(static_cast<hipStream_t>(stream), &flag)) return rc;
    MoeScratch m;
    if (int rc = moe_scratch(s, S, I, 1, &m, op)) return rc;
    fmxq::MoeArgs gu{x, nullptr, {w_gate, w_up}, {s_gate, s_up}, {b_gate, b_up}, inds, nullptr,
                     nullptr, m.h, nullptr, S, I, D, E, T, flag, topk};
    if (int rc = hip_status(fmxq::launch_moe_qmvs(gu, 2, 16, S, s), "switch_glu_combine: gate/up"))
      return rc;
    return hip_status(fmxq::launch_moe_down_combine(m.h, inds, w_down, s_down, b_down, weights,
                                                    shared, shared_gate, out, T, topk, E, D, I,
                                                    flag, s),
                      "switch_glu_combine: down/combine");
  }
  // Otherwise the two calls in sequence, the expert rows in the arena's slot 1.
  void* rows = nullptr;
  if (int rc = stream_arena(s, align_up((size_t)S * D * sizeof(uint16_t)), &rows, op, 1))
    return rc;
  if (int rc = switch_glu_impl(x, inds, w_gate, s_gate, b_gate, w_up, s_up, b_up, w_down, s_down,
                               b_down, static_cast<uint16_t*>(rows), T, topk, E, D, I, group_size,
                               bits, stream, ScratchSource(), op))
    return rc;
  return hip_status(fmxq::launch_moe_combine(static_cast<const uint16_t*>(rows), weights, shared,
                                             shared_gate, out, T, topk, D, s),
                    "switch_glu_combine: combine");
}

extern "C" int fmxq_moe_layer(
    const uint16_t* x, const uint32_t* inds, const uint32_t* w_gate, const uint16_t* s_gate,
    const uint16_t* b_gate, const uint32_t* w_up, const uint16_t* s_up, const uint16_t* b_up,
    const uint32_t* w_down, const uint16_t* s_down, const uint16_t* b_down,
    const uint16_t* weights, const uint32_t* sw_gate, const uint16_t* ss_gate,
    const uint16_t* sb_gate, const uint32_t* sw_up, const uint16_t* ss_up, const uint16_t* sb_up,
    const uint32_t* sw_down, const uint16_t* ss_down, const uint16_t* sb_down,
    const uint16_t* shared_gate, uint16_t* out, int64_t T, int64_t topk, int64_t E, int64_t D,
    int64_t I, int group_size, int bits, void* stream) {
  const char* op = "moe_layer";
  if (int rc = check_quant(group_size, bits, D, true, op)) return rc;
  if (int rc = check_quant(group_size, bits, I, true, op)) return rc;
  if (T < 0 || topk < 1 || E < 1 || D % 2 != 0)
    return fail(FMXQ_ERR_SHAPE, "%s: need T >= 0, top_k >= 1, E >= 1 and an even D", op);
  const int64_t S = T * topk;
  if (S == 0) return FMXQ_OK;
  if (!x || !inds || !w_gate || !s_gate || !b_gate || !w_up || !s_up || !b_up || !w_down ||
      !s_down || !b_down || !weights || !sw_gate || !ss_gate || !sb_gate || !sw_up || !ss_up ||
      !sb_up || !sw_down || !ss_down || !sb_down || !out)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null operand", op);
  if (!aligned16(x) || !aligned16(w_gate) || !aligned16(w_up) || !aligned16(w_down) ||
      !aligned16(sw_gate) || !aligned16(sw_up) || !aligned16(sw_down))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: x and weights must be 16-byte aligned", op);
  if (S + T > 0x7fffffffLL) return fail(FMXQ_ERR_SHAPE, "%s: too many slots", op);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // One token (decode): the shared expert rides along as one more gate/up segment
  // and one more wave of each down/combine block, two launches for the layer.
  if (T == 1 && topk <= 15 && fmxq::moe_combine_unsorted(S, E) && D >= 2048 && D <= 16384 &&
      fmxq::moe_down_combine_supported(T, topk, D, I, bits, group_size) &&
      fmxq::moe_qmvs_supported(I, D, bits, group_size) && aligned16(s_gate) &&
      aligned16(b_gate) && aligned16(s_up) && aligned16(b_up) && aligned16(ss_gate) &&
      aligned16(sb_gate) && aligned16(ss_up) && aligned16(sb_up)) {
    uint32_t* flag = nullptr;
    if (int rc = device_flag(s, &flag)) return rc;
    MoeScratch m;
    if (int rc = moe_scratch(s, S + T, I, 1, &m, op)) return rc;
    fmxq::MoeArgs gu{x, nullptr, {w_gate, w_up}, {s_gate, s_up}, {b_gate, b_up}, inds, nullptr,
                     nullptr, m.h, nullptr, S, I, D, E, T, flag, topk};
    gu.sh_w[0] = sw_gate;
    gu.sh_w[1] = sw_up;
    gu.sh_s[0] = ss_gate;
    gu.sh_s[1] = ss_up;
    gu.sh_b[0] = sb_gate;
    gu.sh_b[1] = sb_up;
    gu.sh_T = T;
    if (int rc = hip_status(fmxq::launch_moe_qmvs(gu, 2, 16, S, s), "moe_layer: gate/up"))
      return rc;
    return hip_status(fmxq::launch_moe_down_combine(m.h, inds, w_down, s_down, b_down, weights,
                                                    nullptr, shared_gate, out, T, topk, E, D, I,
                                                    flag, s, sw_down, ss_down, sb_down),
                      "moe_layer: down/combine");
  }
  // Sorted batches below the grouped GEMM's floor: the shared expert joins the
  // sort as expert id E with one slot per token (after the S routed slots), so its
  // segments ride in the routed gate/up and down launches; the rows land in the
  // arena's slot 1, routed then shared, and the combine reads both.
  {
    const int64_t Sa = S + T;
    const int window = fmxq::moe_window(Sa, E + 1);
    const int64_t max_seg = fmxq::moe_max_segments(Sa, E + 1, window);
    if (!fmxq::moe_combine_unsorted(S, E) && grouped_max_tiles(S, E) == 0 &&
        E + 1 <= kSortMaxExperts && max_seg <= kMaxSegmentsGrid &&
        fmxq::moe_qmvs_supported(I, D, bits, group_size) &&
        fmxq::moe_qmvs_supported(D, I, bits, group_size) && aligned16(s_gate) &&
        aligned16(b_gate) && aligned16(s_up) && aligned16(b_up) && aligned16(s_down) &&
        aligned16(b_down) && aligned16(ss_gate) && aligned16(sb_gate) && aligned16(ss_up) &&
        aligned16(sb_up) && aligned16(ss_down) && aligned16(sb_down)) {
      uint32_t* flag = nullptr;
      if (int rc = device_flag(s, &flag)) return rc;
      MoeScratch m;
      if (int rc = moe_scratch(s, Sa, I, max_seg, &m, op)) return rc;
      void* rows = nullptr;
      if (int rc = stream_arena(s, align_up((size_t)Sa * D * sizeof(uint16_t)), &rows, op, 1))
        return rc;
      uint16_t* y = static_cast<uint16_t*>(rows);
      if (int rc = hip_status(fmxq::launch_sort_slots(inds, S, topk, E, m.order, m.rhs, m.lhs, s,
                                                      nullptr, m.seg, m.nseg, window, nullptr,
                                                      nullptr, 0, 0, T),
                              "moe_layer: sort"))
        return rc;
      fmxq::MoeArgs gu{x, m.lhs, {w_gate, w_up}, {s_gate, s_up}, {b_gate, b_up}, m.rhs, m.seg,
                       m.nseg, m.h, nullptr, Sa, I, D, E, T, flag};
      gu.sh_w[0] = sw_gate;
      gu.sh_w[1] = sw_up;
      gu.sh_s[0] = ss_gate;
      gu.sh_s[1] = ss_up;
      gu.sh_b[0] = sb_gate;
      gu.sh_b[1] = sb_up;
      gu.sh_seg = true;
      if (int rc = hip_status(fmxq::launch_moe_qmvs(gu, 2, window, max_seg, s),
                              "moe_layer: gate/up"))
        return rc;
      fmxq::MoeArgs dn{m.h, nullptr, {w_down, nullptr}, {s_down, nullptr}, {b_down, nullptr},
                       m.rhs, m.seg, m.nseg, y, m.order, Sa, D, I, E, Sa, flag};
      dn.sh_w[0] = sw_down;
      dn.sh_s[0] = ss_down;
      dn.sh_b[0] = sb_down;
      dn.sh_seg = true;
      if (int rc = hip_status(fmxq::launch_moe_qmvs(dn, 1, window, max_seg, s), "moe_layer: down"))
        return rc;
      return hip_status(fmxq::launch_moe_combine(y, weights, y + S * D, shared_gate, out, T, topk,
                                                 D, s),
                        "moe_layer: combine");
    }
  }
  // Otherwise the shared expert as a one-expert SwitchGLU over every token (its
  // rows in the arena's slot 2), then the routed part with those rows as the
  // shared term.  Its all-zero expert ids live in slot 3, which only ever holds
  // zeros: a buffer is filled once, as far as the calls on it have needed.
  void* arena = nullptr;
  if (int rc = stream_arena(s, align_up((size_t)T * D * sizeof(uint16_t)), &arena, op, 2))
    return rc;
  uint16_t* rows = static_cast<uint16_t*>(arena);
  void* zarena = nullptr;
  if (int rc = stream_arena(s, align_up((size_t)T * sizeof(uint32_t)), &zarena, op, 3)) return rc;
  uint32_t* zinds = static_cast<uint32_t*>(zarena);
  // A fill recorded into a graph under capture has not run yet, so only an eager
  // fill counts.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  const bool capturing =
      hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone;
  bool filled = false;
  {
    std::lock_guard<std::mutex> lk(g_arena_mu);
    auto& z = g_zero_filled[zinds];
    filled = z >= T;
    if (!filled && !capturing) z = T;
  }
  if (!filled)
    if (int rc = hip_status(fmxq::launch_fill_u32(zinds, 0u, T, s), "moe_layer: shared ids"))
      return rc;
  if (int rc = switch_glu_impl(x, zinds, sw_gate, ss_gate, sb_gate, sw_up, ss_up, sb_up, sw_down,
                               ss_down, sb_down, rows, T, 1, 1, D, I, group_size, bits, stream,
                               ScratchSource(), op))
    return rc;
  return fmxq_switch_glu_combine(x, inds, w_gate, s_gate, b_gate, w_up, s_up, b_up, w_down,
                                 s_down, b_down, weights, rows, shared_gate, out, T, topk, E, D,
                                 I, group_size, bits, stream);
}

namespace {
int route_common(const void* logits, int logits_bf16, const float* bias, int64_t T, int64_t E,
                 int top_k, int n_group, int topk_group, float scale, bool norm, uint32_t* inds,
                 void* weights, int weights_bf16, bool group, void* stream, const char* op) {
  if (T < 0) return fail(FMXQ_ERR_SHAPE, "%s: negative token count %lld", op, (long long)T);
  if (E < 1 || E > fmxq::kRouteMaxExperts)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: %lld experts (1..%lld supported)", op, (long long)E,
                (long long)fmxq::kRouteMaxExperts);
  if (top_k < 1 || top_k > 64 || top_k > E)
    return fail(FMXQ_ERR_SHAPE, "%s: top_k=%d must be in 1..min(64, E=%lld)", op, top_k,
                (long long)E);
  if (group && (n_group < 1 || n_group > 64 || E % n_group != 0 || topk_group < 1 ||
                topk_group > n_group))
    return fail(FMXQ_ERR_SHAPE,
                "%s: n_group=%d must divide E=%lld (at most 64 groups) and topk_group=%d be in "
                "1..n_group", op, n_group, (long long)E, topk_group);
  if (T == 0) return FMXQ_OK;
  if (!logits || !inds || !weights) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null operand", op);
  const uintptr_t la = reinterpret_cast<uintptr_t>(logits);
  if ((logits_bf16 ? la & 1 : la & 3) || (reinterpret_cast<uintptr_t>(inds) & 3) ||
      (reinterpret_cast<uintptr_t>(weights) & (weights_bf16 ? 1 : 3)) ||
      (bias && (reinterpret_cast<uintptr_t>(bias) & 3)))
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: operands must be aligned to their element size", op);
  fmxq::RouteArgs a{logits, bias, inds, weights, T, E, top_k, n_group, topk_group, scale,
                    norm, logits_bf16 != 0, weights_bf16 != 0};
  return hip_status(fmxq::launch_route(a, group, static_cast<hipStream_t>(stream)), op);
}
}  // namespace

extern "C" int fmxq_route_softmax_topk(const void* logits, int logits_bf16, int64_t T,
                                       int64_t E, int top_k, bool norm_topk_prob,
                                       uint32_t* inds, void* weights, int weights_bf16,
                                       void* stream) {
  return route_common(logits, logits_bf16, nullptr, T, E, top_k, 1, 1, 1.f, norm_topk_prob, inds,
                      weights, weights_bf16, false, stream, "route_softmax_topk");
}

extern "C" int fmxq_route_group_topk(const void* gates, int gates_bf16, const float* bias,
                                     int64_t T, int64_t E, int top_k, int n_group, int topk_group,
                                     float routed_scaling_factor, bool norm_topk_prob,
                                     uint32_t* inds, void* weights, int weights_bf16,
                                     void* stream) {
  return route_common(gates, gates_bf16, bias, T, E, top_k, n_group, topk_group,
                      routed_scaling_factor, norm_topk_prob, inds, weights, weights_bf16, true,
                      stream, "route_group_topk");
}

extern "C" int fmxq_moe_combine(const uint16_t* y, const uint16_t* weights,
                                const uint16_t* shared, const uint16_t* shared_gate,
                                uint16_t* out, int64_t T, int64_t topk, int64_t D, void* stream) {
  const char* op = "moe_combine";
  if (T < 0 || topk < 1 || D < 0 || D % 2 != 0)
    return fail(FMXQ_ERR_SHAPE, "%s: need T >= 0, top_k >= 1 and an even D", op);
  if (T == 0 || D == 0) return FMXQ_OK;
  if (!y || !weights || !out) return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: null operand", op);
  if (shared_gate && !shared)
    return fail(FMXQ_ERR_INVALID_ARGUMENT, "%s: shared_gate without shared", op);
  return hip_status(fmxq::launch_moe_combine(y, weights, shared, shared_gate, out, T, topk, D,
                                             static_cast<hipStream_t>(stream)),
                    op);
}
