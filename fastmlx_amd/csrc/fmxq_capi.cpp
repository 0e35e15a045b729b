// fmxq_capi.cpp -- extern "C" entry points of libfmxq.so (declared in include/fmxq.h).
//
// Validation happens here, before anything is enqueued: a failing call returns a
// nonzero fmxq_status with a message and leaves the stream untouched, the
// contract mlxgo relies on when it frees the result handle on rc != 0
// (mlxgo/binding_cgo.go:636-643).  Dispatch by M:
//   M <= kQmvMaxM  -> decode GEMV (fmxq_qmv.hip), bandwidth bound, no MFMA
//   M >  kQmvMaxM  -> LDS-dequant MFMA GEMM (fmxq_qmm.hip)
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/fmxq.h"
#include "fmxq_internal.hpp"

namespace {

std::mutex g_err_mu;
// The returned pointer must survive until the next failure; keep two buffers
// and alternate so a reader of the previous message is not overwritten mid-read.
char g_err_buf[2][512];
int g_err_slot = 0;

int fail(int code, const char* fmt, ...) {
  char tmp[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(tmp, sizeof(tmp), fmt, ap);
  va_end(ap);
  std::lock_guard<std::mutex> lk(g_err_mu);
  g_err_slot ^= 1;
  std::snprintf(g_err_buf[g_err_slot], sizeof(g_err_buf[0]), "%s", tmp);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return FMXQ_OK;
  return fail(FMXQ_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_quant(int group_size, int bits, int64_t K, bool transpose, const char* op) {
  if (!transpose)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: transpose=false is not supported (the reference "
                "always passes true)", op);
  if (bits != 4 && bits != 8)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: bits=%d not supported (4 or 8)", op, bits);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(FMXQ_ERR_UNSUPPORTED, "%s: group_size=%d not supported (32, 64 or 128)", op,
                group_size);
  if (K <= 0 || K % group_size != 0)
    return fail(FMXQ_ERR_SHAPE, "%s: K=%lld must be a positive multiple of group_size=%d", op,
                (long long)K, group_size);
  return FMXQ_OK;
}

// Per-device error flag raised by gather kernels.
std::mutex g_flag_mu;
std::vector<uint32_t*> g_flags;

int device_flag(uint32_t** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(FMXQ_ERR_DEVICE, "hipGetDevice failed");
  std::lock_guard<std::mutex> lk(g_flag_mu);
  if ((int)g_flags.size() <= dev) g_flags.resize(dev + 1, nullptr);
  if (!g_flags[dev]) {
    uint32_t* p = nullptr;
    hipError_t e = hipMalloc(&p, sizeof(uint32_t));
    if (e != hipSuccess) return hip_status(e, "hipMalloc(error flag)");
    e = hipMemset(p, 0, sizeof(uint32_t));
    if (e != hipSuccess) return hip_status(e, "hipMemset(error flag)");
    g_flags[dev] = p;
  }
  *out = g_flags[dev];
  return FMXQ_OK;
}

// Split-K workspace of the MFMA GEMM, one per (device, stream) so that calls on
// different streams never share it.  Both arrays are zero between calls: the
// kernel's last split per tile restores them.  Growth needs hipMalloc, which is
// refused while the stream is being captured into a graph.
struct SplitWs {
  float* ws = nullptr;
  int64_t ws_floats = 0;
  uint32_t* counters = nullptr;
  int64_t n_counters = 0;
};
std::mutex g_ws_mu;
std::map<std::pair<int, hipStream_t>, SplitWs> g_ws;
std::vector<void*> g_retired;

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
    // A graph captured earlier may still hold the old buffers, so they are kept
    // alive (growth is monotonic, at most doubling the footprint) rather than freed.
    if (w.ws) g_retired.push_back(w.ws);
    if (w.counters) g_retired.push_back(w.counters);
    w.ws = nws;
    w.ws_floats = nf;
    w.counters = ncnt;
    w.n_counters = nc;
  }
  *ws = w.ws;
  *cnt = w.counters;
  return FMXQ_OK;
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
  if (M <= fmxq::kQmvMaxM) return hip_status(fmxq::launch_qmv(a, s), op);
  if (M <= fmxq::kSkinnyMaxM && fmxq::qmv_mfma_supported(a))
    return hip_status(fmxq::launch_qmv_mfma(a, s), op);
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

const char* fmxq_last_error(void) {
  std::lock_guard<std::mutex> lk(g_err_mu);
  return g_err_buf[g_err_slot];
}

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

int fmxq_quantized_matmul(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                          const uint16_t* biases, uint16_t* y, int64_t M, int64_t N,
                          int64_t K, bool transpose, int group_size, int bits, void* stream) {
  return qmm_common(x, w, scales, biases, nullptr, y, M, N, K, transpose, group_size, bits,
                    stream, "quantized_matmul");
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
  if (int rc = device_flag(&flag)) return rc;
  fmxq::GatherArgs a{x,      w,     scales,  biases, lhs_indices, rhs_indices, y,
                     batch,  x_batch, lhs_div, Mx,   N,           K,           E,
                     group_size, bits, flag};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (sorted_indices && batch * Mx >= fmxq::kGroupedMinSlots && fmxq::gather_mfma_supported(a))
    return hip_status(fmxq::launch_gather_mfma(a, s), op);
  return hip_status(fmxq::launch_gather_qmv(a, s), op);
}

int fmxq_device_error(void* stream) {
  uint32_t* flag = nullptr;
  if (int rc = device_flag(&flag)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (int rc = hip_status(hipStreamSynchronize(s), "device_error: synchronize")) return rc;
  uint32_t v = 0;
  if (int rc = hip_status(hipMemcpy(&v, flag, sizeof(v), hipMemcpyDeviceToHost),
                          "device_error: read flag"))
    return rc;
  if (v == 0) return FMXQ_OK;
  if (int rc = hip_status(hipMemset(flag, 0, sizeof(uint32_t)), "device_error: clear flag"))
    return rc;
  return fail(FMXQ_ERR_INDEX, "gather_qmm: an index was out of range (outputs zeroed)");
}

}  // extern "C"
