// fmxq_blaslt.cpp -- the plain bf16 GEMM of the dequantize-then-GEMM path:
// y [M, N] = x [M, K] . wd [N, K]^T with wd the dequantized weights, fp32
// accumulation, through hipBLASLt.
//
// quantized_matmul at prefill sizes (M >= kDeqGemmMinM) spends most of its time
// in the GEMM; the fused prefill kernel dequantizes every weight tile once per M
// tile, and its tile machinery reaches ~70% of the vendor GEMM's speed.  Past
// that M, dequantizing W once into HBM (a bandwidth-bound pass) and running the
// library GEMM on bf16 is faster (MI355X, M = 2048: 290 -> 235 us on
// 14336x4096 with the old dequantizer).
//
// hipBLASLt is column-major.  Row-major y [M, N] is column-major y^T [N, M], so
// the call is D (N x M, ld ldy) = op(A) (N x K) . op(B) (K x M) with A = wd
// stored K x N (ld K) and transposed, B = x stored K x M (ld ldx), not
// transposed.  Algorithms that need workspace are neither requested nor taken
// (the call passes none): no split-K reduction buffer (and with it no memset)
// enters a captured graph.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "fmxq.h"
#include "fmxq_host.hpp"
#include "fmxq_internal.hpp"

namespace fmxq {
namespace {

struct GemmPlan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

std::mutex g_mu;
std::map<int, hipblasLtHandle_t> g_handles;
std::map<std::tuple<int, int64_t, int64_t, int64_t, int64_t, int64_t>, GemmPlan> g_plans;

const char* status_name(hipblasStatus_t st) {
  switch (st) {
    case HIPBLAS_STATUS_NOT_INITIALIZED: return "not initialized";
    case HIPBLAS_STATUS_ALLOC_FAILED: return "allocation failed";
    case HIPBLAS_STATUS_INVALID_VALUE: return "invalid value";
    case HIPBLAS_STATUS_ARCH_MISMATCH: return "architecture mismatch";
    case HIPBLAS_STATUS_EXECUTION_FAILED: return "execution failed";
    case HIPBLAS_STATUS_INTERNAL_ERROR: return "internal error";
    case HIPBLAS_STATUS_NOT_SUPPORTED: return "not supported";
    default: return "error";
  }
}

int lt_fail(hipblasStatus_t st, const char* what) {
  return fail(FMXQ_ERR_DEVICE, "quantized_matmul: hipBLASLt %s: %s", what, status_name(st));
}

constexpr int kCandidates = 16;

// The plan for one shape on one device, made on first use and kept for the
// process: the descriptors and the heuristic's first algorithm that needs no
// workspace (the call passes none).  No algorithm of that kind: FMXQ_ERR_UNSUPPORTED,
// and the caller takes another kernel.
int plan_for(int dev, hipblasLtHandle_t h, int64_t M, int64_t N, int64_t K, int64_t ldx,
             int64_t ldy, GemmPlan** out) {
  auto key = std::make_tuple(dev, M, N, K, ldx, ldy);
  auto it = g_plans.find(key);
  if (it != g_plans.end()) {
    *out = &it->second;
    return FMXQ_OK;
  }
  GemmPlan p;
  hipblasStatus_t st = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
  if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail(st, "matmul descriptor");
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
  if ((st = hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, K, N, K)) != HIPBLAS_STATUS_SUCCESS ||
      (st = hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, K, M, ldx)) != HIPBLAS_STATUS_SUCCESS ||
      (st = hipblasLtMatrixLayoutCreate(&p.lc, HIP_R_16BF, N, M, ldy)) != HIPBLAS_STATUS_SUCCESS)
    return lt_fail(st, "matrix layout");
  hipblasLtMatmulPreference_t pref = nullptr;
  if ((st = hipblasLtMatmulPreferenceCreate(&pref)) != HIPBLAS_STATUS_SUCCESS)
    return lt_fail(st, "preference");
  const uint64_t ws = 0;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                        sizeof(ws));
  hipblasLtMatmulHeuristicResult_t res[kCandidates];
  int n = 0;
  st = hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.la, p.lb, p.lc, p.lc, pref, kCandidates, res,
                                       &n);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail(st, "heuristic");
  int pick = -1;
  for (int i = 0; i < n && pick < 0; ++i)
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize == 0) pick = i;
  if (pick < 0)
    return fail(FMXQ_ERR_UNSUPPORTED,
                "quantized_matmul: hipBLASLt has no workspace-free algorithm for %lldx%lldx%lld",
                (long long)M, (long long)N, (long long)K);
  p.algo = res[pick].algo;
  *out = &(g_plans[key] = p);
  return FMXQ_OK;
}

}  // namespace

int gemm_bf16_plan(int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy, hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(FMXQ_ERR_DEVICE, "hipGetDevice failed");
  std::lock_guard<std::mutex> lk(g_mu);
  hipblasLtHandle_t& h = g_handles[dev];
  if (!h) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
      return fail(FMXQ_ERR_INVALID_ARGUMENT,
                  "quantized_matmul: the GEMM library is first used during graph capture; run "
                  "the same shape once outside capture first");
    const hipblasStatus_t st = hipblasLtCreate(&h);
    if (st != HIPBLAS_STATUS_SUCCESS) {
      h = nullptr;
      return lt_fail(st, "create");
    }
  }
  GemmPlan* p = nullptr;
  return plan_for(dev, h, M, N, K, ldx, ldy, &p);
}

int gemm_bf16_xwt(const uint16_t* x, int64_t ldx, const uint16_t* wd, uint16_t* y, int64_t ldy,
                  int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  if (int rc = gemm_bf16_plan(M, N, K, ldx, ldy, stream)) return rc;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(FMXQ_ERR_DEVICE, "hipGetDevice failed");
  std::lock_guard<std::mutex> lk(g_mu);
  hipblasLtHandle_t h = g_handles[dev];
  GemmPlan* p = nullptr;
  if (int rc = plan_for(dev, h, M, N, K, ldx, ldy, &p)) return rc;
  const float alpha = 1.f, beta = 0.f;
  const hipblasStatus_t st = hipblasLtMatmul(h, p->desc, &alpha, wd, p->la, x, p->lb, &beta, y,
                                             p->lc, y, p->lc, &p->algo, nullptr, 0, stream);
  if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail(st, "matmul");
  return FMXQ_OK;
}

}  // namespace fmxq
