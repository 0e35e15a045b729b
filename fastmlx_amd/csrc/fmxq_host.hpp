// fmxq_host.hpp -- host-side helpers shared by the two C-ABI files
// (fmxq_capi.cpp: raw pointer entry points; fmx_array.cpp: array handles).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fmxq_status.hpp"

namespace fmxq {

// FMXQ_OK for hipSuccess, else FMXQ_ERR_DEVICE with the HIP error string.
int hip_status(hipError_t e, const char* what);
// The index-error flag of `stream` on the current device: a uint32 __device__
// word of that stream's own (zero at load, cleared by fmxq_device_error when it
// reports), resolved without allocating (fmxq_device_state.hip).
int device_flag(hipStream_t stream, uint32_t** out);
// The current device's fixed scratch of FMXQ_NOALLOC_SCRATCH_BYTES, shared by
// every fmxq_switch_glu_noalloc call on that device.
int noalloc_scratch(void** out);
// The quantization geometry every op supports: transpose, bits in {4, 8},
// group_size in {32, 64, 128}, K a positive multiple of group_size.
int check_quant(int group_size, int bits, int64_t K, bool transpose, const char* op);
// y [M, N] = x [M, K] . wd [N, K]^T in bf16 with fp32 accumulation, through
// hipBLASLt on `stream` (fmxq_blaslt.cpp).  No workspace.  gemm_bf16_plan makes
// (or finds) the shape's plan and returns FMXQ_ERR_UNSUPPORTED when the library
// has no workspace-free algorithm for it.
int gemm_bf16_plan(int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy, hipStream_t stream);
int gemm_bf16_xwt(const uint16_t* x, int64_t ldx, const uint16_t* wd, uint16_t* y, int64_t ldy,
                  int64_t M, int64_t N, int64_t K, hipStream_t stream);

}  // namespace fmxq
