// fmxq_host.hpp -- host-side helpers shared by the two C-ABI files
// (fmxq_capi.cpp: raw pointer entry points; fmx_array.cpp: array handles).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fmxq_status.hpp"

namespace fmxq {

// FMXQ_OK for hipSuccess, else FMXQ_ERR_DEVICE with the HIP error string.
int hip_status(hipError_t e, const char* what);
// The index-error flag for a launch on `stream` (current device): a uint32
// __device__ word of that stream's own, or, while the stream is being captured
// into a graph, the device's graph word (a graph can be replayed on any
// stream).  Zero at load, cleared by fmxq_device_error when it reports; resolved
// without allocating (fmxq_device_state.hip).
int device_flag(hipStream_t stream, uint32_t** out);
// The words fmxq_device_error reads for `stream`: its own and the graph word.
int device_flags_to_check(hipStream_t stream, uint32_t** own, uint32_t** graph);
// The current device's fixed scratch of FMXQ_NOALLOC_SCRATCH_BYTES, shared by
// every fmxq_switch_glu_noalloc call on that device.
int noalloc_scratch(void** out);
// The quantization geometry every op supports: transpose, bits in {4, 8},
// group_size in {32, 64, 128}, K a positive multiple of group_size.
int check_quant(int group_size, int bits, int64_t K, bool transpose, const char* op);

}  // namespace fmxq
