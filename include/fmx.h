/*
 * fmx.h -- array-handle layer of libfmxq.so with mlx-c's calling convention.
 *
 * The reference binds MLX through mlx-c (mlxgo/binding_cgo.go:19-23).  For the
 * quantized-linear path it calls exactly these functions; each fmx_* below has
 * the same argument list and ownership rules as the mlx_* it replaces, so a Go
 * binding file built with a `hip` tag can mirror binding_cgo.go line for line:
 *
 *   mlx_array_new / _new_data / _free          binding_cgo.go:71-251
 *   mlx_array_ndim / _dim / _dtype / _size     binding_cgo.go:152-201
 *   mlx_array_eval, mlx_array_data_float32/int32 binding_cgo.go:204-241
 *   mlx_default_gpu_stream_new, mlx_synchronize binding_cgo.go:254-275
 *   mlx_quantized_matmul                        binding_cgo.go:636-643
 *   mlx_gather_qmm                              binding_cgo.go:645-673
 *   mlx_dequantize                              binding_cgo.go:675-682
 *   mlx_quantize, mlx_reshape, mlx_split, mlx_swapaxes, mlx_contiguous
 *                                               binding_cgo.go:684-697,398-483,715-731
 *
 * Ownership: an op writes a newly allocated result into *res (created empty by
 * fmx_array_new); inputs are borrowed; optional operands (biases, lhs_indices,
 * rhs_indices) are passed as empty arrays.  Every function returns 0 on
 * success; on failure *res is left unchanged and fmxq_last_error() has the
 * reason (statuses are the fmxq_status codes of fmxq.h).
 * Execution is eager on the stream's HIP queue; fmx_array_eval waits for the
 * array's stream and reports any device-side index error (FMXQ_ERR_INDEX).
 * Arrays live in device memory (HBM).  Result buffers come from a per-stream
 * cache and return to it on fmx_array_free, so steady-state calls do not call
 * hipMalloc.  An input produced on another stream is waited for with an event,
 * and a buffer read by other streams is fenced before the cache reuses it.
 * Streams, like MLX's, live until the process ends; fmx_stream_free releases
 * only the handle.
 */
#ifndef FMX_H
#define FMX_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same order as the reference's Dtype enum (mlxgo/dtype.go:35-50). */
typedef enum {
  FMX_BOOL = 0,
  FMX_UINT8,
  FMX_UINT16,
  FMX_UINT32,
  FMX_UINT64,
  FMX_INT8,
  FMX_INT16,
  FMX_INT32,
  FMX_INT64,
  FMX_FLOAT16,
  FMX_FLOAT32,
  FMX_BFLOAT16,
  FMX_COMPLEX64,
  FMX_FLOAT64
} fmx_dtype;

typedef struct fmx_array_ {
  void* ctx;
} fmx_array;

typedef struct fmx_stream_ {
  void* ctx;
} fmx_stream;

/* ---- arrays ---- */
fmx_array fmx_array_new(void);
/* Copies size(shape)*dtype bytes of host data to a new device array
 * (mlx_array_new_data).  data may be NULL only for an empty shape product. */
fmx_array fmx_array_new_data(const void* data, const int* shape, int dim, fmx_dtype dtype);
/* Wraps an existing device buffer without taking ownership (for callers that
 * manage device memory themselves); freeing the handle leaves the buffer. */
fmx_array fmx_array_new_device(void* device_ptr, const int* shape, int dim, fmx_dtype dtype);
int fmx_array_free(fmx_array a);
size_t fmx_array_ndim(const fmx_array a);
int fmx_array_dim(const fmx_array a, int dim);
fmx_dtype fmx_array_dtype(const fmx_array a);
size_t fmx_array_size(const fmx_array a);
size_t fmx_array_nbytes(const fmx_array a);
/* Device pointer of the array's data (NULL for an empty handle). */
void* fmx_array_device_ptr(const fmx_array a);
int fmx_array_eval(fmx_array a);
/* Host copies, valid until the array is freed; float32 accepts float32, bf16
 * and float16 arrays (converted), int32 accepts int32 and uint32 arrays. */
const float* fmx_array_data_float32(fmx_array a);
const int32_t* fmx_array_data_int32(fmx_array a);
/* Copies the raw element bytes to host memory dst (nbytes). */
int fmx_array_to_host(void* dst, size_t nbytes, const fmx_array a);

/* ---- streams ---- */
fmx_stream fmx_default_gpu_stream_new(void);
fmx_stream fmx_stream_new(void);
/* Wraps a caller-owned hipStream_t (passed as void*). */
fmx_stream fmx_stream_wrap(void* hip_stream);
int fmx_stream_free(fmx_stream s);
int fmx_synchronize(fmx_stream s);

/* ---- the quantized-linear ops (mlx-c argument lists) ---- */
/* x [..., K] bf16; w [N, K*bits/32] uint32; scales/biases [N, K/group] bf16;
 * res [..., N] bf16.  transpose must be true. */
int fmx_quantized_matmul(fmx_array* res, const fmx_array x, const fmx_array w,
                         const fmx_array scales, const fmx_array biases, bool transpose,
                         int group_size, int bits, const fmx_stream s);
/* x [X..., Mx, K]; w [E, N, K*bits/32]; lhs_indices / rhs_indices integer arrays
 * (or empty: the arange over x's / w's batch).  lhs and rhs broadcast to the
 * output batch shape B; res [B..., Mx, N]:
 *     res[i] = x[lhs[i]] . deq(w[rhs[i]])^T. */
int fmx_gather_qmm(fmx_array* res, const fmx_array x, const fmx_array w,
                   const fmx_array scales, const fmx_array biases, const fmx_array lhs_indices,
                   const fmx_array rhs_indices, bool transpose, int group_size, int bits,
                   bool sorted_indices, const fmx_stream s);
/* w [..., K*bits/32] -> res [..., K] bf16. */
int fmx_dequantize(fmx_array* res, const fmx_array w, const fmx_array scales,
                   const fmx_array biases, int group_size, int bits, const fmx_stream s);

/* ---- fused neighbours of the ops on the path ---- */
/* qlinearBias (compute/models/quant.go:105-111): quantized_matmul followed by
 * the broadcast add of bias [N] bf16 (empty: no add), fused into the epilogue. */
int fmx_quantized_matmul_bias(fmx_array* res, const fmx_array x, const fmx_array w,
                              const fmx_array scales, const fmx_array biases,
                              const fmx_array bias, bool transpose, int group_size, int bits,
                              const fmx_stream s);
/* MoE combine (qwen3next_forward.go:520-523, deepseekv3_forward.go:434-440):
 * res = sum_j y[..., j, :] * weights[..., j]  (+ shared, times sigmoid(shared_gate)
 * when shared_gate is given).  y [..., k, D] bf16, weights [..., k] bf16,
 * shared [..., D] bf16 or empty, shared_gate [..., 1] or [...] bf16 or empty;
 * res [..., D]. */
int fmx_moe_combine(fmx_array* res, const fmx_array y, const fmx_array weights,
                    const fmx_array shared, const fmx_array shared_gate, const fmx_stream s);
/* qembed (compute/models/quant.go:117-142): take rows idx of the packed table,
 * its scales and biases, then dequantize -- one kernel.  idx integer [...];
 * res [..., K] bf16. */
int fmx_dequantize_rows(fmx_array* res, const fmx_array w, const fmx_array scales,
                        const fmx_array biases, const fmx_array idx, int group_size, int bits,
                        const fmx_stream s);
/* switchGLUCore over quantized stacked experts (switch_glu.go:79-153):
 * x [B, L, D], inds [B, L, top_k] -> res [B, L, top_k, D]. */
int fmx_switch_glu(fmx_array* res, const fmx_array x, const fmx_array inds,
                   const fmx_array w_gate, const fmx_array s_gate, const fmx_array b_gate,
                   const fmx_array w_up, const fmx_array s_up, const fmx_array b_up,
                   const fmx_array w_down, const fmx_array s_down, const fmx_array b_down,
                   int group_size, int bits, const fmx_stream s);
/* MoE routers over a row of expert logits (bf16 or float32 [..., E], E <= 1024);
 * results inds [..., top_k] uint32 and weights [..., top_k] in the logits' dtype,
 * largest first, equal scores to the lower expert id.
 * fmx_route_softmax_topk: qwen3NextMoE's softmax top-k with optional
 * renormalization (compute/models/qwen3next_forward.go:513-518).
 * fmx_route_group_topk: DeepSeek-V3's group-limited sigmoid router routeExperts
 * (compute/models/deepseekv3_forward.go:452-491); bias float32 [E] or empty.
 * On failure neither result is touched. */
int fmx_route_softmax_topk(fmx_array* inds, fmx_array* weights, const fmx_array logits,
                           int top_k, bool norm_topk_prob, const fmx_stream s);
int fmx_route_group_topk(fmx_array* inds, fmx_array* weights, const fmx_array gates,
                         const fmx_array bias, int top_k, int n_group, int topk_group,
                         float routed_scaling_factor, bool norm_topk_prob, const fmx_stream s);

/* ---- weight ingest ---- */

/* A parsed safetensors container header (compute/safetensors.go:101-165,
 * ParseSafetensorsHeader): tensors in (begin, name) order with their dtype tag,
 * shape and [begin, end) range in the data buffer, the optional __metadata__
 * string map, the header length and the data start (8 + header length).
 * Validation as the reference: known dtype, begin <= end, end within the data,
 * end - begin = numel * dtype size.  Statuses: FMXQ_ERR_SHAPE for a buffer
 * shorter than 8 bytes (ErrShortBuffer) or a declared header longer than the
 * buffer (ErrHeaderTooLarge); FMXQ_ERR_INVALID_ARGUMENT for the rest. */
typedef struct fmx_st_header_ fmx_st_header;
int fmx_safetensors_parse(const uint8_t* blob, uint64_t len, fmx_st_header** out);
void fmx_safetensors_free(fmx_st_header* h);
uint64_t fmx_safetensors_header_size(const fmx_st_header* h);
uint64_t fmx_safetensors_data_start(const fmx_st_header* h);
int64_t fmx_safetensors_count(const fmx_st_header* h);
/* Tensor i (SafetensorsHeader.Tensors[i]); pointers stay valid until free. */
int fmx_safetensors_tensor(const fmx_st_header* h, int64_t i, const char** name,
                           const char** dtype, int* ndim, const int64_t** shape,
                           uint64_t* begin, uint64_t* end);
/* Index of the named tensor or -1 (SafetensorsHeader.Tensor, safetensors.go:77-83). */
int64_t fmx_safetensors_find(const fmx_st_header* h, const char* name);
/* Entries of __metadata__, or -1 when the header has none (a nil map). */
int64_t fmx_safetensors_metadata_count(const fmx_st_header* h);
int fmx_safetensors_metadata(const fmx_st_header* h, int64_t i, const char** key,
                             const char** value);
/* The array dtype of a safetensors tag; the float8 tags have none
 * (mlxgoDtype, compute/loader.go:13-42). */
int fmx_safetensors_dtype(const char* tag, fmx_dtype* out);
/* Offset in the blob of the data range [begin, end) after data_start,
 * bounds-checked against the blob length (TensorBytes, compute/loader.go:47-55). */
int fmx_safetensors_slice(uint64_t blob_len, uint64_t data_start, uint64_t begin,
                          uint64_t end, uint64_t* offset);
/* Upload tensor i's bytes unchanged into a new device array of its dtype
 * (the per-tensor step of LoadTensors, compute/loader.go:61-84). */
int fmx_safetensors_load(fmx_array* res, const uint8_t* blob, uint64_t len,
                         const fmx_st_header* h, int64_t i);
/* a's bytes as dtype, the last axis scaled by the element-size ratio (mlxgo.View
 * as remapInt4 uses it, compute/models/deepseekv3.go:513). */
int fmx_view(fmx_array* res, const fmx_array a, fmx_dtype dtype, const fmx_stream s);
/* n arrays of one shape and dtype joined on a new axis; axis 0 only (mlxgo.Stack
 * as stackExperts uses it, compute/models/deepseekv3.go:564-592). */
int fmx_stack(fmx_array* res, const fmx_array* arrays, size_t n, int axis, const fmx_stream s);
/* -8 * scale in the scale's dtype (bf16, f16, f32): the affine bias of an int4
 * checkpoint (scaleNeg8, compute/models/deepseekv3.go:539-551). */
int fmx_scale_neg8(fmx_array* res, const fmx_array scale, const fmx_stream s);

/* ---- the kv_b_proj absorption (absorbKVB, compute/models/deepseekv3.go:609-679) ---- */
/* MLX affine quantization (fmxq_quantize has the arithmetic): w [..., K] bf16,
 * at least 2-D -> res_0 packed [..., K*bits/32] uint32, res_1 scales and res_2
 * biases [..., K/group_size] bf16.  Replaces mlx_quantize
 * (mlxgo/binding_cgo.go:684-697). */
int fmx_quantize(fmx_array* res_0, fmx_array* res_1, fmx_array* res_2, const fmx_array w,
                 int group_size, int bits, const fmx_stream s);
/* Arrays of this layer are always row-major and contiguous, so the next three
 * return contiguous copies where MLX returns views; the values are MLX's. */
/* mlx_reshape (binding_cgo.go:398-406): one entry of shape may be -1. */
int fmx_reshape(fmx_array* res, const fmx_array a, const int* shape, size_t ndim,
                const fmx_stream s);
/* mlx_split at explicit indices (binding_cgo.go:463-483).  This ABI has no vector
 * type: res points to n_res = num_indices + 1 handles, part i covering
 * [indices[i-1], indices[i]) of axis; indices ascend within [0, dim]. */
int fmx_split(fmx_array* res, size_t n_res, const fmx_array a, const int* indices,
              size_t num_indices, int axis, const fmx_stream s);
/* mlx_swapaxes (binding_cgo.go:715-722). */
int fmx_swapaxes(fmx_array* res, const fmx_array a, int axis1, int axis2, const fmx_stream s);
/* mlx_contiguous (binding_cgo.go:724-731): a row-major copy. */
int fmx_contiguous(fmx_array* res, const fmx_array a, bool allow_col_major, const fmx_stream s);

#ifdef __cplusplus
}
#endif
#endif /* FMX_H */
