/*
 * fmxq.h -- C ABI of the MI355X quantized-linear library (libfmxq.so).
 *
 * Kernel-level entry points: plain device pointers, element counts and a HIP
 * stream (hipStream_t passed as void*, NULL = the null stream).  Every call is
 * asynchronous on that stream and returns an fmxq_status; a nonzero status
 * means nothing was enqueued, and fmxq_last_error() describes why.
 *
 * Each entry replaces one mlx-c call the reference binds through cgo:
 *   fmxq_quantized_matmul  <- mlx_quantized_matmul  (mlxgo/binding_cgo.go:636-643)
 *   fmxq_gather_qmm        <- mlx_gather_qmm        (mlxgo/binding_cgo.go:645-673)
 *   fmxq_dequantize        <- mlx_dequantize        (mlxgo/binding_cgo.go:675-682)
 *   fmxq_quantize          <- mlx_quantize          (mlxgo/binding_cgo.go:684-697)
 * The array-handle layer with mlx-c's exact argument lists is in fmx.h.  The other
 * entries (SwitchGLU and the MoE layer, the routers, the grouped product and the
 * allocation-free SwitchGLU) fuse what the reference's callers compose from those
 * calls, or have no counterpart; each declaration says which.
 *
 * Data layout (MLX affine quantization):
 *   x       [M, K] bf16 (uint16 bit patterns), row-major
 *   w       [N, K*bits/32] uint32, LSB-first packing (32/bits values per word)
 *   scales  [N, K/group_size] bf16;  biases [N, K/group_size] bf16
 *   y       [M, N] bf16
 * Supported: bits in {4, 8}, group_size in {32, 64, 128}, K a multiple of
 * group_size, transpose = true.  Anything else returns FMXQ_ERR_UNSUPPORTED
 * rather than a wrong answer (the oQ policy in quant/oq.go:21-27 can emit 2/3/5/6
 * bits; those are rejected).
 * All pointers must be 16-byte aligned, and rows of x must be 16-byte aligned
 * (K % 8 == 0 holds for every supported K).
 */
#ifndef FMXQ_H
#define FMXQ_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  FMXQ_OK = 0,
  FMXQ_ERR_INVALID_ARGUMENT = 1, /* null pointer, negative size, misalignment */
  FMXQ_ERR_UNSUPPORTED = 2,      /* bits / group_size / transpose combination */
  FMXQ_ERR_SHAPE = 3,            /* sizes that do not fit together */
  FMXQ_ERR_INDEX = 4,            /* an index out of range (reported by fmxq_device_error) */
  FMXQ_ERR_DEVICE = 5            /* a HIP runtime error */
} fmxq_status;

/* Library version, major*10000 + minor*100 + patch. */
int fmxq_version(void);

/* Text of the most recent failure in this process (any thread).  The pointer
 * stays valid until the next failing call. */
const char* fmxq_last_error(void);

/* w = scale * q + bias per group of group_size along K, written as bf16:
 * out [rows, K].  Rounding: bf16(bf16(q * s) + b), both to nearest-even --
 * MLX's CPU composition multiply(q, scales) then add(., biases).
 * Replaces mlx_dequantize (mlxgo/binding_cgo.go:675-682). */
int fmxq_dequantize(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                    uint16_t* out, int64_t rows, int64_t K, int group_size, int bits,
                    void* stream);

/* MLX affine quantization, the inverse of fmxq_dequantize: w [rows, K] bf16 ->
 * wq [rows, K*bits/32] uint32, scales and biases [rows, K/group_size] bf16.
 * Per group of group_size values, in fp32: delta = max((max - min) /
 * (2^bits - 1), 1e-7); the end of larger magnitude is the edge (min with scale
 * +delta, else max with scale -delta); q0 = rint(edge / scale); when q0 != 0,
 * scale = edge / q0 and bias = edge, else bias = 0; q = clamp(rint((w - bias) /
 * scale), 0, 2^bits - 1).  scale and bias are rounded to nearest-even bf16.
 * Scales can be negative.  Caller: the kv_b_proj absorption of DeepSeek-V3
 * (compute/models/deepseekv3.go:662-669).
 * Replaces mlx_quantize (mlxgo/binding_cgo.go:684-697). */
int fmxq_quantize(const uint16_t* w, uint32_t* wq, uint16_t* scales, uint16_t* biases,
                  int64_t rows, int64_t K, int group_size, int bits, void* stream);

/* qembed over a quantized table (compute/models/quant.go:117-142: take rows idx
 * of w, scales and biases, then dequantize) in one kernel:
 *     out[i] (K) = deq(table row idx[i]),  i < n_idx,  idx[i] < table_rows.
 * An out-of-range index zeroes its row and raises the device error flag
 * (fmxq_device_error reports it). */
int fmxq_dequantize_rows(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                         const uint32_t* idx, uint16_t* out, int64_t n_idx, int64_t table_rows,
                         int64_t K, int group_size, int bits, void* stream);

/* y [M, N] = x [M, K] . deq(W)^T, fp32 accumulation, bf16 output.
 * transpose must be true (the only value the reference passes, quant.go:98).
 * Replaces mlx_quantized_matmul (mlxgo/binding_cgo.go:636-643). */
int fmxq_quantized_matmul(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                          const uint16_t* biases, uint16_t* y, int64_t M, int64_t N,
                          int64_t K, bool transpose, int group_size, int bits, void* stream);

/* No counterpart in the reference: n quantized_matmul products that read the same
 * x, for the projections a model computes from one activation (q, k and v; gate
 * and up), in one launch where the shapes allow (M = 1, int4 group 64, K a multiple
 * of 2048, 16-byte aligned operands) and one launch each otherwise.  Product i is
 * y[i] [M, N[i]] = x [M, K] . deq(w[i], scales[i], biases[i])^T with the operands of
 * fmxq_quantized_matmul; 1 <= n <= 4.  The values agree with fmxq_quantized_matmul's
 * to the same tolerance, not bit for bit: a grouped launch picks its wave shape from
 * the group's total rows, which can change the order of a row's sum. */
int fmxq_quantized_matmul_group(const uint16_t* x, int n, const uint32_t* const* w,
                                const uint16_t* const* scales, const uint16_t* const* biases,
                                uint16_t* const* y, const int64_t* N, int64_t M, int64_t K,
                                bool transpose, int group_size, int bits, void* stream);

/* qlinearBias (compute/models/quant.go:105-111): quantized_matmul followed by a
 * broadcast add of the additive bias [N] (bf16), fused into the epilogue with
 * the op chain's rounding: bf16(bf16(x . deq(W)^T) + bias).  bias may be NULL. */
int fmxq_quantized_matmul_bias(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                               const uint16_t* biases, const uint16_t* bias, uint16_t* y,
                               int64_t M, int64_t N, int64_t K, bool transpose,
                               int group_size, int bits, void* stream);

/* gather_qmm over a stacked expert weight W [E, N, K*bits/32] (scales/biases
 * [E, N, K/group_size]).  The output has `batch` items of Mx rows each:
 *     y[i] (Mx x N) = x[xi] (Mx x K) . deq(W[rhs_indices[i]])^T
 * with xi = lhs_indices[i] when lhs_indices is non-NULL, else xi = i / lhs_div
 * (lhs_div = 1 is the identity; lhs_div = top_k is SwitchGLU's broadcast of one
 * token row against its top_k experts, switch_glu.go:122-130).  x holds x_batch
 * items.  Index arrays are uint32 (int32 bit patterns are accepted; negative
 * values count as out of range).  sorted_indices is a locality hint and never
 * changes the result.  An out-of-range index writes zeros for that item and
 * raises the device error flag read by fmxq_device_error.
 * Replaces mlx_gather_qmm (mlxgo/binding_cgo.go:645-673). */
int fmxq_gather_qmm(const uint16_t* x, const uint32_t* w, const uint16_t* scales,
                    const uint16_t* biases, const uint32_t* lhs_indices,
                    const uint32_t* rhs_indices, uint16_t* y, int64_t batch, int64_t x_batch,
                    int64_t lhs_div, int64_t Mx, int64_t N, int64_t K, int64_t E,
                    bool transpose, int group_size, int bits, bool sorted_indices,
                    void* stream);

/* The SwitchGLU expert MLP over stacked quantized experts -- switchGLUCore with
 * switchLinearQuantized as the projection (compute/models/switch_glu.go:79-153):
 *     out[t, j] = down_e( silu(gate_e(x[t])) * up_e(x[t]) ),  e = inds[t, j]
 * x [T, D] bf16; inds [T, top_k] uint32; gate/up stacks [E, I, D*bits/32] with
 * [E, I, D/group] scales/biases; down stack [E, D, I*bits/32] with [E, D, I/group];
 * out [T, top_k, D] bf16 (the [B, L, top_k, D] result before the router weighting).
 * Below 64 slots (T*top_k) each slot is a gathered GEMV, as the reference's
 * unsorted branch (switch_glu.go:124-130); from 64 slots on the slots are
 * counting-sorted by expert on the device, projected by the grouped kernel
 * and scattered back to token order (the sorted branch, :135-150).  Each op's
 * result is rounded to bf16 as in the reference chain (gather_qmm, sigmoid,
 * mul, mul).  Intermediates live in a per-stream scratch area the library
 * grows on first use of a shape (not allowed during graph capture).
 * Out-of-range expert ids give zero rows and raise the fmxq_device_error flag. */
int fmxq_switch_glu(const uint16_t* x, const uint32_t* inds, const uint32_t* w_gate,
                    const uint16_t* s_gate, const uint16_t* b_gate, const uint32_t* w_up,
                    const uint16_t* s_up, const uint16_t* b_up, const uint32_t* w_down,
                    const uint16_t* s_down, const uint16_t* b_down, uint16_t* out, int64_t T,
                    int64_t top_k, int64_t E, int64_t D, int64_t I, int group_size, int bits,
                    void* stream);

/* One MoE layer's routed part: fmxq_switch_glu followed by fmxq_moe_combine,
 * out [T, D] = sum_j bf16(y[t, j] * weights[t, j]) (+ the shared term), the
 * expert outputs y never leaving the chip for decode-sized batches
 * (qwen3next_forward.go:510-525, deepseekv3_forward.go:427-442).  Arguments are
 * those of the two calls; the op chain and its bf16 roundings are theirs.  Up to
 * 16 routing slots, and up to 256 slots routed over at least twice as many
 * experts (int4, group 64), the slots stay unsorted and the down projection and
 * the weighted sum run as one kernel; otherwise the expert rows go through a
 * per-stream buffer. */
int fmxq_switch_glu_combine(const uint16_t* x, const uint32_t* inds, const uint32_t* w_gate,
                            const uint16_t* s_gate, const uint16_t* b_gate,
                            const uint32_t* w_up, const uint16_t* s_up, const uint16_t* b_up,
                            const uint32_t* w_down, const uint16_t* s_down,
                            const uint16_t* b_down, const uint16_t* weights,
                            const uint16_t* shared, const uint16_t* shared_gate, uint16_t* out,
                            int64_t T, int64_t top_k, int64_t E, int64_t D, int64_t I,
                            int group_size, int bits, void* stream);

/* One MoE layer with its shared expert: out [T, D] = sum_j bf16(y[t, j] *
 * weights[t, j]) plus the shared expert MLP of x (sigmoid-gated by shared_gate
 * [T] when given), deepseekv3_forward.go:427-442 (shared = mlp(x), added) and
 * qwen3next_forward.go:510-525 (sigmoid(shared_expert_gate(x)) * shared_expert(x)).
 * The routed arguments are those of fmxq_switch_glu_combine; sw_ / ss_ / sb_ are
 * the shared expert's gate, up and down triples laid out as one-expert stacks
 * ([1, I, D*bits/32], [1, D, I*bits/32], ...), with the routed experts' I.  The
 * shared expert's op chain and roundings are those of a one-expert SwitchGLU.
 * For one token (decode) the shared expert runs inside the routed kernels (one
 * more gate/up segment, one more wave per down/combine block; top_k <= 15).
 * Batches whose routed slots are sorted (below 4096 slots) sort it in as one
 * more expert with one slot per token, so it runs inside the routed gate/up and
 * down launches.  Otherwise it runs as fmxq_switch_glu on every token, then
 * fmxq_switch_glu_combine adds its rows.  Extends fmxq_switch_glu_combine; the
 * reference computes the shared expert with its own qlinear calls. */
int fmxq_moe_layer(const uint16_t* x, const uint32_t* inds, const uint32_t* w_gate,
                   const uint16_t* s_gate, const uint16_t* b_gate, const uint32_t* w_up,
                   const uint16_t* s_up, const uint16_t* b_up, const uint32_t* w_down,
                   const uint16_t* s_down, const uint16_t* b_down, const uint16_t* weights,
                   const uint32_t* sw_gate, const uint16_t* ss_gate, const uint16_t* sb_gate,
                   const uint32_t* sw_up, const uint16_t* ss_up, const uint16_t* sb_up,
                   const uint32_t* sw_down, const uint16_t* ss_down, const uint16_t* sb_down,
                   const uint16_t* shared_gate, uint16_t* out, int64_t T, int64_t top_k,
                   int64_t E, int64_t D, int64_t I, int group_size, int bits, void* stream);

/* Bytes of device memory each GPU holds, from library load to process exit, for
 * fmxq_switch_glu_noalloc's scratch (a file-scope __device__ array). */
#define FMXQ_NOALLOC_SCRATCH_BYTES (32u << 20)

/* fmxq_switch_glu without any allocation.  This entry point has no counterpart
 * in the reference.  It exists for callers that cannot allocate device memory:
 * code under HIP graph capture, tight serving loops, and harnesses that forbid
 * hipMalloc.
 * - Same arguments, kernels and results as fmxq_switch_glu.
 * - The scratch (sorted slots, segment table, intermediate activations) lives in
 *   one fixed FMXQ_NOALLOC_SCRATCH_BYTES buffer per GPU, not in a per-stream
 *   arena.  That covers, for example, 5120 routed slots at I = 512 or 2048
 *   slots at I = 2048.
 * - A call that needs more scratch returns FMXQ_ERR_SHAPE before anything is
 *   enqueued.
 * - Every call on one GPU shares that GPU's buffer, and nothing in it needs to
 *   start at zero.  Calls that overlap on one GPU (concurrent streams, or a
 *   graph replayed while another call runs) race on it and must be serialized
 *   by the caller.
 * - It calls no hipMalloc, hipFree or allocating library routine. */
int fmxq_switch_glu_noalloc(const uint16_t* x, const uint32_t* inds, const uint32_t* w_gate,
                            const uint16_t* s_gate, const uint16_t* b_gate,
                            const uint32_t* w_up, const uint16_t* s_up, const uint16_t* b_up,
                            const uint32_t* w_down, const uint16_t* s_down,
                            const uint16_t* b_down, uint16_t* out, int64_t T, int64_t top_k,
                            int64_t E, int64_t D, int64_t I, int group_size, int bits,
                            void* stream);

/* MoE combine: out[t] = sum_j y[t, j] * weights[t, j] (+ shared term), the
 * weighted top-k sum of qwen3next_forward.go:519-520 / deepseekv3_forward.go:436-437.
 * y [T, top_k, D], weights [T, top_k], out [T, D], all bf16; D even.  With shared
 * [T, D] non-NULL the shared expert output is added (deepseekv3_forward.go:438-440);
 * with shared_gate [T] also non-NULL it is first scaled by sigmoid(shared_gate)
 * (qwen3next_forward.go:522-524).  Rounding follows the op chain: each product
 * to bf16, the sum in fp32 rounded once, the gated shared term and the final
 * add each rounded to bf16. */
int fmxq_moe_combine(const uint16_t* y, const uint16_t* weights, const uint16_t* shared,
                     const uint16_t* shared_gate, uint16_t* out, int64_t T, int64_t top_k,
                     int64_t D, void* stream);

/* Softmax MoE router of qwen3NextMoE (compute/models/qwen3next_forward.go:513-518):
 *     gates = softmax(logits[t]); inds[t] = the top_k experts by gate (equal gates
 *     to the lower index); weights[t, j] = gates[inds[t, j]], divided by their sum
 *     when norm_topk_prob.
 * logits [T, E] (bf16 when logits_bf16, else fp32), E <= 1024, top_k <= min(E, 64);
 * inds [T, top_k] uint32 and weights [T, top_k] (bf16 when weights_bf16, else fp32),
 * both in selection order (largest gate first).  fp32 arithmetic throughout. */
int fmxq_route_softmax_topk(const void* logits, int logits_bf16, int64_t T, int64_t E,
                            int top_k, bool norm_topk_prob, uint32_t* inds, void* weights,
                            int weights_bf16, void* stream);

/* DeepSeek-V3 group-limited router: routeExperts (compute/models/deepseekv3_forward.go:
 * 452-491), restated on the CPU as GroupExpertSelect (deepseekv3.go:305-384).
 *     o = sigmoid(gates[t]); b = o + bias; with n_group > 1 the groups outside the
 *     topk_group best (a group scores the sum of its two best b) get b = 0; inds[t] =
 *     the top_k experts by b (ties to the lower index); weights = o[inds], divided by
 *     their sum when norm_topk_prob and top_k > 1, times routed_scaling_factor.
 * gates [T, E] (bf16 when gates_bf16, else fp32); bias [E] fp32 or NULL; n_group
 * divides E (<= 64 groups), 1 <= topk_group <= n_group; outputs as for the softmax
 * router. */
int fmxq_route_group_topk(const void* gates, int gates_bf16, const float* bias, int64_t T,
                          int64_t E, int top_k, int n_group, int topk_group,
                          float routed_scaling_factor, bool norm_topk_prob, uint32_t* inds,
                          void* weights, int weights_bf16, void* stream);

/* Synchronizes `stream`, then reports (and clears) the device-side error flags
 * that gather kernels raise on an out-of-range index: returns FMXQ_OK or
 * FMXQ_ERR_INDEX (FMXQ_ERR_DEVICE if a wide-GEMM block gave up waiting).  Two
 * flags are read:
 *   - the stream's own, raised by kernels enqueued on `stream` outside graph
 *     capture (other streams' own flags are neither read nor cleared).  Streams
 *     get these in order of first use, 4095 per device; beyond 4095 streams on
 *     one device they are shared in turn (two streams sharing a word then see
 *     each other's errors);
 *   - the device's graph flag, raised by kernels that were captured into a
 *     graph, wherever the graph is replayed (the replay stream is not known at
 *     capture).  Every stream's query reads and clears it, so with graphs
 *     replayed on several streams at once the report names the device, not the
 *     stream. */
int fmxq_device_error(void* stream);

#ifdef __cplusplus
}
#endif
#endif /* FMXQ_H */
