/*
 * fmxq_oracle.h -- CPU restatement of MLX affine group quantization, the
 * arithmetic that fastmlx's quantized linear path reaches through cgo.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the parity tests,
 * the smoke check and the CPU-baseline leg of bench.py compare against.  The
 * product (libfmxq.so) never links, loads or calls it.
 *
 * Reference call sites restated here:
 *   mlxgo/binding_cgo.go:636-643   QuantizedMatMul -> mlx_quantized_matmul
 *   mlxgo/binding_cgo.go:645-673   GatherQMM       -> mlx_gather_qmm
 *   mlxgo/binding_cgo.go:675-682   Dequantize      -> mlx_dequantize
 *   mlxgo/binding_cgo.go:684-697   Quantize        -> mlx_quantize
 *   compute/models/switch_glu.go:107-153  switchGLUCore choreography
 *   compute/models/qwen3next_forward.go:510-535, deepseekv3_forward.go:427-442
 *
 * Layouts (MLX, transpose=true):
 *   w       [rows, K*bits/32] uint32, element k of a row at bit (k % (32/bits))*bits
 *           of word k / (32/bits) (LSB first)
 *   scales  [rows, K/group] bf16,  biases [rows, K/group] bf16
 *   x       [M, K] bf16 row-major,  y [M, N] bf16
 * bf16 values travel as uint16_t bit patterns.
 */
#ifndef FMXQ_ORACLE_H
#define FMXQ_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Rounding sequences for dequantize.  DEQ_MLX is the definition the build
 * adopts: MLX's CPU composition multiply(q, scales) then add(., biases), each a
 * bf16 op that rounds its result to nearest-even.  DEQ_FUSED rounds once.
 * DEQ_EXACT keeps the affine value s*q + b unrounded (s*q is exact in fp32;
 * the add rounds to fp32 only): the products an integer-domain kernel forms as
 * s*sum(x q) + b*sum(x).  The per-element parity bounds of the tests compare
 * each kernel against the definition it computes (EXACT or FUSED); the
 * published 2e-2 metric is checked against DEQ_MLX. */
enum { ORACLE_DEQ_MLX = 0, ORACLE_DEQ_FUSED = 1, ORACLE_DEQ_EXACT = 2 };

float oracle_bf16_to_f32(uint16_t h);
uint16_t oracle_f32_to_bf16(float f);

/* q value of element k of a packed row. */
uint32_t oracle_unpack(const uint32_t *row_words, int64_t k, int bits);

/* out[r, k] = deq(w, s, b); returns 0, or -1 on unsupported bits/group. */
int oracle_dequantize(const uint32_t *w, const uint16_t *scales,
                      const uint16_t *biases, uint16_t *out, int64_t rows,
                      int64_t K, int group_size, int bits, int mode);

/* MLX affine quantization of w [rows, K] (bf16) into wq [rows, K*bits/32],
 * scales and biases [rows, K/group] (bf16): the requantize step of absorbKVB
 * (deepseekv3.go:662-669, mlx_quantize via mlxgo/binding_cgo.go:684-697).
 * The per-group arithmetic is in fmxq_oracle.c.  Returns 0, or -1 on
 * unsupported bits/group. */
int oracle_quantize(const uint16_t *w, uint32_t *wq, uint16_t *scales, uint16_t *biases,
                    int64_t rows, int64_t K, int group_size, int bits);

/* y[m, n] = sum_k x[m,k] * deq(W)[n,k], accumulated in fp32 in ascending k,
 * rounded once to bf16.  y_f32 (optional) receives the unrounded sums.
 * rows_sel (optional, length M) selects which rows of x to evaluate; NULL
 * means all rows 0..M-1.  Threads: OpenMP over n. */
int oracle_qmm_f32(const uint16_t *x, const uint32_t *w, const uint16_t *scales,
                   const uint16_t *biases, uint16_t *y, float *y_f32,
                   int64_t M, int64_t N, int64_t K, int group_size, int bits,
                   int mode);

/* Same product in fp64 over the dequantized bf16 weights: the "truth" used to
 * separate kernel error from oracle error. */
int oracle_qmm_f64(const uint16_t *x, const uint32_t *w, const uint16_t *scales,
                   const uint16_t *biases, double *y, int64_t M, int64_t N,
                   int64_t K, int group_size, int bits, int mode);

/* Flattened gather_qmm: for each i in [0, S): y[i, :] = x[xrow[i], :] .
 * deq(W[expert[i]])^T.  W stacked [E, N, K*bits/32], scales/biases [E, N, K/g].
 * Returns -2 if an expert id is out of range. */
int oracle_gather_qmm(const uint16_t *x, const uint32_t *w,
                      const uint16_t *scales, const uint16_t *biases,
                      const int32_t *xrow, const int32_t *expert, uint16_t *y,
                      int64_t S, int64_t E, int64_t N, int64_t K,
                      int group_size, int bits, int mode);

/* SwitchGLU over stacked quantized experts (switch_glu.go:107-153), one token
 * slot at a time, rounding each MLX op's result to bf16 the way the op chain
 * does: g = gather_qmm(x, Wg), u = gather_qmm(x, Wu), h = silu(g) * u (silu and
 * mul each bf16-rounded), out = gather_qmm(h, Wd).
 *   x [T, D], inds [T, k] -> out [T, k, D]
 *   gate/up stacked [E, I, D*bits/32], down stacked [E, D, I*bits/32].
 * token_sel (optional, length n_sel) evaluates only those tokens, writing
 * out[j, k, D] for the j-th selected token.  mode is the dequant definition of
 * all three products (ORACLE_DEQ_*).  hscale (optional, [n_sel, k, D]) receives
 * sqrt(sum_i (h_i wd_i)^2) for each output: the scale by which a one-ulp change
 * of the bf16 intermediates h_i can move that output. */
int oracle_switch_glu(const uint16_t *x, const int32_t *inds,
                      const uint32_t *wg, const uint16_t *sg, const uint16_t *bg,
                      const uint32_t *wu, const uint16_t *su, const uint16_t *bu,
                      const uint32_t *wd, const uint16_t *sd, const uint16_t *bd,
                      uint16_t *out, int64_t T, int64_t topk, int64_t E,
                      int64_t D, int64_t I, int group_size, int bits,
                      const int32_t *token_sel, int64_t n_sel, int mode,
                      double *hscale);

/* The CPU baseline: the same fp32-accumulated product as oracle_qmm_f32 with
 * the dequantization factored per group (s * sum(x q) + b * sum(x)), the form a
 * vectorising compiler turns into SIMD code.  Threads: OpenMP over n. */
int oracle_qmm_cpu_fast(const uint16_t *x, const uint32_t *w,
                        const uint16_t *scales, const uint16_t *biases,
                        uint16_t *y, int64_t M, int64_t N, int64_t K,
                        int group_size, int bits);

int oracle_num_threads(void);

/* MoE routers (double arithmetic; top-k by a stable descending sort, so equal
 * scores go to the lower index).
 * oracle_route_group_topk restates GroupExpertSelect
 * (compute/models/deepseekv3.go:305-384) row by row: gates [T, E] fp32, bias [E]
 * fp32 or NULL, inds [T, k], scores [T, k] in selection order.
 * oracle_route_softmax_topk restates the router of qwen3NextMoE
 * (compute/models/qwen3next_forward.go:513-518): softmax over the row, the top_k
 * gates, renormalized over the selection when norm. */
int oracle_route_group_topk(const float *gates, const float *bias, int64_t T, int64_t E,
                            int top_k, int n_group, int topk_group, double scale, int norm,
                            int32_t *inds, double *scores);
int oracle_route_softmax_topk(const float *logits, int64_t T, int64_t E, int top_k, int norm,
                              int32_t *inds, double *weights);

#ifdef __cplusplus
}
#endif
#endif
