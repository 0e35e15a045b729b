"""Algorithmic work of the quantized-linear path and MI355X roofline constants.

These are the figures bench.py divides by measured kernel time.  They count
what the operation must move/compute, never what an implementation happens to
move: packed weights plus per-group scale/bias bytes, activations in and out.
"""
from __future__ import annotations

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s (spec)
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s (spec, no sparsity)


def quantized_tensor_bytes(shape, bits: int, group_size: int, mode: str = "affine") -> int:
    """Stored bytes of a quantized tensor: packed values plus per-group overhead.

    Same arithmetic as the reference's size estimator TensorQuantizedBytes
    (quant/oq.go:315-332): affine groups carry a bf16 scale and a bf16 bias
    (4 bytes), mxfp4 one byte, mxfp8 two; rank < 2 or a last axis that the group
    does not divide stays bf16."""
    n = 1
    for d in shape:
        n *= d
    if len(shape) < 2:
        return n * 2
    last = shape[-1]
    if last % group_size != 0:
        return n * 2
    rows = n // max(last, 1)
    groups = last // group_size
    per_group = {"mxfp4": 1, "mxfp8": 2}.get(mode, 4)
    return (n * bits + 7) // 8 + rows * groups * per_group


def qmm_bytes(M: int, N: int, K: int, bits: int, group_size: int = 64) -> int:
    """HBM bytes of y[M,N] = x[M,K] . deq(W[N,K])^T: weights + x + y."""
    return quantized_tensor_bytes((N, K), bits, group_size) + M * K * 2 + M * N * 2


def qmm_flops(M: int, N: int, K: int) -> int:
    return 2 * M * N * K


def moe_bytes(M: int, D: int, I: int, topk: int, distinct_experts: int, bits: int,
              group_size: int = 64, shared_I: int = 0) -> int:
    """One SwitchGLU MoE layer: U distinct experts' gate/up/down weights (+ shared
    expert), x in and y out, and the routing ids/weights (4 + 4 bytes per slot)."""
    per_expert = 2 * quantized_tensor_bytes((I, D), bits, group_size) + \
        quantized_tensor_bytes((D, I), bits, group_size)
    shared = 0
    if shared_I:
        shared = 2 * quantized_tensor_bytes((shared_I, D), bits, group_size) + \
            quantized_tensor_bytes((D, shared_I), bits, group_size)
    return distinct_experts * per_expert + shared + 2 * M * D * 2 + M * topk * 8


def moe_flops(M: int, D: int, I: int, topk: int, shared_I: int = 0) -> int:
    return 6 * M * topk * D * I + 6 * M * D * shared_I


def roofline_time_s(nbytes: float, flops: float) -> float:
    return max(nbytes / (HBM_PEAK_GBS * 1e9), flops / (BF16_MFMA_PEAK_TFLOPS * 1e12))
