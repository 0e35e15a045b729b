"""torch-facing wrappers over the raw C ABI (include/fmxq.h).

Tensors are device buffers only: bf16 values travel as ``torch.bfloat16`` or
``torch.int16``/``torch.uint16`` bit patterns, packed weights as ``torch.int32``
or ``torch.uint32``, indices as ``torch.int32``/``torch.uint32``.  Every call
is enqueued on torch's current HIP stream.  Nothing here computes on the CPU.
"""
from __future__ import annotations

import torch

from ._lib import check, load

_BF16_LIKE = (torch.bfloat16, torch.int16, torch.uint16)
_U32_LIKE = (torch.int32, torch.uint32)


def _dev(t: torch.Tensor, name: str, dtypes) -> int:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on the GPU (got {t.device})")
    if t.dtype not in dtypes:
        raise TypeError(f"{name} has dtype {t.dtype}, expected one of {dtypes}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def dequantize(w, scales, biases, group_size: int = 64, bits: int = 4, out=None):
    """MLX dequantize: [..., K*bits/32] packed -> [..., K] bf16."""
    K = w.shape[-1] * 32 // bits
    rows = w.numel() // max(w.shape[-1], 1)
    if out is None:
        out = torch.empty(*w.shape[:-1], K, dtype=torch.bfloat16, device=w.device)
    check(load().fmxq_dequantize(_dev(w, "w", _U32_LIKE), _dev(scales, "scales", _BF16_LIKE),
                                 _dev(biases, "biases", _BF16_LIKE), _dev(out, "out", _BF16_LIKE),
                                 rows, K, group_size, bits, _stream(w)))
    return out


def quantize(w, group_size: int = 64, bits: int = 4, out=None):
    """MLX affine quantize: bf16 [..., K] -> (packed [..., K*bits/32] int32 words,
    scales [..., K/group] bf16, biases [..., K/group] bf16); ``out`` may hold the
    three result tensors."""
    K = w.shape[-1]
    rows = w.numel() // max(K, 1)
    if K % group_size:
        raise ValueError(f"K={K} is not a multiple of group_size={group_size}")
    if out is None:
        wq = torch.empty(*w.shape[:-1], K * bits // 32, dtype=torch.int32, device=w.device)
        scales = torch.empty(*w.shape[:-1], K // group_size, dtype=torch.bfloat16,
                             device=w.device)
        biases = torch.empty_like(scales)
    else:
        wq, scales, biases = out
    check(load().fmxq_quantize(_dev(w, "w", _BF16_LIKE), _dev(wq, "wq", _U32_LIKE),
                               _dev(scales, "scales", _BF16_LIKE),
                               _dev(biases, "biases", _BF16_LIKE), rows, K, group_size, bits,
                               _stream(w)))
    return wq, scales, biases


def quantized_matmul(x, w, scales, biases, transpose: bool = True, group_size: int = 64,
                     bits: int = 4, bias=None, out=None):
    """y = x @ deq(W)^T over x [..., K]; W [N, K*bits/32]; y [..., N] bf16."""
    K = x.shape[-1]
    N = w.shape[0]
    M = x.numel() // max(K, 1)
    if w.shape[-1] * 32 // bits != K:
        raise ValueError(f"x has K={K} but w packs {w.shape[-1] * 32 // bits} values per row")
    if out is None:
        out = torch.empty(*x.shape[:-1], N, dtype=torch.bfloat16, device=x.device)
    lib = load()
    args = (_dev(x, "x", _BF16_LIKE), _dev(w, "w", _U32_LIKE),
            _dev(scales, "scales", _BF16_LIKE), _dev(biases, "biases", _BF16_LIKE))
    if bias is None:
        check(lib.fmxq_quantized_matmul(*args, _dev(out, "out", _BF16_LIKE), M, N, K, transpose,
                                        group_size, bits, _stream(x)))
    else:
        check(lib.fmxq_quantized_matmul_bias(*args, _dev(bias, "bias", _BF16_LIKE),
                                             _dev(out, "out", _BF16_LIKE), M, N, K, transpose,
                                             group_size, bits, _stream(x)))
    return out


def quantized_matmul_group(x, mats, group_size: int = 64, bits: int = 4, outs=None):
    """Several products of the same x [..., K]: mats is a list of (w, scales, biases)
    triples (1 to 4), the result a list of y [..., N_i] bf16 (one launch where the
    shapes allow, fmxq_quantized_matmul_group)."""
    import ctypes

    K = x.shape[-1]
    M = x.numel() // max(K, 1)
    n = len(mats)
    for w, _, _ in mats:
        if w.shape[-1] * 32 // bits != K:
            raise ValueError(f"x has K={K} but w packs {w.shape[-1] * 32 // bits} values per row")
    if outs is None:
        outs = [torch.empty(*x.shape[:-1], w.shape[0], dtype=torch.bfloat16, device=x.device)
                for w, _, _ in mats]
    P = ctypes.c_void_p * n
    ws = P(*[_dev(w, "w", _U32_LIKE) for w, _, _ in mats])
    ss = P(*[_dev(s, "scales", _BF16_LIKE) for _, s, _ in mats])
    bs = P(*[_dev(b, "biases", _BF16_LIKE) for _, _, b in mats])
    ys = P(*[_dev(y, "out", _BF16_LIKE) for y in outs])
    Ns = (ctypes.c_int64 * n)(*[w.shape[0] for w, _, _ in mats])
    check(load().fmxq_quantized_matmul_group(_dev(x, "x", _BF16_LIKE), n, ws, ss, bs, ys, Ns, M, K,
                                             True, group_size, bits, _stream(x)))
    return outs


def gather_qmm(x, w, scales, biases, rhs_indices, lhs_indices=None, lhs_div: int = 1,
               transpose: bool = True, group_size: int = 64, bits: int = 4,
               sorted_indices: bool = False, out=None):
    """Flat-index gather_qmm (raw ABI form).

    x [x_batch, Mx, K]; w [E, N, K*bits/32]; rhs_indices [batch];
    lhs_indices [batch] or None (then item i reads x[i // lhs_div]).
    Returns y [batch, Mx, N]."""
    if x.dim() != 3:
        raise ValueError("x must be [x_batch, Mx, K] in the flat form")
    x_batch, Mx, K = x.shape
    E, N = w.shape[0], w.shape[1]
    batch = rhs_indices.numel()
    if out is None:
        out = torch.empty(batch, Mx, N, dtype=torch.bfloat16, device=x.device)
    lhs_ptr = None if lhs_indices is None else _dev(lhs_indices, "lhs_indices", _U32_LIKE)
    check(load().fmxq_gather_qmm(_dev(x, "x", _BF16_LIKE), _dev(w, "w", _U32_LIKE),
                                 _dev(scales, "scales", _BF16_LIKE),
                                 _dev(biases, "biases", _BF16_LIKE), lhs_ptr,
                                 _dev(rhs_indices, "rhs_indices", _U32_LIKE),
                                 _dev(out, "out", _BF16_LIKE), batch, x_batch, lhs_div, Mx, N, K,
                                 E, transpose, group_size, bits, sorted_indices, _stream(x)))
    return out


def switch_glu(x, inds, gate, up, down, group_size: int = 64, bits: int = 4, out=None):
    """SwitchGLU over stacked quantized experts (switchGLUCore).

    x [T, D] bf16; inds [T, top_k] int32/uint32; gate/up/down are (w, scales, biases)
    triples with w [E, I, D*bits/32] (gate, up) and [E, D, I*bits/32] (down).
    Returns [T, top_k, D] bf16."""
    T, D = x.shape
    topk = inds.shape[-1]
    E, I = gate[0].shape[0], gate[0].shape[1]
    if out is None:
        out = torch.empty(T, topk, D, dtype=torch.bfloat16, device=x.device)
    p = [_dev(x, "x", _BF16_LIKE), _dev(inds, "inds", _U32_LIKE)]
    for name, (w, s, b) in (("gate", gate), ("up", up), ("down", down)):
        p += [_dev(w, f"{name}.w", _U32_LIKE), _dev(s, f"{name}.scales", _BF16_LIKE),
              _dev(b, f"{name}.biases", _BF16_LIKE)]
    check(load().fmxq_switch_glu(*p, _dev(out, "out", _BF16_LIKE), T, topk, E, D, I, group_size,
                                 bits, _stream(x)))
    return out


def switch_glu_combine(x, inds, gate, up, down, weights, shared=None, shared_gate=None,
                       group_size: int = 64, bits: int = 4, out=None):
    """One MoE layer's routed part: switch_glu then moe_combine in one call.

    weights [T, top_k] bf16; shared [T, D] (optional) is added, sigmoid-gated by
    shared_gate [T] when given.  Returns [T, D] bf16."""
    T, D = x.shape
    topk = inds.shape[-1]
    E, I = gate[0].shape[0], gate[0].shape[1]
    if out is None:
        out = torch.empty(T, D, dtype=torch.bfloat16, device=x.device)
    p = [_dev(x, "x", _BF16_LIKE), _dev(inds, "inds", _U32_LIKE)]
    for name, (w, s, b) in (("gate", gate), ("up", up), ("down", down)):
        p += [_dev(w, f"{name}.w", _U32_LIKE), _dev(s, f"{name}.scales", _BF16_LIKE),
              _dev(b, f"{name}.biases", _BF16_LIKE)]
    sp = None if shared is None else _dev(shared, "shared", _BF16_LIKE)
    gp = None if shared_gate is None else _dev(shared_gate, "shared_gate", _BF16_LIKE)
    check(load().fmxq_switch_glu_combine(*p, _dev(weights, "weights", _BF16_LIKE), sp, gp,
                                         _dev(out, "out", _BF16_LIKE), T, topk, E, D, I,
                                         group_size, bits, _stream(x)))
    return out


def moe_layer(x, inds, gate, up, down, weights, shared_expert, shared_gate=None,
              group_size: int = 64, bits: int = 4, out=None):
    """switch_glu_combine with the shared expert computed in the same call.

    shared_expert = (gate, up, down) triples of a one-expert stack; shared_gate [T]
    (optional) sigmoid-gates its output.  Returns [T, D] bf16."""
    T, D = x.shape
    topk = inds.shape[-1]
    E, I = gate[0].shape[0], gate[0].shape[1]
    if out is None:
        out = torch.empty(T, D, dtype=torch.bfloat16, device=x.device)
    p = [_dev(x, "x", _BF16_LIKE), _dev(inds, "inds", _U32_LIKE)]
    for name, (w, s, b) in (("gate", gate), ("up", up), ("down", down)):
        p += [_dev(w, f"{name}.w", _U32_LIKE), _dev(s, f"{name}.scales", _BF16_LIKE),
              _dev(b, f"{name}.biases", _BF16_LIKE)]
    p.append(_dev(weights, "weights", _BF16_LIKE))
    for name, (w, s, b) in zip(("shared.gate", "shared.up", "shared.down"), shared_expert):
        p += [_dev(w, f"{name}.w", _U32_LIKE), _dev(s, f"{name}.scales", _BF16_LIKE),
              _dev(b, f"{name}.biases", _BF16_LIKE)]
    gp = None if shared_gate is None else _dev(shared_gate, "shared_gate", _BF16_LIKE)
    check(load().fmxq_moe_layer(*p, gp, _dev(out, "out", _BF16_LIKE), T, topk, E, D, I,
                                group_size, bits, _stream(x)))
    return out


def moe_combine(y, weights, shared=None, shared_gate=None, out=None):
    """sum_j y[:, j] * weights[:, j] (+ shared, optionally sigmoid-gated); y [T, k, D]."""
    T, topk, D = y.shape
    if out is None:
        out = torch.empty(T, D, dtype=torch.bfloat16, device=y.device)
    sp = None if shared is None else _dev(shared, "shared", _BF16_LIKE)
    gp = None if shared_gate is None else _dev(shared_gate, "shared_gate", _BF16_LIKE)
    check(load().fmxq_moe_combine(_dev(y, "y", _BF16_LIKE), _dev(weights, "weights", _BF16_LIKE),
                                  sp, gp, _dev(out, "out", _BF16_LIKE), T, topk, D, _stream(y)))
    return out


def _route_io(logits, T, k, weights_dtype):
    if logits.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"router logits must be bfloat16 or float32, got {logits.dtype}")
    if weights_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"router weights must be bfloat16 or float32, got {weights_dtype}")
    inds = torch.empty(T, k, dtype=torch.int32, device=logits.device)
    weights = torch.empty(T, k, dtype=weights_dtype, device=logits.device)
    return inds, weights


def route_softmax_topk(logits, top_k, norm_topk_prob=True, weights_dtype=torch.bfloat16):
    """Softmax router (qwen3next_forward.go:513-518): logits [T, E] -> (inds [T, k] int32
    holding uint32 ids, weights [T, k]), largest gate first."""
    T, E = logits.shape
    inds, weights = _route_io(logits, T, top_k, weights_dtype)
    ptr = _dev(logits, "logits", (torch.bfloat16, torch.float32))
    check(load().fmxq_route_softmax_topk(ptr, int(logits.dtype == torch.bfloat16), T, E, top_k,
                                         bool(norm_topk_prob), _dev(inds, "inds", _U32_LIKE),
                                         weights.data_ptr(),
                                         int(weights_dtype == torch.bfloat16), _stream(logits)))
    return inds, weights


def route_group_topk(gates, bias, top_k, n_group, topk_group, routed_scaling_factor=1.0,
                     norm_topk_prob=True, weights_dtype=torch.float32):
    """DeepSeek-V3 group-limited router (deepseekv3_forward.go:452-491): gates [T, E],
    bias [E] float32 or None -> (inds [T, k] int32 holding uint32 ids, weights [T, k])."""
    T, E = gates.shape
    inds, weights = _route_io(gates, T, top_k, weights_dtype)
    bptr = None if bias is None else _dev(bias, "bias", (torch.float32,))
    ptr = _dev(gates, "gates", (torch.bfloat16, torch.float32))
    check(load().fmxq_route_group_topk(ptr, int(gates.dtype == torch.bfloat16), bptr, T, E, top_k,
                                       n_group, topk_group, float(routed_scaling_factor),
                                       bool(norm_topk_prob), _dev(inds, "inds", _U32_LIKE),
                                       weights.data_ptr(), int(weights_dtype == torch.bfloat16),
                                       _stream(gates)))
    return inds, weights


def device_error(device=None) -> None:
    """Raise FmxqError(FMXQ_ERR_INDEX) if a gather met an out-of-range index."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    check(load().fmxq_device_error(torch.cuda.current_stream(dev).cuda_stream))
