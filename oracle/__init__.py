"""ctypes front end of the CPU oracle (``liboracle.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py``.  The product library never imports it.

Every function takes and returns numpy arrays; bf16 tensors are ``uint16`` bit
patterns, packed weights are ``uint32``.  The C side documents which reference
file:line each routine restates (``oracle/fmxq_oracle.c``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_HERE, "liboracle.so")
_lib = None

DEQ_MLX = 0
DEQ_FUSED = 1
DEQ_EXACT = 2

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB):
        subprocess.run(["make", "-s", "-B" if force else "-s", "liboracle.so"],
                       cwd=_HERE, check=True)
    return _LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        L = ctypes.CDLL(_LIB)
        L.oracle_dequantize.argtypes = [_p, _p, _p, _p, _i64, _i64, _int, _int, _int]
        L.oracle_quantize.argtypes = [_p, _p, _p, _p, _i64, _i64, _int, _int]
        L.oracle_qmm_f32.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _int, _int, _int]
        L.oracle_qmm_f64.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, _i64, _int, _int, _int]
        L.oracle_gather_qmm.argtypes = [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64,
                                        _i64, _int, _int, _int]
        L.oracle_switch_glu.argtypes = [_p] * 12 + [_i64] * 5 + [_int, _int, _p, _i64, _int, _p]
        L.oracle_qmm_cpu_fast.argtypes = [_p, _p, _p, _p, _p, _i64, _i64, _i64, _int, _int]
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_bf16_to_f32.restype = ctypes.c_float
        L.oracle_num_threads.restype = _int
        L.oracle_route_group_topk.argtypes = [_p, _p, _i64, _i64, _int, _int, _int,
                                              ctypes.c_double, _int, _p, _p]
        L.oracle_route_softmax_topk.argtypes = [_p, _i64, _i64, _int, _int, _p, _p]
        _lib = L
    return _lib


def _ptr(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what} failed with rc={rc}")


def num_threads() -> int:
    return lib().oracle_num_threads()


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (vectorised twin of the C routine)."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def dequantize(w, scales, biases, group_size=64, bits=4, mode=DEQ_MLX):
    rows = w.shape[0] if w.ndim >= 1 else 0
    lead = w.shape[:-1]
    K = w.shape[-1] * 32 // bits
    rows = int(np.prod(lead)) if lead else 1
    out = np.empty(lead + (K,), dtype=np.uint16)
    _check(lib().oracle_dequantize(_ptr(w), _ptr(scales), _ptr(biases), _ptr(out),
                                   rows, K, group_size, bits, mode), "dequantize")
    return out


def quantize(w, group_size=64, bits=4):
    """MLX affine quantization of bf16 w [rows, K]: (wq, scales, biases)."""
    w = np.ascontiguousarray(w, dtype=np.uint16)
    rows, K = w.shape
    wq = np.empty((rows, K * bits // 32), dtype=np.uint32)
    scales = np.empty((rows, K // group_size), dtype=np.uint16)
    biases = np.empty_like(scales)
    _check(lib().oracle_quantize(_ptr(w), _ptr(wq), _ptr(scales), _ptr(biases), rows, K,
                                 group_size, bits), "quantize")
    return wq, scales, biases


def qmm(x, w, scales, biases, group_size=64, bits=4, mode=DEQ_MLX, want_f32=False):
    """y = x . deq(W)^T with fp32 accumulation; x [M, K] bf16 bits."""
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), dtype=np.uint16)
    yf = np.empty((M, N), dtype=np.float32) if want_f32 else None
    _check(lib().oracle_qmm_f32(_ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(y),
                                _ptr(yf), M, N, K, group_size, bits, mode), "qmm_f32")
    return (y, yf) if want_f32 else y


def qmm_f64(x, w, scales, biases, group_size=64, bits=4, mode=DEQ_MLX):
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), dtype=np.float64)
    _check(lib().oracle_qmm_f64(_ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(y),
                                M, N, K, group_size, bits, mode), "qmm_f64")
    return y


def gather_qmm(x, w, scales, biases, xrow, expert, group_size=64, bits=4, mode=DEQ_MLX):
    """Flattened gather: y[i] = x[xrow[i]] . deq(W[expert[i]])^T; W [E, N, Kw]."""
    E, N = w.shape[0], w.shape[1]
    K = x.shape[-1]
    xrow = np.ascontiguousarray(xrow, dtype=np.int32)
    expert = np.ascontiguousarray(expert, dtype=np.int32)
    S = xrow.shape[0]
    y = np.empty((S, N), dtype=np.uint16)
    _check(lib().oracle_gather_qmm(_ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(xrow),
                                   _ptr(expert), _ptr(y), S, E, N, K, group_size, bits, mode),
           "gather_qmm")
    return y


def switch_glu(x, inds, gate, up, down, group_size=64, bits=4, token_sel=None, mode=DEQ_MLX,
               want_hscale=False):
    """SwitchGLU over stacked quantized experts; gate/up/down are (w, s, b) triples.

    x [T, D] bf16 bits, inds [T, k] int32 -> out [T or n_sel, k, D] bf16 bits, and
    with want_hscale also sqrt(sum_i (h_i wd_i)^2) per output (float64)."""
    T, D = x.shape
    topk = inds.shape[1]
    E, I = gate[0].shape[0], gate[0].shape[1]
    inds = np.ascontiguousarray(inds, dtype=np.int32)
    sel = None if token_sel is None else np.ascontiguousarray(token_sel, dtype=np.int32)
    nt = T if sel is None else sel.shape[0]
    out = np.empty((nt, topk, D), dtype=np.uint16)
    hs = np.empty((nt, topk, D), dtype=np.float64) if want_hscale else None
    _check(lib().oracle_switch_glu(_ptr(x), _ptr(inds), _ptr(gate[0]), _ptr(gate[1]),
                                   _ptr(gate[2]), _ptr(up[0]), _ptr(up[1]), _ptr(up[2]),
                                   _ptr(down[0]), _ptr(down[1]), _ptr(down[2]), _ptr(out),
                                   T, topk, E, D, I, group_size, bits, _ptr(sel),
                                   0 if sel is None else nt, mode, _ptr(hs)), "switch_glu")
    return (out, hs) if want_hscale else out


def qmm_cpu_fast(x, w, scales, biases, group_size=64, bits=4):
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), dtype=np.uint16)
    _check(lib().oracle_qmm_cpu_fast(_ptr(x), _ptr(w), _ptr(scales), _ptr(biases), _ptr(y),
                                     M, N, K, group_size, bits), "qmm_cpu_fast")
    return y


def route_group_topk(gates, bias, top_k, n_group, topk_group, scale=1.0, norm=True):
    """GroupExpertSelect (compute/models/deepseekv3.go:305-384) per row of gates [T, E]:
    returns (inds [T, k] int32, scores [T, k] float64) in selection order."""
    g = np.ascontiguousarray(np.atleast_2d(gates), dtype=np.float32)
    T, E = g.shape
    k = min(top_k, E)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    inds = np.zeros((T, k), np.int32)
    sc = np.zeros((T, k), np.float64)
    _check(lib().oracle_route_group_topk(_ptr(g), None if b is None else _ptr(b), T, E, k,
                                         n_group, topk_group, float(scale), int(bool(norm)),
                                         _ptr(inds), _ptr(sc)), "route_group_topk")
    return inds, sc


def route_softmax_topk(logits, top_k, norm=True):
    """qwen3NextMoE's router (compute/models/qwen3next_forward.go:513-518) per row of
    logits [T, E]: returns (inds [T, k] int32, weights [T, k] float64)."""
    x = np.ascontiguousarray(np.atleast_2d(logits), dtype=np.float32)
    T, E = x.shape
    inds = np.zeros((T, top_k), np.int32)
    w = np.zeros((T, top_k), np.float64)
    _check(lib().oracle_route_softmax_topk(_ptr(x), T, E, top_k, int(bool(norm)), _ptr(inds),
                                           _ptr(w)), "route_softmax_topk")
    return inds, w
