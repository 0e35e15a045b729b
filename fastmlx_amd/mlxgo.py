"""The reference's ``mlxgo`` surface for the quantized-linear path, over fmx.h.

Mirrors the Go API the reference's models call (mlxgo/binding_cgo.go and its
stub twin mlxgo/binding_stub.go) with Python naming:

    NewBytes / NewFloat32 / NewInt32   -> Array.new_bytes / new_float32 / new_int32
    Shape, Dtype, Ndim, Size, Eval     -> Array.shape() ... Array.eval()
    ToFloat32 / ToInt32, Free          -> Array.to_float32() / to_int32(), Array.free()
    DefaultStream, NewStream, Synchronize -> default_stream(), new_stream(), Stream.synchronize()
    QuantizedMatMul, GatherQMM, Dequantize -> quantized_matmul, gather_qmm, dequantize

plus the fused neighbours of include/fmx.h (quantized_matmul_bias,
dequantize_rows, switch_glu, moe_combine).  Go returns ``(nil, err)`` with the
single sentinel ``ErrMLXUnavailable`` (mlxgo/dtype.go:29); here every failing
call raises :class:`MLXError` carrying the library's status and message, and
``ErrMLXUnavailable`` names that class so ``isinstance(e, ErrMLXUnavailable)``
reads like ``errors.Is``.  Every op runs on the GPU through libfmxq.so; there is
no host fallback.
"""
from __future__ import annotations

import ctypes
import enum
from typing import Optional, Sequence

import numpy as np

from ._lib import FmxArray, FmxqError, FmxStream, load


class Dtype(enum.IntEnum):
    """Element types in the reference's order (mlxgo/dtype.go:35-50)."""

    BOOL = 0
    UINT8 = 1
    UINT16 = 2
    UINT32 = 3
    UINT64 = 4
    INT8 = 5
    INT16 = 6
    INT32 = 7
    INT64 = 8
    FLOAT16 = 9
    FLOAT32 = 10
    BFLOAT16 = 11
    COMPLEX64 = 12
    FLOAT64 = 13

    def size(self) -> int:
        """Bytes per element (mlxgo/dtype.go Size)."""
        return _DTYPE_SIZE[self]


_DTYPE_SIZE = {Dtype.BOOL: 1, Dtype.UINT8: 1, Dtype.UINT16: 2, Dtype.UINT32: 4, Dtype.UINT64: 8,
               Dtype.INT8: 1, Dtype.INT16: 2, Dtype.INT32: 4, Dtype.INT64: 8, Dtype.FLOAT16: 2,
               Dtype.FLOAT32: 4, Dtype.BFLOAT16: 2, Dtype.COMPLEX64: 8, Dtype.FLOAT64: 8}

# numpy storage type of each dtype (bf16 travels as its uint16 bit pattern)
_NP = {Dtype.BOOL: np.bool_, Dtype.UINT8: np.uint8, Dtype.UINT16: np.uint16,
       Dtype.UINT32: np.uint32, Dtype.UINT64: np.uint64, Dtype.INT8: np.int8,
       Dtype.INT16: np.int16, Dtype.INT32: np.int32, Dtype.INT64: np.int64,
       Dtype.FLOAT16: np.float16, Dtype.FLOAT32: np.float32, Dtype.BFLOAT16: np.uint16,
       Dtype.COMPLEX64: np.complex64, Dtype.FLOAT64: np.float64}
_FROM_NP = {np.dtype(np.bool_): Dtype.BOOL, np.dtype(np.uint8): Dtype.UINT8,
            np.dtype(np.uint16): Dtype.UINT16, np.dtype(np.uint32): Dtype.UINT32,
            np.dtype(np.uint64): Dtype.UINT64, np.dtype(np.int8): Dtype.INT8,
            np.dtype(np.int16): Dtype.INT16, np.dtype(np.int32): Dtype.INT32,
            np.dtype(np.int64): Dtype.INT64, np.dtype(np.float16): Dtype.FLOAT16,
            np.dtype(np.float32): Dtype.FLOAT32, np.dtype(np.float64): Dtype.FLOAT64,
            np.dtype(np.complex64): Dtype.COMPLEX64}


class MLXError(FmxqError):
    """A failing fmx_* call (nonzero status; message from fmxq_last_error)."""


ErrMLXUnavailable = MLXError


def _check(rc: int) -> None:
    if rc != 0:
        msg = load().fmxq_last_error()
        raise MLXError(rc, msg.decode() if msg else "")


def _shape_arg(shape: Sequence[int]):
    n = len(shape)
    buf = (ctypes.c_int * max(n, 1))(*[int(d) for d in shape])
    return buf, n


def _count(shape: Sequence[int]) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


class Stream:
    """An fmx_stream handle (mlxgo Stream)."""

    __slots__ = ("_h", "_keep")

    def __init__(self, handle: FmxStream, keep=None):
        if not handle.ctx:
            _check(5)  # FMXQ_ERR_DEVICE: the stream could not be created
        self._h = handle
        self._keep = keep

    @property
    def handle(self) -> FmxStream:
        return self._h

    def synchronize(self) -> None:
        """Block until the stream's queued work completes (Stream.Synchronize)."""
        _check(load().fmx_synchronize(self._h))

    def __del__(self):
        try:
            if self._h.ctx:
                load().fmx_stream_free(self._h)
                self._h = FmxStream(None)
        except Exception:
            pass


def default_stream() -> Stream:
    """The default GPU stream of the current device (DefaultStream)."""
    return Stream(load().fmx_default_gpu_stream_new())


def new_stream() -> Stream:
    """A new stream on the current device (NewStream)."""
    return Stream(load().fmx_stream_new())


def wrap_stream(hip_stream: int, keep=None) -> Stream:
    """A handle over an existing hipStream_t (e.g. torch's ``cuda_stream``)."""
    return Stream(load().fmx_stream_wrap(hip_stream), keep)


def _sh(s: Optional[Stream]) -> FmxStream:
    return s.handle if s is not None else FmxStream(None)


class Array:
    """An fmx_array handle (mlxgo Array).  ``free()`` is idempotent and also runs
    when the object is collected, as the Go finalizer does."""

    __slots__ = ("_h", "_keep", "__weakref__")

    def __init__(self, handle: FmxArray, keep=None):
        self._h = handle
        self._keep = keep

    # -- construction --
    @classmethod
    def empty(cls) -> "Array":
        return cls(load().fmx_array_new())

    @classmethod
    def new_bytes(cls, data: bytes, dtype: Dtype, *shape: int) -> "Array":
        """Raw little-endian element bytes of any dtype (NewBytes)."""
        dtype = Dtype(dtype)
        if len(data) != _count(shape) * dtype.size():
            raise ValueError(f"NewBytes: {len(data)} bytes do not fill shape {list(shape)} "
                             f"of {dtype.name}")
        buf, n = _shape_arg(shape)
        raw = ctypes.create_string_buffer(bytes(data), max(len(data), 1))
        h = load().fmx_array_new_data(raw, buf, n, int(dtype))
        if not h.ctx:
            _check(1)
        return cls(h)

    @classmethod
    def new_float32(cls, data, *shape: int) -> "Array":
        a = np.ascontiguousarray(np.asarray(data, dtype=np.float32))
        if a.size != _count(shape):
            raise ValueError(f"NewFloat32: {a.size} values do not fill shape {list(shape)}")
        return cls.new_bytes(a.tobytes(), Dtype.FLOAT32, *shape)

    @classmethod
    def new_int32(cls, data, *shape: int) -> "Array":
        a = np.ascontiguousarray(np.asarray(data, dtype=np.int32))
        if a.size != _count(shape):
            raise ValueError(f"NewInt32: {a.size} values do not fill shape {list(shape)}")
        return cls.new_bytes(a.tobytes(), Dtype.INT32, *shape)

    @classmethod
    def from_numpy(cls, a: np.ndarray, dtype: Optional[Dtype] = None) -> "Array":
        """Copy a host array to the device; bf16 data is passed as uint16 bits with
        ``dtype=Dtype.BFLOAT16``."""
        a = np.ascontiguousarray(a)
        if dtype is None:
            if a.dtype not in _FROM_NP:
                raise TypeError(f"no fmx dtype for numpy {a.dtype}")
            dtype = _FROM_NP[a.dtype]
        dtype = Dtype(dtype)
        if a.dtype.itemsize != dtype.size():
            raise TypeError(f"numpy {a.dtype} cannot carry {dtype.name}")
        return cls.new_bytes(a.tobytes(), dtype, *a.shape)

    @classmethod
    def from_device(cls, ptr: int, shape: Sequence[int], dtype: Dtype, keep=None) -> "Array":
        """Borrow an existing device buffer (not freed with the handle); ``keep``
        holds its owner (e.g. a torch tensor) alive as long as the handle."""
        buf, n = _shape_arg(shape)
        h = load().fmx_array_new_device(ptr, buf, n, int(Dtype(dtype)))
        if not h.ctx:
            _check(1)
        return cls(h, keep)

    @classmethod
    def from_torch(cls, t) -> "Array":
        import torch

        m = {torch.bfloat16: Dtype.BFLOAT16, torch.float16: Dtype.FLOAT16,
             torch.float32: Dtype.FLOAT32, torch.int32: Dtype.INT32, torch.int64: Dtype.INT64,
             torch.uint8: Dtype.UINT8, torch.int16: Dtype.INT16, torch.int8: Dtype.INT8,
             torch.bool: Dtype.BOOL}
        if hasattr(torch, "uint32"):
            m[torch.uint32] = Dtype.UINT32
        if t.dtype not in m:
            raise TypeError(f"no fmx dtype for {t.dtype}")
        if not t.is_contiguous():
            raise ValueError("tensor must be contiguous")
        return cls.from_device(t.data_ptr(), list(t.shape), m[t.dtype], keep=t)

    # -- queries --
    @property
    def handle(self) -> FmxArray:
        return self._h

    def is_empty(self) -> bool:
        return not self._h.ctx

    def shape(self) -> list:
        lib = load()
        return [lib.fmx_array_dim(self._h, i) for i in range(lib.fmx_array_ndim(self._h))]

    def dtype(self) -> Dtype:
        return Dtype(load().fmx_array_dtype(self._h))

    def ndim(self) -> int:
        return int(load().fmx_array_ndim(self._h))

    def size(self) -> int:
        return int(load().fmx_array_size(self._h))

    def nbytes(self) -> int:
        return int(load().fmx_array_nbytes(self._h))

    def device_ptr(self) -> int:
        return load().fmx_array_device_ptr(self._h) or 0

    # -- materialization --
    def eval(self) -> None:
        _check(load().fmx_array_eval(self._h))

    def to_float32(self) -> np.ndarray:
        """Evaluate and copy out as float32 (ToFloat32); bf16/fp16 are widened."""
        self.eval()
        p = load().fmx_array_data_float32(self._h)
        if not p:
            _check(1)
        n = self.size()
        return np.ctypeslib.as_array(p, shape=(n,)).copy().reshape(self.shape())

    def to_int32(self) -> np.ndarray:
        self.eval()
        p = load().fmx_array_data_int32(self._h)
        if not p:
            _check(1)
        n = self.size()
        return np.ctypeslib.as_array(p, shape=(n,)).copy().reshape(self.shape())

    def to_numpy(self) -> np.ndarray:
        """The raw elements in their storage type (bf16 as uint16 bits)."""
        out = np.empty(self.shape(), dtype=_NP[self.dtype()])
        _check(load().fmx_array_to_host(out.ctypes.data if out.size else None, out.nbytes,
                                        self._h))
        return out

    def free(self) -> None:
        if self._h.ctx:
            load().fmx_array_free(self._h)
            self._h = FmxArray(None)
        self._keep = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def __repr__(self) -> str:
        if self.is_empty():
            return "Array(empty)"
        return f"Array(shape={self.shape()}, dtype={self.dtype().name})"


def _ah(a: Optional[Array]) -> FmxArray:
    return a.handle if a is not None else FmxArray(None)


def _op(fn, *args) -> Array:
    out = FmxArray(None)
    _check(fn(ctypes.byref(out), *args))
    return Array(out)


def quantized_matmul(x: Array, w: Array, scales: Array, biases: Array, transpose: bool,
                     group_size: int, bits: int, s: Optional[Stream] = None) -> Array:
    """QuantizedMatMul (mlxgo/binding_cgo.go:636-643): x [..., K] . deq(w)^T."""
    return _op(load().fmx_quantized_matmul, _ah(x), _ah(w), _ah(scales), _ah(biases),
               bool(transpose), int(group_size), int(bits), _sh(s))


def quantized_matmul_bias(x: Array, w: Array, scales: Array, biases: Array,
                          bias: Optional[Array], transpose: bool, group_size: int, bits: int,
                          s: Optional[Stream] = None) -> Array:
    """qlinearBias fused: quantized_matmul + bias [N] in the epilogue."""
    return _op(load().fmx_quantized_matmul_bias, _ah(x), _ah(w), _ah(scales), _ah(biases),
               _ah(bias), bool(transpose), int(group_size), int(bits), _sh(s))


def gather_qmm(x: Array, w: Array, scales: Array, biases: Optional[Array],
               lhs_indices: Optional[Array], rhs_indices: Optional[Array], transpose: bool,
               group_size: int, bits: int, sorted_indices: bool,
               s: Optional[Stream] = None) -> Array:
    """GatherQMM (mlxgo/binding_cgo.go:645-673); nil operands become empty arrays."""
    return _op(load().fmx_gather_qmm, _ah(x), _ah(w), _ah(scales), _ah(biases),
               _ah(lhs_indices), _ah(rhs_indices), bool(transpose), int(group_size), int(bits),
               bool(sorted_indices), _sh(s))


def dequantize(w: Array, scales: Array, biases: Array, group_size: int, bits: int,
               s: Optional[Stream] = None) -> Array:
    """Dequantize (mlxgo/binding_cgo.go:675-682), bit-exact."""
    return _op(load().fmx_dequantize, _ah(w), _ah(scales), _ah(biases), int(group_size),
               int(bits), _sh(s))


def dequantize_rows(w: Array, scales: Array, biases: Array, idx: Array, group_size: int,
                    bits: int, s: Optional[Stream] = None) -> Array:
    """take(w|scales|biases, idx, 0) then Dequantize, as one kernel (qembed)."""
    return _op(load().fmx_dequantize_rows, _ah(w), _ah(scales), _ah(biases), _ah(idx),
               int(group_size), int(bits), _sh(s))


def switch_glu(x: Array, inds: Array, gate, up, down, group_size: int, bits: int,
               s: Optional[Stream] = None) -> Array:
    """switchGLUCore over quantized experts; gate/up/down are (w, scales, biases)."""
    args = [_ah(x), _ah(inds)]
    for trip in (gate, up, down):
        args += [_ah(t) for t in trip]
    return _op(load().fmx_switch_glu, *args, int(group_size), int(bits), _sh(s))


def _op2(fn, *args):
    a, b = FmxArray(None), FmxArray(None)
    _check(fn(ctypes.byref(a), ctypes.byref(b), *args))
    return Array(a), Array(b)


def route_softmax_topk(logits: Array, top_k: int, norm_topk_prob: bool,
                       s: Optional[Stream] = None):
    """qwen3NextMoE's router (qwen3next_forward.go:513-518): (inds, scores)."""
    return _op2(load().fmx_route_softmax_topk, _ah(logits), int(top_k), bool(norm_topk_prob),
                _sh(s))


def route_group_topk(gates: Array, bias: Optional[Array], top_k: int, n_group: int,
                     topk_group: int, routed_scaling_factor: float, norm_topk_prob: bool,
                     s: Optional[Stream] = None):
    """DeepSeek-V3 routeExperts (deepseekv3_forward.go:452-491): (inds, weights)."""
    return _op2(load().fmx_route_group_topk, _ah(gates), _ah(bias), int(top_k), int(n_group),
                int(topk_group), float(routed_scaling_factor), bool(norm_topk_prob), _sh(s))


def moe_combine(y: Array, weights: Array, shared: Optional[Array] = None,
                shared_gate: Optional[Array] = None, s: Optional[Stream] = None) -> Array:
    """sum over top-k of y * weights (+ shared, sigmoid-gated when shared_gate)."""
    return _op(load().fmx_moe_combine, _ah(y), _ah(weights), _ah(shared), _ah(shared_gate),
               _sh(s))


def view(a: Array, dtype: Dtype, s: Optional[Stream] = None) -> Array:
    """View (as remapInt4 calls it, compute/models/deepseekv3.go:513): a's bytes as
    dtype, the last axis scaled by the element-size ratio (a copy here)."""
    return _op(load().fmx_view, _ah(a), int(Dtype(dtype)), _sh(s))


def stack(parts: Sequence[Array], axis: int = 0, s: Optional[Stream] = None) -> Array:
    """Stack along a new leading axis (stackExperts, deepseekv3.go:564-592)."""
    hs = (FmxArray * max(len(parts), 1))(*[_ah(p) for p in parts])
    return _op(load().fmx_stack, hs, len(parts), int(axis), _sh(s))


def quantize(w: Array, group_size: int, bits: int, s: Optional[Stream] = None):
    """Quantize (mlxgo/binding_cgo.go:684-697): (packed, scales, biases)."""
    a, b, c = FmxArray(None), FmxArray(None), FmxArray(None)
    _check(load().fmx_quantize(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c), _ah(w),
                               int(group_size), int(bits), _sh(s)))
    return Array(a), Array(b), Array(c)


def reshape(a: Array, shape: Sequence[int], s: Optional[Stream] = None) -> Array:
    """Reshape (mlxgo/binding_cgo.go:398-406); one entry may be -1."""
    dims = (ctypes.c_int * max(len(shape), 1))(*[int(v) for v in shape])
    return _op(load().fmx_reshape, _ah(a), dims, len(shape), _sh(s))


def split_sections(a: Array, indices: Sequence[int], axis: int,
                   s: Optional[Stream] = None) -> list:
    """SplitSections (mlxgo/binding_cgo.go:463-483): len(indices) + 1 parts."""
    n = len(indices) + 1
    outs = (FmxArray * n)()
    idx = (ctypes.c_int * max(len(indices), 1))(*[int(v) for v in indices])
    _check(load().fmx_split(outs, n, _ah(a), idx, len(indices), int(axis), _sh(s)))
    return [Array(FmxArray(outs[i].ctx)) for i in range(n)]


def swapaxes(a: Array, axis1: int, axis2: int, s: Optional[Stream] = None) -> Array:
    """Swapaxes (mlxgo/binding_cgo.go:715-722)."""
    return _op(load().fmx_swapaxes, _ah(a), int(axis1), int(axis2), _sh(s))


def contiguous(a: Array, s: Optional[Stream] = None) -> Array:
    """Contiguous (mlxgo/binding_cgo.go:724-731)."""
    return _op(load().fmx_contiguous, _ah(a), False, _sh(s))


def scale_neg8(scale: Array, s: Optional[Stream] = None) -> Array:
    """-8 * scale in the scale's dtype: Mul by the float32 scalar then Astype back
    (scaleNeg8, deepseekv3.go:539-551)."""
    return _op(load().fmx_scale_neg8, _ah(scale), _sh(s))
