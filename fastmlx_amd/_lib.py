"""Loader for libfmxq.so, the HIP library behind every op in this package.

There is no CPU fallback: if the library is missing or a call fails, the
caller gets an exception.  ``load()`` resolves every symbol the C headers
declare, so a stale or partial build fails at load time, not mid-run.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfmxq.so")

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_bool = ctypes.c_bool

# name -> (restype, argtypes); the raw kernel ABI of include/fmxq.h
FMXQ_SYMBOLS = {
    "fmxq_version": (_int, []),
    "fmxq_last_error": (ctypes.c_char_p, []),
    "fmxq_dequantize": (_int, [_p, _p, _p, _p, _i64, _i64, _int, _int, _p]),
    "fmxq_dequantize_rows": (_int, [_p] * 5 + [_i64] * 3 + [_int, _int, _p]),
    "fmxq_quantize": (_int, [_p, _p, _p, _p, _i64, _i64, _int, _int, _p]),
    "fmxq_quantized_matmul": (_int, [_p, _p, _p, _p, _p, _i64, _i64, _i64, _bool, _int, _int, _p]),
    "fmxq_quantized_matmul_bias": (_int, [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _bool, _int,
                                          _int, _p]),
    "fmxq_quantized_matmul_group": (_int, [_p, _int, _p, _p, _p, _p, _p, _i64, _i64, _bool, _int,
                                           _int, _p]),
    "fmxq_gather_qmm": (_int, [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64,
                               _i64, _bool, _int, _int, _bool, _p]),
    "fmxq_device_error": (_int, [_p]),
    "fmxq_switch_glu": (_int, [_p] * 12 + [_i64] * 5 + [_int, _int, _p]),
    "fmxq_switch_glu_noalloc": (_int, [_p] * 12 + [_i64] * 5 + [_int, _int, _p]),
    "fmxq_switch_glu_combine": (_int, [_p] * 15 + [_i64] * 5 + [_int, _int, _p]),
    "fmxq_moe_layer": (_int, [_p] * 23 + [_i64] * 5 + [_int, _int, _p]),
    "fmxq_moe_combine": (_int, [_p] * 5 + [_i64] * 3 + [_p]),
    "fmxq_route_softmax_topk": (_int, [_p, _int, _i64, _i64, _int, _bool, _p, _p, _int, _p]),
    "fmxq_route_group_topk": (_int, [_p, _int, _p, _i64, _i64, _int, _int, _int, ctypes.c_float,
                                     _bool, _p, _p, _int, _p]),
}



class FmxArray(ctypes.Structure):
    """fmx_array handle (include/fmx.h); ctx NULL is the empty array."""
    _fields_ = [("ctx", ctypes.c_void_p)]


class FmxStream(ctypes.Structure):
    """fmx_stream handle (include/fmx.h)."""
    _fields_ = [("ctx", ctypes.c_void_p)]


_A = FmxArray
_S = FmxStream
_Ap = ctypes.POINTER(FmxArray)
_sz = ctypes.c_size_t
_u64 = ctypes.c_uint64
_cs = ctypes.c_char_p

# the array-handle layer of include/fmx.h (mlx-c calling convention)
FMX_SYMBOLS = {
    "fmx_array_new": (_A, []),
    "fmx_array_new_data": (_A, [_p, ctypes.POINTER(_int), _int, _int]),
    "fmx_array_new_device": (_A, [_p, ctypes.POINTER(_int), _int, _int]),
    "fmx_array_free": (_int, [_A]),
    "fmx_array_ndim": (_sz, [_A]),
    "fmx_array_dim": (_int, [_A, _int]),
    "fmx_array_dtype": (_int, [_A]),
    "fmx_array_size": (_sz, [_A]),
    "fmx_array_nbytes": (_sz, [_A]),
    "fmx_array_device_ptr": (_p, [_A]),
    "fmx_array_eval": (_int, [_A]),
    "fmx_array_data_float32": (ctypes.POINTER(ctypes.c_float), [_A]),
    "fmx_array_data_int32": (ctypes.POINTER(ctypes.c_int32), [_A]),
    "fmx_array_to_host": (_int, [_p, _sz, _A]),
    "fmx_default_gpu_stream_new": (_S, []),
    "fmx_stream_new": (_S, []),
    "fmx_stream_wrap": (_S, [_p]),
    "fmx_stream_free": (_int, [_S]),
    "fmx_synchronize": (_int, [_S]),
    "fmx_quantized_matmul": (_int, [_Ap, _A, _A, _A, _A, _bool, _int, _int, _S]),
    "fmx_gather_qmm": (_int, [_Ap] + [_A] * 6 + [_bool, _int, _int, _bool, _S]),
    "fmx_dequantize": (_int, [_Ap, _A, _A, _A, _int, _int, _S]),
    "fmx_quantized_matmul_bias": (_int, [_Ap] + [_A] * 5 + [_bool, _int, _int, _S]),
    "fmx_moe_combine": (_int, [_Ap] + [_A] * 4 + [_S]),
    "fmx_dequantize_rows": (_int, [_Ap] + [_A] * 4 + [_int, _int, _S]),
    "fmx_switch_glu": (_int, [_Ap] + [_A] * 11 + [_int, _int, _S]),
    "fmx_route_softmax_topk": (_int, [_Ap, _Ap, _A, _int, _bool, _S]),
    "fmx_route_group_topk": (_int, [_Ap, _Ap, _A, _A, _int, _int, _int, ctypes.c_float, _bool,
                                    _S]),
    # weight ingest
    "fmx_safetensors_parse": (_int, [_p, _u64, ctypes.POINTER(_p)]),
    "fmx_safetensors_free": (None, [_p]),
    "fmx_safetensors_header_size": (_u64, [_p]),
    "fmx_safetensors_data_start": (_u64, [_p]),
    "fmx_safetensors_count": (_i64, [_p]),
    "fmx_safetensors_tensor": (_int, [_p, _i64, ctypes.POINTER(_cs), ctypes.POINTER(_cs),
                                      ctypes.POINTER(_int), ctypes.POINTER(ctypes.POINTER(_i64)),
                                      ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "fmx_safetensors_find": (_i64, [_p, _cs]),
    "fmx_safetensors_metadata_count": (_i64, [_p]),
    "fmx_safetensors_metadata": (_int, [_p, _i64, ctypes.POINTER(_cs), ctypes.POINTER(_cs)]),
    "fmx_safetensors_dtype": (_int, [_cs, ctypes.POINTER(_int)]),
    "fmx_safetensors_slice": (_int, [_u64, _u64, _u64, _u64, ctypes.POINTER(_u64)]),
    "fmx_safetensors_load": (_int, [_Ap, _p, _u64, _p, _i64]),
    "fmx_view": (_int, [_Ap, _A, _int, _S]),
    "fmx_stack": (_int, [_Ap, ctypes.POINTER(_A), _sz, _int, _S]),
    "fmx_scale_neg8": (_int, [_Ap, _A, _S]),
    "fmx_quantize": (_int, [_Ap, _Ap, _Ap, _A, _int, _int, _S]),
    "fmx_reshape": (_int, [_Ap, _A, ctypes.POINTER(_int), _sz, _S]),
    "fmx_split": (_int, [_Ap, _sz, _A, ctypes.POINTER(_int), _sz, _int, _S]),
    "fmx_swapaxes": (_int, [_Ap, _A, _int, _int, _S]),
    "fmx_contiguous": (_int, [_Ap, _A, _bool, _S]),
}

STATUS = {
    0: "FMXQ_OK",
    1: "FMXQ_ERR_INVALID_ARGUMENT",
    2: "FMXQ_ERR_UNSUPPORTED",
    3: "FMXQ_ERR_SHAPE",
    4: "FMXQ_ERR_INDEX",
    5: "FMXQ_ERR_DEVICE",
}

_lib = None


class FmxqError(RuntimeError):
    """A libfmxq call returned a nonzero status."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS.get(code, code)}: {message}")
        self.code = code


def all_symbols() -> dict:
    return {**FMXQ_SYMBOLS, **FMX_SYMBOLS}


def load(path: str | None = None):
    """Load libfmxq.so and bind every declared symbol (raises if any is missing)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise FileNotFoundError(
            f"{p} is missing: build it with `python -m fastmlx_amd.build` (no CPU fallback exists)")
    lib = ctypes.CDLL(p)
    for name, (res, args) in all_symbols().items():
        fn = getattr(lib, name)  # AttributeError if the build lacks the symbol
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load().fmxq_last_error()
        raise FmxqError(rc, msg.decode() if msg else "")
