"""CPU checks of the array-handle layer (include/fmx.h): dtype order, handle
queries, and that every op validates shapes/dtypes and rejects bad calls with a
status and message before it touches the device.  Arrays here borrow fake
device addresses (fmx_array_new_device), which is safe only because nothing
reaches a kernel: those cases never get past validation.
"""
import os
import re

import numpy as np
import pytest

from fastmlx_amd import mlxgo
from fastmlx_amd._lib import load
from fastmlx_amd.mlxgo import Array, Dtype, MLXError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FAKE = 0x7F0000001000  # a 4 KiB-aligned address no test dereferences


def _gpu_visible():
    try:
        import torch

        return torch.cuda.device_count() > 0
    except Exception:
        return False


# A case that wrongly passed validation would launch on FAKE; without a GPU it
# fails at the device query instead, so these run only where no GPU is visible.
pytestmark = pytest.mark.skipif(_gpu_visible(), reason="fake device addresses: CPU-only checks")

BF, U32, I32 = Dtype.BFLOAT16, Dtype.UINT32, Dtype.INT32


def fake(*shape, dtype=BF):
    return Array.from_device(FAKE, list(shape), dtype)


def status(e):
    return e.value.code


def test_dtype_order_matches_header_and_reference():
    text = open(os.path.join(ROOT, "include", "fmx.h")).read()
    body = re.search(r"typedef enum \{(.*?)\} fmx_dtype;", text, re.S).group(1)
    names = re.findall(r"FMX_([A-Z0-9]+)", body)
    # mlxgo/dtype.go:35-50 order
    want = ["BOOL", "UINT8", "UINT16", "UINT32", "UINT64", "INT8", "INT16", "INT32", "INT64",
            "FLOAT16", "FLOAT32", "BFLOAT16", "COMPLEX64", "FLOAT64"]
    assert names == want
    assert [d.name for d in Dtype] == want
    assert [d.size() for d in (Dtype.BFLOAT16, Dtype.UINT32, Dtype.INT64, Dtype.COMPLEX64)] == \
        [2, 4, 8, 8]


def test_handle_queries_without_device():
    a = fake(3, 5, 7, dtype=U32)
    assert a.shape() == [3, 5, 7] and a.ndim() == 3 and a.size() == 105
    assert a.dtype() == U32 and a.nbytes() == 420 and a.device_ptr() == FAKE
    s = fake(dtype=BF)  # rank 0: one element
    assert s.shape() == [] and s.size() == 1
    e = Array.empty()
    assert e.is_empty() and e.size() == 0 and e.ndim() == 0
    a.free()
    a.free()  # idempotent, like mlxgo Array.Free
    assert a.is_empty()


def test_bad_handle_construction():
    lib = load()
    import ctypes

    dims = (ctypes.c_int * 2)(2, -1)
    assert not lib.fmx_array_new_device(FAKE, dims, 2, int(BF)).ctx
    assert b"negative" in lib.fmxq_last_error()
    dims = (ctypes.c_int * 1)(4)
    assert not lib.fmx_array_new_device(FAKE, dims, 1, 99).ctx
    assert not lib.fmx_array_new_device(None, dims, 1, int(BF)).ctx
    with pytest.raises(ValueError):
        Array.new_bytes(b"\0" * 6, Dtype.FLOAT32, 2)


S = mlxgo.wrap_stream(0)  # wraps the null stream: no device call to create it


def qmm(x, w, sc, bi, transpose=True, gs=64, bits=4):
    return mlxgo.quantized_matmul(x, w, sc, bi, transpose, gs, bits, S)


def test_quantized_matmul_validation():
    x, w, sc = fake(2, 3, 128), fake(16, 16, dtype=U32), fake(16, 2)
    with pytest.raises(MLXError) as e:
        qmm(fake(2, 128, dtype=Dtype.FLOAT32), w, sc, sc)
    assert status(e) == 2 and "x has dtype float32" in str(e.value)
    with pytest.raises(MLXError) as e:
        qmm(x, fake(16, 16, dtype=I32), sc, sc)
    assert status(e) == 2
    with pytest.raises(MLXError) as e:
        qmm(x, fake(2, 16, 16, dtype=U32), sc, sc)
    assert status(e) == 2 and "w must be [N, K*bits/32]" in str(e.value)
    with pytest.raises(MLXError) as e:
        qmm(fake(2, 64), w, sc, sc)
    assert status(e) == 3 and "K=64" in str(e.value)
    with pytest.raises(MLXError) as e:
        qmm(x, w, fake(16, 4), sc)
    assert status(e) == 3 and "scales has shape [16 4]" in str(e.value)
    with pytest.raises(MLXError) as e:
        qmm(x, w, sc, sc, bits=3)
    assert status(e) == 2
    with pytest.raises(MLXError) as e:
        qmm(x, w, sc, sc, transpose=False)
    assert status(e) == 2
    with pytest.raises(MLXError) as e:
        qmm(x, w, sc, Array.empty())
    assert status(e) == 1 and "biases is an empty array" in str(e.value)
    with pytest.raises(MLXError) as e:
        mlxgo.quantized_matmul_bias(x, w, sc, sc, fake(8), True, 64, 4, S)
    assert status(e) == 3 and "bias" in str(e.value)


def gq(x, w, sc, bi, lhs=None, rhs=None, gs=64, bits=4, srt=False):
    return mlxgo.gather_qmm(x, w, sc, bi, lhs, rhs, True, gs, bits, srt, S)


def test_gather_qmm_validation():
    w, sc = fake(4, 16, 8, dtype=U32), fake(4, 16, 1)
    x = fake(2, 3, 1, 1, 64)
    with pytest.raises(MLXError) as e:  # [2,3] vs [2,5]: do not broadcast
        gq(x, w, sc, sc, rhs=fake(2, 5, dtype=I32))
    assert status(e) == 3 and "do not broadcast" in str(e.value)
    with pytest.raises(MLXError) as e:
        gq(x, w, sc, sc, rhs=fake(2, 3, dtype=Dtype.FLOAT32))
    assert status(e) == 1 and "integral" in str(e.value)
    with pytest.raises(MLXError) as e:
        gq(fake(64), w, sc, sc)
    assert status(e) == 3
    with pytest.raises(MLXError) as e:
        gq(x, w, fake(4, 16, 2), sc)
    assert status(e) == 3 and "scales" in str(e.value)
    with pytest.raises(MLXError) as e:  # nil biases: the affine path needs them
        gq(x, w, sc, None, rhs=fake(2, 3, dtype=I32))
    assert status(e) == 1


def test_dequantize_and_rows_validation():
    w, sc = fake(4, 16, dtype=U32), fake(4, 2)
    with pytest.raises(MLXError) as e:
        mlxgo.dequantize(w, fake(4, 1), sc, 64, 4, S)
    assert status(e) == 3
    with pytest.raises(MLXError) as e:
        mlxgo.dequantize(w, sc, sc, 48, 4, S)
    assert status(e) == 2
    with pytest.raises(MLXError) as e:
        mlxgo.dequantize_rows(w, sc, sc, fake(3, dtype=BF), 64, 4, S)
    assert status(e) == 1 and "idx must be integral" in str(e.value)
    with pytest.raises(MLXError) as e:
        mlxgo.dequantize_rows(fake(2, 4, 16, dtype=U32), sc, sc, fake(3, dtype=I32), 64, 4, S)
    assert status(e) == 3


def _experts(E=5, D=64, I=128, bits=4, gs=64):
    pf = 32 // bits
    gu = (fake(E, I, D // pf, dtype=U32), fake(E, I, D // gs), fake(E, I, D // gs))
    dn = (fake(E, D, I // pf, dtype=U32), fake(E, D, I // gs), fake(E, D, I // gs))
    return gu, gu, dn


def test_switch_glu_validation():
    gate, up, down = _experts()
    with pytest.raises(MLXError) as e:  # the reference's rank guard, same message
        mlxgo.switch_glu(fake(2, 64), fake(1, 2, 3, dtype=I32), gate, up, down, 64, 4, S)
    assert status(e) == 3
    assert "switchGLU: want x [B,L,D] and inds [B,L,top_k], got x [2 64] inds [1 2 3]" in \
        str(e.value)
    with pytest.raises(MLXError) as e:
        mlxgo.switch_glu(fake(1, 2, 64), fake(1, 2, 3, dtype=I32), gate, up, gate, 64, 4, S)
    assert status(e) == 3 and "w_down" in str(e.value)
    with pytest.raises(MLXError) as e:
        mlxgo.switch_glu(fake(1, 2, 64), fake(1, 3, 3, dtype=I32), gate, up, down, 64, 4, S)
    assert status(e) == 3


def test_moe_combine_validation():
    y = fake(2, 3, 4, 8)
    with pytest.raises(MLXError) as e:
        mlxgo.moe_combine(y, fake(2, 3, 5), s=S)
    assert status(e) == 3
    with pytest.raises(MLXError) as e:
        mlxgo.moe_combine(y, fake(2, 3, 4), None, fake(2, 3), s=S)
    assert status(e) == 1 and "shared_gate without shared" in str(e.value)
    with pytest.raises(MLXError) as e:
        mlxgo.moe_combine(y, fake(2, 3, 4), fake(2, 3, 9), s=S)
    assert status(e) == 3


def test_from_numpy_dtype_rules():
    with pytest.raises(TypeError):
        Array.from_numpy(np.zeros(3, np.float32), Dtype.BFLOAT16)
    with pytest.raises(TypeError):
        Array.from_numpy(np.zeros(3, dtype=np.dtype("U1")))
