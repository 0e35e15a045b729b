"""CPU checks of the C ABI: every declared symbol is exported, and argument
validation rejects bad calls with a status (never a crash) before any GPU work.

Mirrors the reference's error-path tests: unsupported quantization falls back
to an error rather than a wrong answer (compute/models/quant_test.go:30-59), shape
guards fire before any kernel (switch_glu_test.go:202-219), and every op reports a
failure status the binding turns into an error (mlxgo/binding_stub_test.go:125-185).
"""
import ctypes
import os
import re

import pytest

from fastmlx_amd import FmxqError, _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:fmxq|fmx)_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    lib = _lib.load()
    for header in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not header.endswith(".h"):
            continue
        names = _declared(header)
        assert names, header
        for name in names:
            assert hasattr(lib, name), f"{header}: {name} missing from libfmxq.so"
            assert name in _lib.all_symbols(), f"{name} has no ctypes signature"


def test_version():
    assert _lib.load().fmxq_version() >= 100


def _qmm(**kw):
    args = dict(x=None, w=None, s=None, b=None, y=None, M=1, N=16, K=64, transpose=True,
                group=64, bits=4)
    args.update(kw)
    return _lib.load().fmxq_quantized_matmul(args["x"], args["w"], args["s"], args["b"],
                                             args["y"], args["M"], args["N"], args["K"],
                                             args["transpose"], args["group"], args["bits"],
                                             None)


def _status(rc):
    return _lib.STATUS[rc]


@pytest.mark.parametrize("bits", [2, 3, 5, 6, 16])
def test_unsupported_bits_is_an_error(bits):
    # oQ can emit 2/3/5/6-bit (quant/oq.go:21-27): rejected, never computed wrongly
    assert _status(_qmm(bits=bits)) == "FMXQ_ERR_UNSUPPORTED"
    assert b"bits" in _lib.load().fmxq_last_error()


def test_group_transpose_and_shape_errors():
    assert _status(_qmm(group=48)) == "FMXQ_ERR_UNSUPPORTED"
    assert _status(_qmm(transpose=False)) == "FMXQ_ERR_UNSUPPORTED"
    assert _status(_qmm(K=100)) == "FMXQ_ERR_SHAPE"
    assert _status(_qmm(M=-1)) == "FMXQ_ERR_SHAPE"
    assert _status(_qmm()) == "FMXQ_ERR_INVALID_ARGUMENT"  # null operands
    assert _qmm(M=0) == 0 and _qmm(N=0) == 0              # empty: nothing to do


def test_misaligned_pointer_rejected():
    buf = (ctypes.c_uint8 * 256)()
    base = ctypes.addressof(buf)
    p = base + (16 - base % 16) % 16 + 2  # 2 bytes past 16-byte alignment
    rc = _qmm(x=p, w=p, s=p, b=p, y=p)
    assert _status(rc) == "FMXQ_ERR_INVALID_ARGUMENT"


def test_gather_and_dequantize_validation():
    lib = _lib.load()
    g = lambda **k: lib.fmxq_gather_qmm(
        k.get("x"), k.get("w"), k.get("s"), k.get("b"), k.get("lhs"), k.get("rhs"), k.get("y"),
        k.get("batch", 4), k.get("xb", 4), k.get("div", 1), k.get("mx", 1), k.get("N", 8),
        k.get("K", 64), k.get("E", 2), True, k.get("group", 64), k.get("bits", 4), False, None)
    assert _status(g(bits=3)) == "FMXQ_ERR_UNSUPPORTED"
    assert _status(g(E=0)) == "FMXQ_ERR_SHAPE"
    assert _status(g(div=0)) == "FMXQ_ERR_INVALID_ARGUMENT"
    assert _status(g(batch=9, xb=2, div=4)) == "FMXQ_ERR_SHAPE"
    assert _status(g()) == "FMXQ_ERR_INVALID_ARGUMENT"
    assert g(batch=0) == 0
    d = lib.fmxq_dequantize
    assert _status(d(None, None, None, None, 4, 65, 64, 4, None)) == "FMXQ_ERR_SHAPE"
    assert _status(d(None, None, None, None, 4, 64, 64, 7, None)) == "FMXQ_ERR_UNSUPPORTED"
    assert d(None, None, None, None, 0, 64, 64, 4, None) == 0
    q = lib.fmxq_quantize
    assert _status(q(None, None, None, None, 4, 96, 64, 4, None)) == "FMXQ_ERR_SHAPE"
    assert _status(q(None, None, None, None, 4, 64, 64, 2, None)) == "FMXQ_ERR_UNSUPPORTED"
    assert _status(q(None, None, None, None, 4, 64, 48, 4, None)) == "FMXQ_ERR_UNSUPPORTED"
    assert _status(q(None, None, None, None, -1, 64, 64, 4, None)) == "FMXQ_ERR_SHAPE"
    assert _status(q(None, None, None, None, 4, 64, 64, 4, None)) == "FMXQ_ERR_INVALID_ARGUMENT"
    assert q(None, None, None, None, 0, 64, 64, 4, None) == 0


def test_switch_glu_and_combine_validation():
    lib = _lib.load()
    sg = lambda **k: lib.fmxq_switch_glu(*([None] * 12), k.get("T", 2), k.get("topk", 2),
                                         k.get("E", 4), k.get("D", 64), k.get("I", 64),
                                         k.get("group", 64), k.get("bits", 4), None)
    assert _status(sg(bits=2)) == "FMXQ_ERR_UNSUPPORTED"
    assert _status(sg(D=100)) == "FMXQ_ERR_SHAPE"
    assert _status(sg(topk=0)) == "FMXQ_ERR_SHAPE"
    assert _status(sg()) == "FMXQ_ERR_INVALID_ARGUMENT"
    assert sg(T=0) == 0
    ml = lambda ptrs, **k: lib.fmxq_moe_layer(*ptrs, k.get("T", 1), k.get("topk", 2),
                                              k.get("E", 4), k.get("D", 64), k.get("I", 64),
                                              k.get("group", 64), k.get("bits", 4), None)
    fake = ctypes.c_void_p(0x1000)
    full = [fake] * 21 + [None, fake]  # routed + weights + shared triples, no gate, out
    assert _status(ml([None] * 23, bits=2)) == "FMXQ_ERR_UNSUPPORTED"
    assert _status(ml([None] * 23, D=100)) == "FMXQ_ERR_SHAPE"
    assert _status(ml([None] * 23, topk=0)) == "FMXQ_ERR_SHAPE"
    assert ml([None] * 23, T=0) == 0
    for i in range(12, 21):  # each of the shared expert's pointers is required
        ptrs = list(full)
        ptrs[i] = None
        assert _status(ml(ptrs)) == "FMXQ_ERR_INVALID_ARGUMENT", i
    ptrs = list(full)
    ptrs[18] = ctypes.c_void_p(0x1008)  # shared down weights not 16-byte aligned
    assert _status(ml(ptrs)) == "FMXQ_ERR_INVALID_ARGUMENT"
    mc = lib.fmxq_moe_combine
    assert _status(mc(None, None, None, None, None, 2, 2, 7, None)) == "FMXQ_ERR_SHAPE"
    assert _status(mc(None, None, None, None, None, 2, 2, 8, None)) == "FMXQ_ERR_INVALID_ARGUMENT"


def test_router_validation():
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)

    def soft(T=4, E=64, k=4, logits=fake, inds=fake, w=fake, lbf=1, wbf=1):
        return lib.fmxq_route_softmax_topk(logits, lbf, T, E, k, True, inds, w, wbf, None)

    def grp(T=4, E=64, k=4, ng=8, tg=4, bias=None, logits=fake, inds=fake, w=fake):
        return lib.fmxq_route_group_topk(logits, 0, bias, T, E, k, ng, tg, 1.0, True, inds, w, 0,
                                         None)

    assert _status(soft(E=2048)) == "FMXQ_ERR_UNSUPPORTED"   # more experts than a wave holds
    assert _status(soft(k=0)) == "FMXQ_ERR_SHAPE"
    assert _status(soft(E=8, k=9)) == "FMXQ_ERR_SHAPE"
    assert _status(soft(T=-1)) == "FMXQ_ERR_SHAPE"
    assert _status(soft(logits=None)) == "FMXQ_ERR_INVALID_ARGUMENT"
    assert _status(soft(logits=ctypes.c_void_p(0x1001))) == "FMXQ_ERR_INVALID_ARGUMENT"
    assert soft(T=0) == 0
    assert _status(grp(ng=7)) == "FMXQ_ERR_SHAPE"            # groups must divide E
    assert _status(grp(tg=9)) == "FMXQ_ERR_SHAPE"
    assert _status(grp(tg=0)) == "FMXQ_ERR_SHAPE"
    assert _status(grp(bias=ctypes.c_void_p(0x1002))) == "FMXQ_ERR_INVALID_ARGUMENT"
    assert grp(T=0) == 0


def test_check_raises_with_message():
    rc = _qmm(bits=3)
    with pytest.raises(FmxqError) as ei:
        _lib.check(rc)
    assert ei.value.code == 2 and "bits=3" in str(ei.value)
