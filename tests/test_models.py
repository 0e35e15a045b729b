"""CPU tests of the model-side mirror (fastmlx_amd/models.py), case for case after
the reference's compute/models/quant_test.go:30-180 and
compute/models/switch_glu_test.go:46-231.

The reference's "reaches the seam" tests run on a build without a backend and
expect ErrMLXUnavailable from the first kernel.  Here the library is present but
no GPU is: a valid call passes validation and fails at the device query with
FMXQ_ERR_DEVICE, the same observable contract (an MLXError, no panic, no
result).  Operands borrow fake device addresses, so these run only where no GPU
is visible; the same paths run for real in tests/test_gpu_handles.py.
"""
import pytest

from fastmlx_amd import models
from fastmlx_amd.mlxgo import Array, Dtype, ErrMLXUnavailable, MLXError
from fastmlx_amd.models import FB, QLinear, QuantConfig, SwitchQuant

FAKE = 0x7F0000002000


def _gpu_visible():
    try:
        import torch

        return torch.cuda.device_count() > 0
    except Exception:
        return False


seam = pytest.mark.skipif(_gpu_visible(), reason="fake device addresses: CPU-only checks")


def arr(*shape, dtype=Dtype.BFLOAT16):
    return Array.from_device(FAKE, list(shape), dtype)


# ---- quant_test.go:30-59 ----
@pytest.mark.parametrize("cfg,want", [
    ('{"hidden_size":8}', QuantConfig()),
    ('{"quantization":{"group_size":64,"bits":4,"mode":"affine"}}', QuantConfig(64, 4)),
    ('{"quantization":{"group_size":32,"bits":8}}', QuantConfig(32, 8)),
    ('{"quantization":{"group_size":32,"bits":4,"mode":"mxfp4"}}', QuantConfig()),
    ('{"quantization":{"group_size":64,"bits":0}}', QuantConfig()),
], ids=["absent", "affine", "no_mode", "mxfp4", "zero_bits"])
def test_parse_quant_config(cfg, want):
    assert models.parse_quant_config(cfg.encode()) == want
    assert want.quantized() == (want.bits > 0)


def test_parse_quant_config_bad_json():
    with pytest.raises(ValueError):
        models.parse_quant_config(b"{")


# ---- quant_test.go:61-128 ----
def test_load_qlinear_dense():
    a = arr(1)
    w = models.load_qlinear({"layer.proj.weight": a}, "layer.proj", QuantConfig())
    assert not w.is_quantized() and w.w is a


def test_load_qlinear_quantized():
    a = arr(1)
    weights = {"layer.proj.weight": a, "layer.proj.scales": a, "layer.proj.biases": a}
    w = models.load_qlinear(weights, "layer.proj", QuantConfig(64, 4))
    assert w.is_quantized() and (w.group_size, w.bits) == (64, 4)


def test_load_qlinear_scales_but_dense_config():
    a = arr(1)
    weights = {"layer.proj.weight": a, "layer.proj.scales": a, "layer.proj.biases": a}
    assert not models.load_qlinear(weights, "layer.proj", QuantConfig()).is_quantized()


def test_load_qlinear_missing_weight():
    with pytest.raises(KeyError):
        models.load_qlinear({}, "layer.proj", QuantConfig())


def test_load_qlinear_quantized_missing_biases():
    a = arr(1)
    with pytest.raises(KeyError, match="missing biases"):
        models.load_qlinear({"layer.proj.weight": a, "layer.proj.scales": a}, "layer.proj",
                            QuantConfig(64, 4))


def _quant_linear(N=16, K=64):
    return QLinear(arr(N, K // 8, dtype=Dtype.UINT32), arr(N, K // 64), arr(N, K // 64), 64, 4)


# ---- quant_test.go:130-156 ----
@seam
def test_qlinear_reaches_seam():
    x = arr(1, 64)
    # dense: unsupported here (2); quantized: valid, stops at the device query (5)
    for w, code in ((QLinear(arr(16, 64)), 2), (_quant_linear(), 5)):
        b = FB()
        assert b.qlinear(x, w) is None
        assert isinstance(b.err, ErrMLXUnavailable) and b.err.code == code
    b = FB()
    assert b.qlinear_bias(x, _quant_linear(), arr(16)) is None
    assert isinstance(b.err, MLXError) and b.err.code == 5


def test_qlinear_sticky_error():
    prior = RuntimeError("prior")
    b = FB(err=prior)
    assert b.qlinear(arr(1, 1), QLinear(arr(1, 1))) is None
    assert b.qembed(_quant_linear(), arr(1, dtype=Dtype.INT32)) is None
    assert b.moe_combine(arr(1, 2, 8), arr(1, 2)) is None
    assert b.err is prior


# ---- quant_test.go:158-180 ----
@seam
def test_qembed_reaches_seam():
    idx = arr(1, dtype=Dtype.INT32)
    for table, code in ((QLinear(arr(16, 64)), 2), (_quant_linear(), 5)):
        b = FB()
        assert b.qembed(table, idx) is None
        assert isinstance(b.err, ErrMLXUnavailable) and b.err.code == code


# ---- switch_glu_test.go:123-231 ----
def switch_quant_weights(E, d, h, group=64, bits=4):
    q = lambda i, o: SwitchQuant(arr(E, o, i * bits // 32, dtype=Dtype.UINT32),
                                 arr(E, o, i // group), arr(E, o, i // group), group, bits)
    return q(d, h), q(d, h), q(h, d)


def switch_inputs(L, d, k):
    return arr(1, L, d), arr(1, L, k, dtype=Dtype.INT32)


@seam
@pytest.mark.parametrize("E,L,k", [(5, 2, 3), (8, 32, 2)], ids=["no_sort", "sort"])
def test_switch_glu_quantized_graceful(E, L, k):
    gate, up, down = switch_quant_weights(E, 64, 128)
    x, inds = switch_inputs(L, 64, k)
    b = FB()
    assert b.switch_glu_quantized(x, gate, up, down, inds) is None
    assert isinstance(b.err, ErrMLXUnavailable) and b.err.code == 5


def test_switch_glu_quantized_bad_shape():
    gate, up, down = switch_quant_weights(5, 64, 128)
    b = FB()
    b.switch_glu_quantized(arr(2, 64), gate, up, down, arr(1, 2, 3, dtype=Dtype.INT32))
    assert b.err is not None and not isinstance(b.err, ErrMLXUnavailable)
    assert "want x [B,L,D] and inds [B,L,top_k], got x [2 64] inds [1 2 3]" in str(b.err)


def test_switch_glu_quantized_sticky_error():
    gate, up, down = switch_quant_weights(5, 64, 128)
    x, inds = switch_inputs(2, 64, 3)
    sentinel = RuntimeError("prior failure")
    b = FB(err=sentinel)
    assert b.switch_glu_quantized(x, gate, up, down, inds) is None
    assert b.err is sentinel


def test_switch_glu_for_dispatch():
    gate, up, down = switch_quant_weights(5, 64, 128)
    ql = lambda q: QLinear(q.w, q.scales, q.biases, q.group_size, q.bits)
    x, inds = switch_inputs(2, 64, 3)
    b = FB()
    assert b.switch_glu_for(x, QLinear(arr(5, 128, 64)), QLinear(arr(5, 128, 64)),
                            QLinear(arr(5, 64, 128)), inds) is None
    assert isinstance(b.err, MLXError) and "dense" in str(b.err)
    assert ql(gate).switch_quant().bits == 4
