"""GPU checks of the weight ingest: tensors uploaded byte for byte from a
safetensors container, the int4 remap ops (u8 -> u32 view, -8 * scale) against
closed forms, the expert stack, and a synthetic compressed-tensors int4
checkpoint taken through load -> remapInt4 -> stackExperts -> SwitchGLU against
the oracle (compute/models/deepseekv3.go:486-592, compute/loader.go:61-84).
"""
import base64
import json
import os
import struct

import numpy as np
import pytest

from gpu_util import announce
import parity
from synth import make_x, topk_uniform

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))

_TAG = {np.dtype(np.uint8): "U8", np.dtype(np.int64): "I64", np.dtype(np.float32): "F32",
        np.dtype(np.float16): "F16", np.dtype(np.int32): "I32"}


def write_safetensors(tensors: dict, metadata=None) -> bytes:
    """A container from {name: (tag or None, ndarray)}; bf16 passes as uint16 bits
    with tag "BF16"."""
    header, chunks, off = {}, [], 0
    for name, (tag, arr) in tensors.items():
        arr = np.ascontiguousarray(arr)
        raw = arr.tobytes()
        header[name] = {"dtype": tag or _TAG[arr.dtype], "shape": list(arr.shape),
                        "data_offsets": [off, off + len(raw)]}
        chunks.append(raw)
        off += len(raw)
    if metadata is not None:
        header["__metadata__"] = metadata
    hj = json.dumps(header).encode()
    hj += b" " * (-len(hj) % 8)
    return struct.pack("<Q", len(hj)) + hj + b"".join(chunks)


def test_load_tensors_parity(gpu):
    from fastmlx_amd import loader
    from fastmlx_amd.mlxgo import Dtype

    with open(os.path.join(HERE, "golden", "loader_tensors.json")) as f:
        fx = json.load(f)["data"]
    blob = base64.b64decode(fx["blob_b64"])
    announce("load_tensors fixture")
    w = loader.load_tensors(blob)
    assert sorted(w) == sorted(fx["expected"])
    tags = {Dtype.FLOAT32: "F32", Dtype.INT32: "I32", Dtype.BFLOAT16: "BF16"}
    for name, exp in fx["expected"].items():
        a = w[name]
        assert a.shape() == exp["shape"] and tags[a.dtype()] == exp["dtype"], name
        assert a.to_numpy().tobytes() == base64.b64decode(exp["bytes_b64"]), name


def test_scale_neg8_known_answers(gpu):
    """-8 * s changes only sign and exponent: known bf16 results (normal, negative,
    subnormal, overflow to infinity) and the same identity over a sweep, for
    bf16, f16 and f32 scales."""
    from fastmlx_amd.mlxgo import Array, Dtype, scale_neg8

    announce("scale_neg8")
    cases = {0x3F80: 0xC100,   # 1.0 -> -8.0
             0xBF00: 0x4080,   # -0.5 -> 4.0
             0x0001: 0x8008,   # smallest subnormal 2^-133 -> -2^-130 (still subnormal)
             0x0000: 0x8000,   # +0 -> -0
             0x7F7F: 0xFF80,   # largest finite -> -inf
             0x3C23: 0xBDA3}   # 0.00995 (2^-7 * 1.2734) -> -0.0796 (2^-4 * 1.2734)
    s = np.array(list(cases), dtype=np.uint16)
    got = scale_neg8(Array.from_numpy(s, Dtype.BFLOAT16)).to_numpy()
    assert got.tolist() == list(cases.values())
    # sweep: every finite bf16 exponent; the result's bits are the input's with the
    # sign flipped and the exponent raised by 3 (or infinity past the top)
    rng = np.random.default_rng(3)
    pats = rng.integers(0, 0x7F80, size=4096).astype(np.uint16)
    pats |= (rng.integers(0, 2, size=4096).astype(np.uint16) << 15)
    got = scale_neg8(Array.from_numpy(pats, Dtype.BFLOAT16)).to_numpy()
    with np.errstate(over="ignore"):
        f = (pats.astype(np.uint32) << 16).view(np.float32) * np.float32(-8.0)
    assert np.array_equal(got, (f.view(np.uint32) >> 16).astype(np.uint16))
    h = rng.standard_normal(1000).astype(np.float16) * np.float16(3000)
    got = scale_neg8(Array.from_numpy(h)).to_numpy()
    with np.errstate(over="ignore"):
        assert np.array_equal(got.view(np.uint16),
                              (h.astype(np.float32) * -8).astype(np.float16).view(np.uint16))
    f32 = rng.standard_normal(1000).astype(np.float32)
    assert np.array_equal(scale_neg8(Array.from_numpy(f32)).to_numpy(), f32 * np.float32(-8))


def test_view_and_stack(gpu):
    from fastmlx_amd.mlxgo import Array, Dtype, MLXError, stack, view

    announce("view / stack")
    rng = np.random.default_rng(5)
    u8 = rng.integers(0, 256, size=(3, 16), dtype=np.uint8)
    v = view(Array.from_numpy(u8), Dtype.UINT32)
    assert v.shape() == [3, 4] and v.dtype() == Dtype.UINT32
    assert np.array_equal(v.to_numpy(), u8.view("<u4"))
    with pytest.raises(MLXError):
        view(Array.from_numpy(u8[:, :7].copy()), Dtype.UINT32)
    parts = [rng.standard_normal((2, 5)).astype(np.float32) for _ in range(3)]
    st = stack([Array.from_numpy(p) for p in parts])
    assert st.shape() == [3, 2, 5]
    assert np.array_equal(st.to_numpy(), np.stack(parts))
    with pytest.raises(MLXError):
        stack([Array.from_numpy(parts[0]), Array.from_numpy(parts[1][:, :4].copy())])


def test_int4_checkpoint_to_switch_glu(gpu, oracle):
    """A compressed-tensors int4 MoE layer: per-expert weight_packed (u8) /
    weight_scale (bf16) / weight_shape keys in a safetensors container, loaded,
    remapped (w viewed as u32, biases = -8 * scale), stacked, then SwitchGLU on
    the device against the oracle on the same bytes."""
    from fastmlx_amd import loader, mlxgo
    from synth import f32_to_bf16

    rng = np.random.default_rng(11)
    E, D, I, T, k = 4, 256, 128, 9, 2
    tensors, ref = {}, {}
    for e in range(E):
        for proj, (n, kk) in (("gate_proj", (I, D)), ("up_proj", (I, D)), ("down_proj", (D, I))):
            base = f"model.layers.0.mlp.experts.{e}.{proj}."
            packed = rng.integers(0, 256, size=(n, kk // 2), dtype=np.uint8)
            scale = f32_to_bf16(rng.uniform(0.002, 0.02, size=(n, kk // 64)).astype(np.float32))
            tensors[base + "weight_packed"] = (None, packed)
            tensors[base + "weight_scale"] = ("BF16", scale)
            tensors[base + "weight_shape"] = (None, np.array([n, kk], dtype=np.int64))
            ref[(e, proj)] = (packed, scale)
    tensors["model.embed_tokens.weight"] = ("BF16", make_x(rng, 8, D))
    blob = write_safetensors(tensors, {"format": "pt"})
    announce("int4 checkpoint -> remap -> stack -> switch_glu")
    w = loader.load_tensors(blob)
    loader.remap_int4(w)
    loader.stack_experts(w, 1, E)
    key = "model.layers.0.mlp.switch_mlp.{}.{}"
    assert not any(".experts." in k for k in w)
    trip = {}
    for proj in ("gate_proj", "up_proj", "down_proj"):
        ws, ss, bs = (w[key.format(proj, c)] for c in ("weight", "scales", "biases"))
        pk = np.stack([ref[(e, proj)][0] for e in range(E)])
        sc = np.stack([ref[(e, proj)][1] for e in range(E)])
        assert np.array_equal(ws.to_numpy(), pk.view("<u4"))
        assert np.array_equal(ss.to_numpy(), sc)
        bexp = (((sc.astype(np.uint32) << 16).view(np.float32) * np.float32(-8))
                .view(np.uint32) >> 16).astype(np.uint16)
        assert np.array_equal(bs.to_numpy(), bexp)
        trip[proj] = (ws, ss, bs)
    x = make_x(rng, T, D)
    inds = topk_uniform(rng, T, E, k)
    y = mlxgo.switch_glu(mlxgo.Array.from_numpy(x.reshape(1, T, D), mlxgo.Dtype.BFLOAT16),
                         mlxgo.Array.from_numpy(inds.reshape(1, T, k).astype(np.int32)),
                         trip["gate_proj"], trip["up_proj"], trip["down_proj"], 64, 4)
    got = y.to_numpy().reshape(T, k, D)
    np_trip = {p: tuple(a.to_numpy() for a in trip[p]) for p in trip}
    sref = parity.SwitchRef(x, inds, np_trip["gate_proj"], np_trip["up_proj"],
                            np_trip["down_proj"], 64, 4)
    parity.check_switch(got, sref)
