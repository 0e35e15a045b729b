"""CPU checks of the weight-ingest host side: the native safetensors header parser
against the reference's own fixtures and error cases, tensor byte ranges, the
dtype mapping, the shard index, and the host-side rules of the DeepSeek int4
remap and expert stacking (no device work: the reference's stub-backed tests
exercise the same rules, compute/models/deepseekv3_test.go:296-395).

Mirrors compute/safetensors_test.go:29-160 and compute/loader_test.go:43-150.
"""
import base64
import json
import os
import struct

import pytest

from fastmlx_amd import loader
from fastmlx_amd.mlxgo import Dtype, MLXError

HERE = os.path.dirname(os.path.abspath(__file__))


def _fixture(name):
    with open(os.path.join(HERE, "golden", name)) as f:
        return json.load(f)["data"]


def _blob(header_json: str, data_len: int) -> bytes:
    h = header_json.encode()
    return struct.pack("<Q", len(h)) + h + bytes(data_len)


def test_parse_safetensors_header_parity():
    """The reference fixture cases (single, mixed, scalar, multi-rank, metadata,
    zero-size): sizes, tensor order, shapes, ranges, lookups and metadata."""
    for c in _fixture("safetensors_header.json"):
        blob = base64.b64decode(c["blob_b64"])
        h = loader.parse_safetensors_header(blob)
        t = c["truth"]
        assert h.header_size == t["header_size"], c["label"]
        assert h.data_start == t["data_start"], c["label"]
        assert len(blob) - h.data_start == t["data_len"], c["label"]
        assert len(h.tensors) == len(t["tensors"]), c["label"]
        for got, want in zip(h.tensors, t["tensors"]):
            assert (got.name, got.dtype, got.begin, got.end) == \
                (want["name"], want["dtype"], want["begin"], want["end"]), c["label"]
            assert got.shape == (want["shape"] or []), c["label"]
            info, ok = h.tensor(want["name"])
            assert ok and info.begin == want["begin"]
        assert h.metadata == t["metadata"], c["label"]


def test_parse_safetensors_header_errors():
    with pytest.raises(loader.ErrShortBuffer):
        loader.parse_safetensors_header(bytes([0, 1, 2]))
    with pytest.raises(loader.ErrHeaderTooLarge):
        loader.parse_safetensors_header(struct.pack("<Q", 1000))
    bad = [
        ('{"w":{"dtype":"Q4","shape":[2],"data_offsets":[0,8]}}', 8),    # unknown dtype
        ('{"w":{"dtype":"F32","shape":[2],"data_offsets":[0,16]}}', 16),  # size mismatch
        ('{"w":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}', 4),   # past the data
        ('{"w":{"dtype":"F32","shape":[0],"data_offsets":[8,0]}}', 8),   # begin > end
    ]
    for hj, n in bad:
        with pytest.raises(MLXError) as ei:
            loader.parse_safetensors_header(_blob(hj, n))
        assert not isinstance(ei.value, (loader.ErrShortBuffer, loader.ErrHeaderTooLarge)), hj


def test_parse_json_forms():
    """JSON the reference's decoder accepts or rejects: escapes, repeated keys (last
    wins), unknown fields, whitespace, null shape (a scalar), float8 tags."""
    hj = ('{ "caf\\u00e9\\ud83d\\ude00" : {"dtype":"F32","shape":[1],"data_offsets":[0,4],'
          '"extra":{"a":[1,2.5e3,true,null]}},\n "w":{"dtype":"F32","shape":[9],'
          '"data_offsets":[0,36]}, "w":{"dtype":"U8","shape":[2],"data_offsets":[4,6]},'
          '"s":{"dtype":"F8_E4M3","shape":null,"data_offsets":[6,7]},'
          '"__metadata__":{"k":"v\\n","k":"last"} }\t')
    h = loader.parse_safetensors_header(_blob(hj, 7))
    assert [t.name for t in h.tensors] == ["café\U0001F600", "w", "s"]
    assert [t.dtype for t in h.tensors] == ["F32", "U8", "F8_E4M3"]
    assert h.tensors[2].shape == [] and h.tensors[1].shape == [2]
    assert h.metadata == {"k": "last"}
    for hj_bad in ['{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}} x',   # trailing
                   '{"w":{"dtype":"F32","shape":[1.0],"data_offsets":[0,4]}}',   # float dim
                   '{"w":{"dtype":"F32","shape":[1],"data_offsets":[-1,4]}}',    # negative
                   '{"__metadata__":{"k":1}}',                                   # non-string
                   '{"w":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}',      # unclosed
                   '["w"]', '{"w":3}', '{"w":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}}']:
        with pytest.raises(MLXError):
            loader.parse_safetensors_header(_blob(hj_bad, 4))
    # A name or metadata string that decodes a NUL is refused: the C-ABI hands
    # names out as C strings, so such a tensor could not be looked up again (Go
    # strings can hold it; this is the one form the reference accepts and this
    # parser does not).
    for hj_nul in ['{"a\\u0000b":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}',
                   '{"__metadata__":{"k\\u0000":"v"}}', '{"__metadata__":{"k":"\\u0000"}}']:
        with pytest.raises(MLXError, match="NUL"):
            loader.parse_safetensors_header(_blob(hj_nul, 4))
    # a null entry decodes to the zero record, whose empty dtype is unknown
    with pytest.raises(MLXError):
        loader.parse_safetensors_header(_blob('{"w":null}', 0))
    # metadata null is a nil map; {} an empty one
    assert loader.parse_safetensors_header(_blob('{"__metadata__":null}', 0)).metadata is None
    assert loader.parse_safetensors_header(_blob('{"__metadata__":{}}', 0)).metadata == {}


def test_tensor_bytes_parity():
    f = _fixture("loader_tensors.json")
    blob = base64.b64decode(f["blob_b64"])
    h = loader.parse_safetensors_header(blob)
    assert h.data_start == f["data_start"]
    for name, exp in f["expected"].items():
        info, ok = h.tensor(name)
        assert ok, name
        assert bytes(loader.tensor_bytes(blob, h, info)) == base64.b64decode(exp["bytes_b64"])
        assert info.dtype == exp["dtype"] and info.shape == exp["shape"]


def test_tensor_bytes_out_of_bounds():
    f = _fixture("loader_tensors.json")
    blob = base64.b64decode(f["blob_b64"])
    h = loader.parse_safetensors_header(blob)
    bad = loader.TensorInfo("x", "F32", [4], 0, 16)
    with pytest.raises(MLXError):
        loader.tensor_bytes(blob[:h.data_start + 4], h, bad)


def test_mlxgo_dtype():
    assert loader.mlxgo_dtype("F8_E5M2") == (None, False)
    assert loader.mlxgo_dtype("F8_E4M3") == (None, False)
    for tag, want in {"BOOL": Dtype.BOOL, "F16": Dtype.FLOAT16, "BF16": Dtype.BFLOAT16,
                      "F32": Dtype.FLOAT32, "I64": Dtype.INT64, "U8": Dtype.UINT8,
                      "U32": Dtype.UINT32, "I32": Dtype.INT32, "F64": Dtype.FLOAT64}.items():
        assert loader.mlxgo_dtype(tag) == (want, True), tag


def test_parse_safetensors_index():
    doc = ('{"metadata":{"total_size":1024},"weight_map":{'
           '"model.layers.0.w":"model-00001-of-00002.safetensors",'
           '"model.layers.1.w":"model-00002-of-00002.safetensors",'
           '"model.embed":"model-00001-of-00002.safetensors"}}')
    idx = loader.parse_safetensors_index(doc)
    assert idx.shards == ["model-00001-of-00002.safetensors",
                          "model-00002-of-00002.safetensors"]
    assert idx.shard_for("model.embed") == ("model-00001-of-00002.safetensors", True)
    assert idx.shard_for("missing")[1] is False
    with pytest.raises(MLXError):
        loader.parse_safetensors_index('{"weight_map":{}}')


def test_merge_tensors():
    merged = loader.merge_tensors({"w1": 1}, {"w2": 2})
    assert merged == {"w1": 1, "w2": 2}
    with pytest.raises(MLXError):
        loader.merge_tensors({"dup": 1}, {"dup": 2})


def test_checkpoint_file_selection(tmp_path):
    d = tmp_path / "ck"
    d.mkdir()
    with pytest.raises(MLXError):
        loader.load_checkpoint(str(d))  # no config.json
    (d / "config.json").write_text("{}")
    with pytest.raises(MLXError):
        loader.shard_files(str(d))      # no safetensors
    for n in ("b.safetensors", "a.safetensors"):
        (d / n).write_bytes(b"")
    assert [os.path.basename(p) for p in loader.shard_files(str(d))] == \
        ["a.safetensors", "b.safetensors"]
    (d / "model.safetensors.index.json").write_text('{"weight_map":{"w":"b.safetensors"}}')
    assert [os.path.basename(p) for p in loader.shard_files(str(d))] == ["b.safetensors"]
    (d / "model.safetensors.index.json").write_text('{"weight_map":{}}')
    with pytest.raises(MLXError):
        loader.shard_files(str(d))


def test_remap_int4_host_rules():
    base = "model.layers.0.mlp.gate_proj."
    with pytest.raises(MLXError):
        loader.remap_int4({base + "weight_scale": 0, base + "weight_shape": 0})
    with pytest.raises(MLXError):
        loader.remap_int4({base + "weight_packed": 0, base + "weight_shape": 0})
    no_shape = {base + "weight_scale": 0, base + "weight_packed": 0,
                "model.layers.0.attn.weight_scale_inv": 0, "model.embed_tokens.weight": 0}
    loader.remap_int4(no_shape)
    assert sorted(no_shape) == ["model.embed_tokens.weight",
                                "model.layers.0.attn.weight_scale_inv"]


def test_stack_experts_host_rules():
    stacked = {"model.layers.0.mlp.switch_mlp.gate_proj.weight": 0}
    loader.stack_experts(stacked, 1, 3)
    assert list(stacked) == ["model.layers.0.mlp.switch_mlp.gate_proj.weight"]
    missing = {"model.layers.0.mlp.experts.0.gate_proj.weight": 0,
               "model.layers.0.mlp.experts.1.gate_proj.weight": 0}
    with pytest.raises(MLXError):
        loader.stack_experts(missing, 1, 3)


def test_absorb_kvb_host_rules():
    """TestAbsorbKVB's host-side cases (deepseekv3_test.go:398-447): a quantized
    kv_b_proj without biases is a missing-key error raised before any device op,
    and a checkpoint already carrying embed_q / unembed_out (no kv_b_proj) passes
    through untouched."""
    prefix = "model.layers.0.self_attn"
    missing = {prefix + ".kv_b_proj.weight": 0, prefix + ".kv_b_proj.scales": 0}
    with pytest.raises(MLXError) as ei:
        loader.absorb_kvb(missing, 1, 4, 64, 32, 128)
    assert "kv_b_proj.biases" in str(ei.value)
    absorbed = {prefix + ".embed_q.weight": 0, prefix + ".unembed_out.weight": 0}
    loader.absorb_kvb(absorbed, 1, 4, 64, 32, 128)
    assert sorted(absorbed) == [prefix + ".embed_q.weight", prefix + ".unembed_out.weight"]
    assert absorbed[prefix + ".embed_q.weight"] == 0
