"""Weight ingest: safetensors checkpoints into device arrays, and the DeepSeek
int4 sanitize steps that turn them into the affine triples the kernels read.

Mirrors, name for name:
    ParseSafetensorsHeader, TensorInfo, SafetensorsHeader  (compute/safetensors.go)
    ParseSafetensorsIndex, SafetensorsIndex                (compute/safetensors_index.go)
    mlxgoDtype, TensorBytes, LoadTensors, MergeTensors     (compute/loader.go)
    LoadCheckpoint, shardFiles                             (compute/checkpoint.go)
    remapInt4, scaleNeg8, stackExperts                     (compute/models/deepseekv3.go:486-592)
    absorbKVB                                              (compute/models/deepseekv3.go:609-679)

The container header is parsed by libfmxq's native parser
(fmx_safetensors_parse); tensor bytes go to the device unchanged through
fmx_safetensors_load.  Errors raise MLXError subclasses; the two sentinel
header errors of the reference have their own classes.
"""
from __future__ import annotations

import ctypes
import glob
import json
import os
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

from ._lib import FmxArray, load
from .mlxgo import (Array, Dtype, MLXError, Stream, _check, contiguous, dequantize, quantize,
                    reshape, scale_neg8, split_sections, stack, swapaxes, view)


class ErrShortBuffer(MLXError):
    """The data is too small to hold the 8-byte length prefix."""


class ErrHeaderTooLarge(MLXError):
    """The declared header length does not fit in the buffer."""


@dataclass
class TensorInfo:
    """One weight of a container: dtype tag, shape and the [begin, end) byte range
    of its data relative to the data start (safetensors.go:42-48)."""

    name: str
    dtype: str
    shape: List[int]
    begin: int
    end: int

    def num_elements(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    def num_bytes(self) -> int:
        return self.end - self.begin


@dataclass
class SafetensorsHeader:
    """Tensors in (begin, name) order, a name index, the optional __metadata__ map
    (None when absent), the header length and the data start (safetensors.go:65-76)."""

    tensors: List[TensorInfo]
    by_name: Dict[str, int]
    metadata: Optional[Dict[str, str]]
    header_size: int
    data_start: int

    def tensor(self, name: str) -> Tuple[Optional[TensorInfo], bool]:
        i = self.by_name.get(name)
        return (None, False) if i is None else (self.tensors[i], True)


def _blob_ptr(blob):
    """(pointer, length, keepalive) of a bytes-like or numpy blob, without a copy."""
    a = blob if isinstance(blob, np.ndarray) else np.frombuffer(blob, dtype=np.uint8)
    if a.dtype != np.uint8 or not a.flags.c_contiguous:
        a = np.ascontiguousarray(a).view(np.uint8)
    return (a.ctypes.data if a.size else None), int(a.size), a


class _Header:
    """Owns an fmx_st_header handle."""

    def __init__(self, blob):
        self.ptr, self.len, self._keep = _blob_ptr(blob)
        h = ctypes.c_void_p()
        rc = load().fmx_safetensors_parse(self.ptr, self.len, ctypes.byref(h))
        if rc != 0:
            msg = load().fmxq_last_error()
            text = msg.decode() if msg else ""
            if rc == 3:
                raise (ErrShortBuffer if self.len < 8 else ErrHeaderTooLarge)(rc, text)
            raise MLXError(rc, text)
        self.h = h

    def close(self):
        if self.h:
            load().fmx_safetensors_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def to_python(self) -> SafetensorsHeader:
        lib = load()
        tensors = []
        for i in range(lib.fmx_safetensors_count(self.h)):
            name, dt = ctypes.c_char_p(), ctypes.c_char_p()
            nd = ctypes.c_int()
            shp = ctypes.POINTER(ctypes.c_int64)()
            b, e = ctypes.c_uint64(), ctypes.c_uint64()
            _check(lib.fmx_safetensors_tensor(self.h, i, ctypes.byref(name), ctypes.byref(dt),
                                              ctypes.byref(nd), ctypes.byref(shp),
                                              ctypes.byref(b), ctypes.byref(e)))
            tensors.append(TensorInfo(name.value.decode("utf-8", "surrogateescape"),
                                      dt.value.decode(), [shp[d] for d in range(nd.value)],
                                      b.value, e.value))
        nm = lib.fmx_safetensors_metadata_count(self.h)
        meta = None
        if nm >= 0:
            meta = {}
            for i in range(nm):
                k, v = ctypes.c_char_p(), ctypes.c_char_p()
                _check(lib.fmx_safetensors_metadata(self.h, i, ctypes.byref(k), ctypes.byref(v)))
                meta[k.value.decode("utf-8", "surrogateescape")] = \
                    v.value.decode("utf-8", "surrogateescape")
        return SafetensorsHeader(tensors, {t.name: i for i, t in enumerate(tensors)}, meta,
                                 int(lib.fmx_safetensors_header_size(self.h)),
                                 int(lib.fmx_safetensors_data_start(self.h)))


def parse_safetensors_header(data) -> SafetensorsHeader:
    """ParseSafetensorsHeader (safetensors.go:101-165): validate and list the
    container's tensors; the data itself is not read."""
    h = _Header(data)
    try:
        return h.to_python()
    finally:
        h.close()


def mlxgo_dtype(tag: str) -> Tuple[Optional[Dtype], bool]:
    """The array dtype of a safetensors tag; float8 tags have none (loader.go:13-42)."""
    out = ctypes.c_int()
    if load().fmx_safetensors_dtype(tag.encode(), ctypes.byref(out)) != 0:
        return None, False
    return Dtype(out.value), True


def tensor_bytes(blob, h: SafetensorsHeader, t: TensorInfo) -> memoryview:
    """The raw data slice of one tensor, bounds-checked against the blob
    (TensorBytes, loader.go:47-55)."""
    _, n, keep = _blob_ptr(blob)
    off = ctypes.c_uint64()
    rc = load().fmx_safetensors_slice(n, h.data_start, t.begin, t.end, ctypes.byref(off))
    if rc != 0:
        msg = load().fmxq_last_error()
        raise MLXError(rc, f"tensor {t.name!r}: " + (msg.decode() if msg else ""))
    return memoryview(keep)[off.value:off.value + (t.end - t.begin)]


def load_tensors(blob, s: Optional[Stream] = None) -> Dict[str, Array]:
    """LoadTensors (loader.go:61-84): every tensor's bytes uploaded unchanged into
    a device array of its dtype; __metadata__ is not a tensor."""
    h = _Header(blob)
    try:
        lib = load()
        out: Dict[str, Array] = {}
        for i in range(lib.fmx_safetensors_count(h.h)):
            a = FmxArray(None)
            _check(lib.fmx_safetensors_load(ctypes.byref(a), h.ptr, h.len, h.h, i))
            name = ctypes.c_char_p()
            _check(lib.fmx_safetensors_tensor(h.h, i, ctypes.byref(name), None, None, None, None,
                                              None))
            out[name.value.decode("utf-8", "surrogateescape")] = Array(a)
        return out
    finally:
        h.close()


def merge_tensors(*shards: Dict[str, Array]) -> Dict[str, Array]:
    """MergeTensors (loader.go:88-103): a name in more than one shard is an error."""
    out: Dict[str, Array] = {}
    for sh in shards:
        for name, arr in sh.items():
            if name in out:
                raise MLXError(1, f"safetensors: weight {name!r} present in more than one shard")
            out[name] = arr
    return out


@dataclass
class SafetensorsIndex:
    """model.safetensors.index.json (safetensors_index.go:15-25)."""

    weight_map: Dict[str, str]
    shards: List[str]
    metadata: Optional[dict] = field(default=None)

    def shard_for(self, weight: str) -> Tuple[Optional[str], bool]:
        f = self.weight_map.get(weight)
        return f, f is not None


def parse_safetensors_index(data) -> SafetensorsIndex:
    """ParseSafetensorsIndex (safetensors_index.go:30-56): a non-empty weight_map;
    shards deduplicated and sorted."""
    try:
        doc = json.loads(data)
    except (ValueError, TypeError) as e:
        raise MLXError(1, f"safetensors index: {e}") from None
    if not isinstance(doc, dict):
        raise MLXError(1, "safetensors index: not an object")
    wm = doc.get("weight_map") or {}
    if not isinstance(wm, dict) or not wm or not all(isinstance(v, str) for v in wm.values()):
        raise MLXError(1, "safetensors index: empty or missing weight_map")
    return SafetensorsIndex(dict(wm), sorted(set(wm.values())), doc.get("metadata"))


CONFIG_FILE_NAME = "config.json"
SAFETENSORS_INDEX_NAME = "model.safetensors.index.json"


def shard_files(dir: str) -> List[str]:
    """shardFiles (checkpoint.go:67-90): the index's shards, else every
    *.safetensors in the directory, sorted."""
    ip = os.path.join(dir, SAFETENSORS_INDEX_NAME)
    if os.path.exists(ip):
        with open(ip, "rb") as f:
            idx = parse_safetensors_index(f.read())
        return [os.path.join(dir, n) for n in idx.shards]
    files = sorted(glob.glob(os.path.join(dir, "*.safetensors")))
    if not files:
        raise MLXError(1, f"checkpoint: no safetensors files in {dir}")
    return files


def load_checkpoint(dir: str, s: Optional[Stream] = None) -> Tuple[bytes, Dict[str, Array]]:
    """LoadCheckpoint (checkpoint.go:31-64): config.json plus the merged weights
    of every shard; each shard is memory-mapped, not read whole."""
    try:
        with open(os.path.join(dir, CONFIG_FILE_NAME), "rb") as f:
            cfg = f.read()
    except OSError as e:
        raise MLXError(1, f"checkpoint: read config: {e}") from None
    shards = []
    for path in shard_files(dir):
        try:
            blob = np.memmap(path, dtype=np.uint8, mode="r") if os.path.getsize(path) else b""
        except OSError as e:
            raise MLXError(1, f"checkpoint: read shard {os.path.basename(path)}: {e}") from None
        try:
            shards.append(load_tensors(blob, s))
        except MLXError as e:
            raise MLXError(e.code, f"checkpoint: load shard {os.path.basename(path)}: {e}") \
                from None
    return cfg, merge_tensors(*shards)


def remap_int4(weights: Dict[str, Array], s: Optional[Stream] = None) -> None:
    """remapInt4 (deepseekv3.go:497-537): each BASEweight_shape triple becomes
    BASEweight (packed bytes viewed as uint32), BASEscales (the scale) and
    BASEbiases (-8 * scale in the scale's dtype); the source keys and any orphan
    weight_scale / weight_packed keys are dropped (weight_scale_inv is kept)."""
    bases = [k[:-len("weight_shape")] for k in list(weights) if k.endswith("weight_shape")]
    for base in bases:
        packed = weights.get(base + "weight_packed")
        if packed is None:
            raise MLXError(1, f"deepseekv3: int4 remap missing {base + 'weight_packed'!r}")
        scale = weights.get(base + "weight_scale")
        if scale is None:
            raise MLXError(1, f"deepseekv3: int4 remap missing {base + 'weight_scale'!r}")
        w = view(packed, Dtype.UINT32, s)
        biases = scale_neg8(scale, s)
        for suffix in ("weight_shape", "weight_packed", "weight_scale"):
            del weights[base + suffix]
        weights[base + "weight"] = w
        weights[base + "scales"] = scale
        weights[base + "biases"] = biases
    for k in list(weights):
        if k.endswith("weight_scale") or k.endswith("weight_packed"):
            del weights[k]


def stack_experts(weights: Dict[str, Array], num_layers: int, num_experts: int,
                  s: Optional[Stream] = None) -> None:
    """stackExperts (deepseekv3.go:564-592): model.layers.L.mlp.experts.E.PROJ.COMP
    joined along a new expert axis into model.layers.L.mlp.switch_mlp.PROJ.COMP."""
    for layer in range(num_layers):
        for proj in ("gate_proj", "down_proj", "up_proj"):
            for comp in ("weight", "scales", "biases"):
                first = f"model.layers.{layer}.mlp.experts.0.{proj}.{comp}"
                if first not in weights:
                    continue
                parts = []
                for e in range(num_experts):
                    key = f"model.layers.{layer}.mlp.experts.{e}.{proj}.{comp}"
                    if key not in weights:
                        raise MLXError(1, f"deepseekv3: stack experts missing {key!r}")
                    parts.append(weights[key])
                stacked = stack(parts, 0, s)
                for e in range(num_experts):
                    del weights[f"model.layers.{layer}.mlp.experts.{e}.{proj}.{comp}"]
                weights[f"model.layers.{layer}.mlp.switch_mlp.{proj}.{comp}"] = stacked


def absorb_kvb(weights: Dict[str, Array], num_layers: int, num_attention_heads: int,
               qk_nope_head_dim: int, v_head_dim: int, kv_lora_rank: int,
               s: Optional[Stream] = None) -> None:
    """absorbKVB (deepseekv3.go:609-679): each layer's self_attn.kv_b_proj
    [heads * (nope + v), kv_lora] becomes embed_q [heads, kv_lora, nope] (the nope
    band, transposed) and unembed_out [heads, v, kv_lora] (the value band).  A
    quantized kv_b_proj is dequantized first, with bits and group size read off
    the packed and scale shapes, and both results are requantized with them.
    A layer without kv_b_proj (already absorbed) is left as it is."""
    head_dim = qk_nope_head_dim + v_head_dim
    for layer in range(num_layers):
        prefix = f"model.layers.{layer}.self_attn"
        v = weights.pop(prefix + ".kv_b_proj.weight", None)
        if v is None:
            continue
        quantized = False
        bits = group_size = 0
        scales = weights.get(prefix + ".kv_b_proj.scales")
        if scales is not None:
            quantized = True
            biases = weights.get(prefix + ".kv_b_proj.biases")
            if biases is None:
                raise MLXError(1, f"deepseekv3: kv_b_proj absorption missing "
                                  f"{prefix + '.kv_b_proj.biases'!r}")
            del weights[prefix + ".kv_b_proj.scales"]
            del weights[prefix + ".kv_b_proj.biases"]
            bits = (v.shape()[-1] * 32) // kv_lora_rank
            group_size = kv_lora_rank // scales.shape()[-1]
            v = dequantize(v, scales, biases, group_size, bits, s)
        v = reshape(v, [num_attention_heads, head_dim, -1], s)
        nope, val = split_sections(v, [qk_nope_head_dim], 1, s)
        wk = contiguous(swapaxes(nope, -1, -2, s), s)
        wv = contiguous(val, s)
        if quantized:
            wk_p, wk_s, wk_b = quantize(wk, group_size, bits, s)
            wv_p, wv_s, wv_b = quantize(wv, group_size, bits, s)
            weights[prefix + ".embed_q.scales"] = wk_s
            weights[prefix + ".unembed_out.scales"] = wv_s
            weights[prefix + ".embed_q.biases"] = wk_b
            weights[prefix + ".unembed_out.biases"] = wv_b
            wk, wv = wk_p, wv_p
        weights[prefix + ".embed_q.weight"] = wk
        weights[prefix + ".unembed_out.weight"] = wv
