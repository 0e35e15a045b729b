"""The reference's model-side quantized-linear layer, over :mod:`fastmlx_amd.mlxgo`.

Restates, with the same names, rules and error behaviour:

* compute/models/quant.go -- ``QuantConfig`` / ``parse_quant_config`` (:15-46),
  ``QLinear`` / ``load_qlinear`` (:54-85), ``FB.qlinear`` (:91-101),
  ``FB.qlinear_bias`` (:105-111), ``FB.qembed`` (:117-142);
* compute/models/switch_glu.go -- ``SwitchQuant`` (:51-61), ``FB.switch_glu_for``
  (:68-73), ``FB.switch_glu_quantized`` / ``switch_glu_core`` (:79-153) with the
  rank guard of :13-15 and :113-116;
* the MoE combine of qwen3next_forward.go:520-523 and deepseekv3_forward.go:434-440
  (``FB.moe_combine``).

``FB`` is the reference's forward builder: its first error is sticky and every
later call returns ``None`` without touching the device.  The quantized paths
run on libfmxq.so; dense weights (no ``.scales``) belong to the host model's own
matmul and are reported as unsupported here rather than computed on the CPU.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from typing import Dict, Optional, Tuple

from . import mlxgo
from .mlxgo import Array, MLXError, Stream


@dataclass(frozen=True)
class QuantConfig:
    """Affine quantization geometry of a checkpoint; bits == 0 means dense."""

    group_size: int = 0
    bits: int = 0

    def quantized(self) -> bool:
        return self.bits > 0


def parse_quant_config(config_json) -> QuantConfig:
    """Read the top-level "quantization" block (quant.go:28-46).

    Absent block, bits 0, or a mode other than "affine" -> dense (zero value).
    Malformed JSON raises ``ValueError``."""
    if isinstance(config_json, (bytes, bytearray)):
        config_json = config_json.decode()
    c = json.loads(config_json)
    if not isinstance(c, dict):
        raise ValueError("config is not a JSON object")
    q = c.get("quantization")
    if not isinstance(q, dict) or not q.get("bits"):
        return QuantConfig()
    mode = q.get("mode") or ""
    if mode not in ("", "affine"):
        return QuantConfig()
    return QuantConfig(group_size=int(q.get("group_size") or 0), bits=int(q["bits"]))


@dataclass
class SwitchQuant:
    """A quantized stacked-expert projection (switch_glu.go:51-61)."""

    w: Array
    scales: Array
    biases: Array
    group_size: int
    bits: int

    def triple(self):
        return (self.w, self.scales, self.biases)


@dataclass
class QLinear:
    """A linear weight that may be affine-quantized (quant.go:54-64)."""

    w: Array
    scales: Optional[Array] = None
    biases: Optional[Array] = None
    group_size: int = 0
    bits: int = 0

    def is_quantized(self) -> bool:
        return self.scales is not None

    def switch_quant(self) -> SwitchQuant:
        return SwitchQuant(self.w, self.scales, self.biases, self.group_size, self.bits)


def load_qlinear(weights: Dict[str, Array], name: str, q: QuantConfig) -> QLinear:
    """Resolve ``name.weight`` (+ ``.scales``/``.biases``) (quant.go:68-85).

    Quantized only when the config is quantized *and* the checkpoint holds the
    module's scales; a quantized module without biases is an error."""
    w = weights.get(name + ".weight")
    if w is None:
        raise KeyError(f"models: missing weight {name + '.weight'!r}")
    lw = QLinear(w=w)
    scales = weights.get(name + ".scales")
    if q.quantized() and (name + ".scales") in weights:
        biases = weights.get(name + ".biases")
        if biases is None:
            raise KeyError(f"models: quantized {name!r} missing biases")
        lw.scales, lw.biases = scales, biases
        lw.group_size, lw.bits = q.group_size, q.bits
    return lw


def bad_switch_shape(x_shape, ind_shape) -> ValueError:
    """errBadSwitchShape (switch_glu.go:13-15)."""
    fmt = lambda s: "[" + " ".join(str(d) for d in s) + "]"
    return ValueError(f"switchGLU: want x [B,L,D] and inds [B,L,top_k], got x {fmt(x_shape)} "
                      f"inds {fmt(ind_shape)}")


class FB:
    """Forward builder with a sticky error (qwen3_forward.go:103-109)."""

    def __init__(self, s: Optional[Stream] = None, err: Optional[BaseException] = None):
        self.s = s
        self.err = err

    def _run(self, fn, *args):
        try:
            return fn(*args)
        except MLXError as e:
            self.err = e
            return None

    def _dense(self, what: str):
        self.err = MLXError(2, f"{what}: dense weights are computed by the host model's matmul, "
                               "not by this library")
        return None

    # quant.go:91-101
    def qlinear(self, x: Array, w: QLinear) -> Optional[Array]:
        if self.err is not None:
            return None
        if not w.is_quantized():
            return self._dense("qlinear")
        return self._run(mlxgo.quantized_matmul, x, w.w, w.scales, w.biases, True, w.group_size,
                         w.bits, self.s)

    # quant.go:105-111, the bias add fused into the matmul epilogue
    def qlinear_bias(self, x: Array, w: QLinear, bias: Optional[Array]) -> Optional[Array]:
        if bias is None:
            return self.qlinear(x, w)
        if self.err is not None:
            return None
        if not w.is_quantized():
            return self._dense("qlinearBias")
        return self._run(mlxgo.quantized_matmul_bias, x, w.w, w.scales, w.biases, bias, True,
                         w.group_size, w.bits, self.s)

    # quant.go:117-142, the take and the dequantize as one kernel
    def qembed(self, table: QLinear, idx: Array) -> Optional[Array]:
        if self.err is not None:
            return None
        if not table.is_quantized():
            return self._dense("qembed")
        return self._run(mlxgo.dequantize_rows, table.w, table.scales, table.biases, idx,
                         table.group_size, table.bits, self.s)

    # switch_glu.go:68-73
    def switch_glu_for(self, x: Array, gate: QLinear, up: QLinear, down: QLinear,
                       inds: Array) -> Optional[Array]:
        if self.err is not None:
            return None
        if gate.is_quantized():
            return self.switch_glu_quantized(x, gate.switch_quant(), up.switch_quant(),
                                             down.switch_quant(), inds)
        return self._dense("switchGLU")

    # switch_glu.go:79-153: the rank guard runs on the host before any kernel; the
    # routing choreography (sort at >= 64 slots, gather, silu(gate) * up, down,
    # unsort) runs on the device in one call.
    def switch_glu_quantized(self, x: Array, gate: SwitchQuant, up: SwitchQuant,
                             down: SwitchQuant, inds: Array) -> Optional[Array]:
        if self.err is not None:
            return None
        xs, ins = x.shape(), inds.shape()
        if len(xs) != 3 or len(ins) != 3:
            self.err = bad_switch_shape(xs, ins)
            return None
        if len({(q.group_size, q.bits) for q in (gate, up, down)}) != 1:
            self.err = MLXError(2, "switchGLU: gate/up/down must share group_size and bits")
            return None
        return self._run(mlxgo.switch_glu, x, inds, gate.triple(), up.triple(), down.triple(),
                         gate.group_size, gate.bits, self.s)

    # qwen3next_forward.go:513-518: softmax over the router logits, the top-k
    # experts and their gates, renormalized when norm_topk_prob.
    def route_softmax(self, gates_logits: Array, top_k: int,
                      norm_topk_prob: bool) -> Tuple[Optional[Array], Optional[Array]]:
        if self.err is not None:
            return None, None
        out = self._run(mlxgo.route_softmax_topk, gates_logits, top_k, norm_topk_prob, self.s)
        return (None, None) if out is None else out

    # deepseekv3_forward.go:452-491 (routeExperts): group-limited sigmoid routing.
    def route_experts(self, gates: Array, bias: Optional[Array], top_k: int, n_group: int,
                      topk_group: int, routed_scaling_factor: float,
                      norm_topk_prob: bool) -> Tuple[Optional[Array], Optional[Array]]:
        if self.err is not None:
            return None, None
        out = self._run(mlxgo.route_group_topk, gates, bias, top_k, n_group, topk_group,
                        routed_scaling_factor, norm_topk_prob, self.s)
        return (None, None) if out is None else out

    # qwen3next_forward.go:520-523 / deepseekv3_forward.go:434-440
    def moe_combine(self, y: Array, scores: Array, shared: Optional[Array] = None,
                    shared_gate: Optional[Array] = None) -> Optional[Array]:
        if self.err is not None:
            return None
        return self._run(mlxgo.moe_combine, y, scores, shared, shared_gate, self.s)
