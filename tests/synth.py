"""Seeded synthetic inputs for the BASELINE configurations (numpy, test side).

Distributions follow BASELINE.json's configs:
  int4: q ~ U{0..15}, s ~ U[0.002, 0.02] -> bf16, b = bf16(-8 s + N(0, 1e-3))
  int8: q ~ U{0..255}, s ~ U[1e-4, 2e-3] -> bf16, b = bf16(-128 s)
  x ~ N(0, 1) -> bf16
All bf16 tensors are uint16 bit patterns; packed weights are uint32.
"""
from __future__ import annotations

import numpy as np

from oracle import bf16_to_f32, f32_to_bf16


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """Pack [..., K] integers LSB-first into [..., K*bits/32] uint32."""
    per = 32 // bits
    q = q.astype(np.uint32)
    shp = q.shape[:-1] + (q.shape[-1] // per, per)
    q = q.reshape(shp)
    shifts = (np.arange(per, dtype=np.uint32) * bits).astype(np.uint32)
    return np.bitwise_or.reduce(q << shifts, axis=-1).astype(np.uint32)


def unpack(w: np.ndarray, bits: int) -> np.ndarray:
    per = 32 // bits
    shifts = (np.arange(per, dtype=np.uint32) * bits).astype(np.uint32)
    q = (w[..., None] >> shifts) & np.uint32((1 << bits) - 1)
    return q.reshape(w.shape[:-1] + (w.shape[-1] * per,))


def make_x(rng: np.random.Generator, *shape) -> np.ndarray:
    return f32_to_bf16(rng.standard_normal(shape, dtype=np.float32))


def make_quant(rng: np.random.Generator, lead: tuple, K: int, bits: int = 4, group: int = 64):
    """Quantized weight triple with leading shape `lead` (e.g. (N,) or (E, N))."""
    G = K // group
    # uniform random words are uniform, independent q values in every nibble/byte
    w = rng.integers(0, 1 << 32, size=lead + (K * bits // 32,), dtype=np.uint32)
    if bits == 4:
        s = rng.uniform(0.002, 0.02, size=lead + (G,)).astype(np.float32)
        s16 = f32_to_bf16(s)
        sf = bf16_to_f32(s16)
        noise = (rng.standard_normal(lead + (G,), dtype=np.float32) * np.float32(1e-3))
        b16 = f32_to_bf16(np.float32(-8.0) * sf + noise)
    else:
        s = rng.uniform(1e-4, 2e-3, size=lead + (G,)).astype(np.float32)
        s16 = f32_to_bf16(s)
        b16 = f32_to_bf16(np.float32(-128.0) * bf16_to_f32(s16))
    return np.ascontiguousarray(w), np.ascontiguousarray(s16), np.ascontiguousarray(b16)


def deq_numpy(w, s16, b16, bits: int, group: int, fused: bool = False) -> np.ndarray:
    """Independent vectorised dequantize (numpy), fp32 value of each bf16 result."""
    q = unpack(w, bits).astype(np.float32)
    s = np.repeat(bf16_to_f32(s16), group, axis=-1)
    b = np.repeat(bf16_to_f32(b16), group, axis=-1)
    if fused:
        return bf16_to_f32(f32_to_bf16(q * s + b))
    return bf16_to_f32(f32_to_bf16(bf16_to_f32(f32_to_bf16(q * s)) + b))


def rel_err(y, ref) -> float:
    """max|y - ref| / max|ref|, the parity metric of the north star."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref))
    return float(np.max(np.abs(y - ref)) / (den if den > 0 else 1.0))


TOL = 2e-2  # max-abs-rel on bf16 outputs with fp32 accumulation


def topk_uniform(rng, M: int, E: int, k: int) -> np.ndarray:
    """Each token picks k distinct experts uniformly (config 3)."""
    return np.stack([rng.choice(E, size=k, replace=False) for _ in range(M)]).astype(np.int32)


def topk_zipf(rng, M: int, E: int, k: int, s: float = 1.1) -> np.ndarray:
    """k distinct ids per token by sequential draws from Zipf p(r) ~ r^-s (config 4)."""
    p = np.arange(1, E + 1, dtype=np.float64) ** (-s)
    out = np.empty((M, k), dtype=np.int32)
    for t in range(M):
        pp = p.copy()
        for j in range(k):
            pp_n = pp / pp.sum()
            e = rng.choice(E, p=pp_n)
            out[t, j] = e
            pp[e] = 0.0
    return out
