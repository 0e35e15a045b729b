"""Per-element parity bounds for the product tests (test infrastructure).

The published metric (max|y - ref| / max|ref| <= 2e-2 against the fp32 oracle
with the MLX dequant) is loose: on a 14336-deep row, dropping one 64-value
group moves one output by about 2% of max|y| and still passes.  Every product
test therefore also checks each output element against an fp64 reference:

    |y - y64| <= 2^-8 * max(|y|, |y64|) + 2^-18 * A,   A = sum_k |x_k| (q_k |s| + |b|)

- The first term is the final bf16 rounding: half an ulp is at most 2^-8 of
  the value.
- The second term covers the fp32 accumulation.  The kernels' typical error is
  under 1% of that term, and a dropped, doubled or mis-scaled group is 50-200
  times larger.
- y64 is the fp64 product under the dequant definition the kernel computes.
  The integer-domain kernels (GEMV, skinny MFMA, MoE walks) form s*sum(xq) +
  b*sum(x), which is the exact affine value (oracle DEQ_EXACT). The prefill
  GEMM rounds fma(s, q, b) to bf16 once (DEQ_FUSED).
- The check takes the nearer of the two references per element. The two
  definitions differ by random-walk noise of ~0.2% of |y|, so a real slip fails
  against both.

For the SwitchGLU outputs the gate/up results pass through bf16 roundings
before the down product.  The GPU and the oracle round each intermediate
separately, so where their fp32 values straddle a rounding point an h_i
differs by an ulp.  The bound there is 2^-7 of the value (both sides are bf16)
plus 2^-5 * H, where H = sqrt(sum_i (h_i wd_i)^2) comes from the oracle per
output: four times the scale of one-ulp changes in every h_i.  A slip in one
64-value group of a down row moves the output by about sqrt(64 / I) * H, which
is 5-11 times that allowance at the configurations' I of 512 and 2048.
"""
from __future__ import annotations

import numpy as np

import oracle as _o
from synth import TOL, rel_err

ROUND = 2.0 ** -8    # half an ulp of a bf16 value, relative
ACCUM = 2.0 ** -18   # fp32 accumulation allowance, relative to A


def _abs16(h: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(h, dtype=np.uint16) & np.uint16(0x7FFF)


def f64(h: np.ndarray) -> np.ndarray:
    return _o.bf16_to_f32(h).astype(np.float64)


class DenseRef:
    """fp64 references of y = x . deq(W)^T (both kernel definitions) and A."""

    def __init__(self, x, w, s, b, group, bits, mlx=True):
        x = np.ascontiguousarray(x)
        self.exact = _o.qmm_f64(x, w, s, b, group, bits, mode=_o.DEQ_EXACT)
        self.fused = _o.qmm_f64(x, w, s, b, group, bits, mode=_o.DEQ_FUSED)
        self.mag = _o.qmm_f64(_abs16(x), w, _abs16(s), _abs16(b), group, bits,
                              mode=_o.DEQ_EXACT)
        # the published metric's reference: fp32 accumulation, MLX dequant
        self.mlx = _o.bf16_to_f32(_o.qmm(x, w, s, b, group, bits)) if mlx else None


def gather_refs(x2d, w, s, b, xrow, expert, group=64, bits=4, mlx=True):
    """DenseRef rows for a flattened gather: slot i is x2d[xrow[i]] . deq(W[expert[i]])^T."""
    xrow = np.asarray(xrow, dtype=np.int64)
    expert = np.asarray(expert, dtype=np.int64)
    S, N = xrow.size, w.shape[1]
    out = DenseRef.__new__(DenseRef)
    out.exact = np.zeros((S, N))
    out.fused = np.zeros((S, N))
    out.mag = np.zeros((S, N))
    out.mlx = np.zeros((S, N), dtype=np.float32) if mlx else None
    for e in np.unique(expert):
        sl = np.nonzero(expert == e)[0]
        r = DenseRef(np.ascontiguousarray(x2d[xrow[sl]]), w[e], s[e], b[e], group, bits, mlx)
        out.exact[sl], out.fused[sl], out.mag[sl] = r.exact, r.fused, r.mag
        if mlx:
            out.mlx[sl] = r.mlx
    return out


def _report(err, bound, got, ref, what):
    ratio = err / bound
    i = np.unravel_index(int(np.argmax(ratio)), ratio.shape)
    assert np.all(err <= bound), (
        f"{what}: {int(np.count_nonzero(err > bound))} of {err.size} elements outside the "
        f"per-element bound; worst at {i}: got {got[i]:.6g}, ref {ref[i]:.6g}, "
        f"|diff| {err[i]:.3g} > bound {bound[i]:.3g}")
    return float(ratio.max())


def check_dense(got16: np.ndarray, ref: DenseRef, bias16=None, what="qmm") -> float:
    """Assert the per-element bound (and the 2e-2 metric) for bf16 outputs got16.

    bias16: the additive bias of qlinearBias, added by the kernel as
    bf16(bf16(acc) + bias): one more rounding of at most 2^-8 of the result."""
    got = f64(got16).reshape(ref.exact.shape)
    refs = [ref.exact, ref.fused]
    extra = 0.0
    mlx = ref.mlx
    if bias16 is not None:
        bv = f64(bias16)[None, :]
        extra = ROUND * np.maximum(np.abs(ref.exact), np.abs(ref.fused))
        refs = [r + bv for r in refs]
        if mlx is not None:
            mlx = _o.bf16_to_f32(_o.f32_to_bf16(mlx + bv.astype(np.float32)))
    d = [np.abs(got - r) for r in refs]
    pick = np.argmin(np.stack(d), axis=0)
    near = np.choose(pick, refs)
    err = np.minimum(d[0], d[1])
    bound = ROUND * np.maximum(np.abs(got), np.abs(near)) + ACCUM * ref.mag + extra + 1e-30
    worst = _report(err, bound, got, near, what)
    if mlx is not None:
        e = rel_err(got, mlx)
        assert e <= TOL, f"{what}: max-abs-rel {e:.3e} > {TOL} against the fp32 MLX-dequant oracle"
    return worst


class SwitchRef:
    """SwitchGLU oracle outputs [n_sel, k, D] under the kernel definitions (EXACT,
    and FUSED for batches that can reach the grouped GEMM), the MLX-definition
    output for the 2e-2 metric, and H = sqrt(sum_i (h_i wd_i)^2) per output."""

    def __init__(self, x, inds, gate, up, down, group=64, bits=4, token_sel=None,
                 fused=True):
        kw = dict(group_size=group, bits=bits, token_sel=token_sel)
        y, self.hscale = _o.switch_glu(x, inds, gate, up, down, mode=_o.DEQ_EXACT,
                                       want_hscale=True, **kw)
        self.refs = [f64(y)]
        if fused:
            self.refs.append(f64(_o.switch_glu(x, inds, gate, up, down, mode=_o.DEQ_FUSED,
                                               **kw)))
        self.mlx = f64(_o.switch_glu(x, inds, gate, up, down, mode=_o.DEQ_MLX, **kw))

    def masked(self, keep):
        out = SwitchRef.__new__(SwitchRef)
        out.refs = [r[keep] for r in self.refs]
        out.mlx, out.hscale = self.mlx[keep], self.hscale[keep]
        return out


def switch_bound(got, near, hscale):
    """Per-element allowance for a SwitchGLU output.

    Both sides are bf16, so they can be one ulp apart: 2^-7 of the value. On top
    of that, the intermediates g, u, silu(g) and h are each rounded to bf16 by
    both sides separately. Where the two fp32 values straddle a rounding point,
    h_i differs by about one ulp (2^-8..2^-7 of |h_i|, a little more after two
    roundings in a row). The effect on an output is sum_i dh_i wd_i, a random
    sum whose scale is 2^-7 H. The allowance is four times that, 2^-5 H, as if
    every channel had flipped."""
    return (2.0 * ROUND * np.maximum(np.abs(got), np.abs(near)) + 2.0 ** -5 * hscale
            + 1e-30)


def nearest(got16, sref: SwitchRef) -> np.ndarray:
    """Per slot (last axis D), the reference (kernel definition) the slot is nearest to."""
    got = f64(got16).reshape(sref.refs[0].shape)
    score = np.stack([(np.abs(got - r) / switch_bound(got, r, sref.hscale)).max(axis=-1)
                      for r in sref.refs])
    return np.choose(np.argmin(score, axis=0)[..., None], sref.refs)


def check_switch(got16, sref: SwitchRef, what="switch_glu") -> float:
    """Per-element bound on SwitchGLU outputs against the nearest kernel definition,
    whole slots at a time (one kernel family computes a slot), plus the 2e-2
    metric against the MLX-dequant oracle."""
    got = f64(got16).reshape(sref.refs[0].shape)
    near = nearest(got16, sref)
    worst = _report(np.abs(got - near), switch_bound(got, near, sref.hscale), got, near, what)
    e = rel_err(got, sref.mlx)
    assert e <= TOL, f"{what}: max-abs-rel {e:.3e} > {TOL} against the MLX-dequant oracle"
    return worst


def combine_check(got16, ys_near, ys_allow, w16, shared=None, what="moe combine"):
    """y = bf16(sum_k bf16(w_k * e_k)) [+ shared, rounded]: per-element bound
    against the combine of the oracle's expert outputs ys_near [T, k, D] (float64
    of bf16 values), whose own allowance ys_allow is carried through the weights.
    shared: (values, allowance) of the shared-expert row, or None."""
    got = f64(got16)
    wf = f64(w16)[:, :, None]
    prod = wf * ys_near
    comb = prod.sum(1)
    allow = (np.abs(wf) * ys_allow).sum(1)
    allow += ROUND * (np.abs(prod).sum(1) + 2.0 * np.abs(comb))
    if shared is not None:
        sv, sa = shared
        comb = comb + sv
        allow += sa + ROUND * np.abs(comb)
    allow += ROUND * np.abs(got) + 1e-30
    return _report(np.abs(got - comb), allow, got, comb, what)
