"""GPU parity: the SwitchGLU MoE expert MLP and the top-k combine vs the oracle.

Shapes mirror the reference's own SwitchGLU tests (compute/models/switch_glu_test.go:
5 experts, d=64, h=128, group 64 int4 for the unsorted branch with 2x3 slots; 8
experts with 32x2 = 64 slots for the sorted branch) and BASELINE configs 3 and 4.
"""
import numpy as np
import pytest
import torch

import parity
from gpu_util import announce, to_dev, to_np
from synth import make_quant, make_x, topk_uniform, topk_zipf

pytestmark = pytest.mark.gpu


def _stack(rng, E, D, I, bits=4, group=64):
    return (make_quant(rng, (E, I), D, bits, group), make_quant(rng, (E, I), D, bits, group),
            make_quant(rng, (E, D), I, bits, group))


def _check(got, x, inds, gate, up, down, bits=4, token_sel=None, keep=None, what="switch_glu"):
    """Per-element bound and 2e-2 metric of SwitchGLU outputs against the oracle
    (tests/parity.py).  keep: a [T, k] mask of the slots to compare."""
    T, k = inds.shape
    sref = parity.SwitchRef(x, inds, gate, up, down, 64, bits, token_sel=token_sel,
                            fused=T * k >= 4096)
    if keep is not None:
        got, sref = got[keep], sref.masked(keep)
    return parity.check_switch(got, sref, what=what)


def _run(gpu, x, inds, gate, up, down, group=64, bits=4):
    from fastmlx_amd import ops

    dev = lambda t: to_dev(t, gpu)
    out = ops.switch_glu(dev(x), dev(inds.astype(np.uint32)), tuple(map(dev, gate)),
                         tuple(map(dev, up)), tuple(map(dev, down)), group, bits)
    torch.cuda.synchronize()
    return to_np(out)


@pytest.mark.parametrize("E,T,k,D,I,bits", [(5, 2, 3, 64, 128, 4), (8, 32, 2, 64, 128, 4),
                                            (5, 2, 3, 64, 128, 8), (8, 40, 2, 128, 64, 8)])
def test_switch_glu_reference_shapes(gpu, oracle, E, T, k, D, I, bits):
    rng = np.random.default_rng(E * 100 + T + bits)
    gate, up, down = _stack(rng, E, D, I, bits)
    x = make_x(rng, T, D)
    inds = topk_uniform(rng, T, E, k)
    announce(f"switch_glu E={E} T={T} k={k} slots={T * k} bits={bits}")
    got = _run(gpu, x, inds, gate, up, down, bits=bits)
    assert got.shape == (T, k, D)
    _check(got, x, inds, gate, up, down, bits=bits)


def test_sorted_and_unsorted_branches_agree(gpu, oracle):
    """63 slots take the per-slot branch, 64 the sorted one; the same tokens give
    the same rows (switch_glu.go:28-30) up to bf16 rounding."""
    rng = np.random.default_rng(11)
    E, D, I, k = 8, 128, 64, 1
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, 64, D)
    inds = topk_uniform(rng, 64, E, k)
    announce("switch_glu 63 vs 64 slots")
    a = _run(gpu, x[:63].copy(), inds[:63].copy(), gate, up, down)
    b = _run(gpu, x, inds, gate, up, down)
    fa = oracle.bf16_to_f32(a).astype(np.float64)
    fb = oracle.bf16_to_f32(b[:63]).astype(np.float64)
    assert np.max(np.abs(fa - fb) / (np.abs(fb) * 2.0 ** -6 + 1e-3)) <= 1.0
    _check(b, x, inds, gate, up, down)


def test_switch_glu_bad_expert_id(gpu, oracle):
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(12)
    E, D, I = 4, 64, 64
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, 40, D)
    inds = topk_uniform(rng, 40, E, 2)
    inds[7, 1] = 99
    announce("switch_glu out-of-range id")
    got = _run(gpu, x, inds, gate, up, down)
    assert np.all(got[7, 1] == 0)
    with pytest.raises(FmxqError):
        ops.device_error()
    keep = np.ones((40, 2), dtype=bool)
    keep[7, 1] = False
    _check(got, x, np.where(inds >= E, 0, inds), gate, up, down, keep=keep)


def test_bad_expert_id_reported_after_graph_replay(gpu, oracle):
    """An out-of-range id in work captured into a graph raises the device's graph
    flag, which fmxq_device_error reads from any stream: the replay stream is not
    the capture stream.  Eager launches keep their stream's own flag, which other
    streams' queries neither see nor clear."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(13)
    E, D, I = 4, 64, 64
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, 8, D)
    inds = topk_uniform(rng, 8, E, 2)
    inds[3, 0] = 77
    dev = lambda t: to_dev(t, gpu)
    dx, di = dev(x), dev(inds.astype(np.uint32))
    stacks = [tuple(map(dev, m)) for m in (gate, up, down)]
    out = torch.empty(8, 2, D, dtype=torch.bfloat16, device=gpu)
    side, other = torch.cuda.Stream(), torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    announce("switch_glu bad id: eager on a side stream, then graph replay on others")
    with torch.cuda.stream(side):
        ops.switch_glu(dx, di, *stacks, 64, 4, out=out)  # warms the side stream's scratch
    torch.cuda.synchronize()
    ops.device_error()  # the default stream's own flag: not raised by the side stream
    with torch.cuda.stream(side), pytest.raises(FmxqError):
        ops.device_error()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        ops.switch_glu(dx, di, *stacks, 64, 4, out=out)
    with torch.cuda.stream(side):
        ops.device_error()  # capture ran nothing
    eager = to_np(out).copy()
    for q in (None, other):
        out.zero_()
        g.replay()  # on the default stream
        torch.cuda.synchronize()
        assert np.array_equal(to_np(out), eager)
        if q is None:
            with pytest.raises(FmxqError):
                ops.device_error()
        else:
            with torch.cuda.stream(q), pytest.raises(FmxqError):
                ops.device_error()
        ops.device_error()  # cleared by the report
    assert np.all(eager[3, 0] == 0)


_LAYER_CACHE = {}


def _layer_weights(gpu, cfg):
    """Config 3 / 4 expert stacks (and config 4's shared expert), generated once per
    session on the host and on the device: 0.9 GB and 6.4 GB of packed weights."""
    if cfg not in _LAYER_CACHE:
        _LAYER_CACHE.clear()  # hold one configuration at a time
        rng = np.random.default_rng(880 if cfg == "c3" else 881)
        E, D, I = (512, 2048, 512) if cfg == "c3" else (256, 7168, 2048)
        host = _stack(rng, E, D, I)
        shared = _stack(rng, 1, D, I) if cfg == "c4" else None
        dev = lambda q: tuple(to_dev(t, gpu) for t in q)
        _LAYER_CACHE[cfg] = (host, tuple(dev(q) for q in host), shared,
                             None if shared is None else tuple(dev(q) for q in shared))
    return _LAYER_CACHE[cfg]


@pytest.mark.parametrize("cfg,M", [("c3", 1), ("c3", 16), ("c3", 128), ("c3", 512),
                                   ("c4", 1), ("c4", 32), ("c4", 256)])
def test_moe_layer_configs(gpu, oracle, cfg, M):
    """BASELINE configs 3 and 4 at every token count the bench times: SwitchGLU,
    the weighted top-k combine and, for config 4, the shared expert MLP computed by
    the library (a one-expert SwitchGLU, deepseekv3_forward.go:438-440) and added
    with weight 1.  A sample of tokens is checked element by element: the expert
    outputs, the shared expert and the combined row."""
    from fastmlx_amd import ops

    (gate, up, down), dstack, shared, dshared = _layer_weights(gpu, cfg)
    rng = np.random.default_rng(800 + M)
    E, I, D = gate[0].shape[0], gate[0].shape[1], down[0].shape[1]
    if cfg == "c3":
        k = 10
        inds = topk_uniform(rng, M, E, k)
        logits = rng.standard_normal((M, k)).astype(np.float32)
        wts = np.exp(logits - logits.max(1, keepdims=True))
        wts = wts / wts.sum(1, keepdims=True)
    else:
        k = 8
        inds = topk_zipf(rng, M, E, k)
        g = 1 / (1 + np.exp(-rng.standard_normal((M, k))))
        wts = (g / g.sum(1, keepdims=True)).astype(np.float32)
    x = make_x(rng, M, D)
    w16 = oracle.f32_to_bf16(wts.astype(np.float32))
    dx = to_dev(x, gpu)
    announce(f"moe layer {cfg} M={M} slots={M * k}")
    y = ops.switch_glu(dx, to_dev(inds.astype(np.uint32), gpu), *dstack, 64, 4)
    ysh = None
    if dshared is not None:
        zero = torch.zeros(M, 1, dtype=torch.int32, device=gpu)
        ysh = ops.switch_glu(dx, zero, *dshared, 64, 4)
    out = ops.moe_combine(y, to_dev(w16, gpu), None if ysh is None else ysh.view(M, D))
    torch.cuda.synchronize()
    got_y, got = to_np(y), to_np(out)
    sel = np.unique(np.concatenate([[0, M - 1], rng.choice(M, size=min(M, 3), replace=False)]))
    fused = M * k >= 4096
    sref = parity.SwitchRef(x, inds, gate, up, down, token_sel=sel, fused=fused)
    parity.check_switch(got_y[sel], sref, what=f"{cfg} M={M} experts")
    near = parity.nearest(got_y[sel], sref)
    sh = None
    if shared is not None:
        zi = np.zeros((M, 1), dtype=np.int32)
        ssref = parity.SwitchRef(x, zi, *shared, token_sel=sel, fused=False)
        parity.check_switch(to_np(ysh)[sel], ssref, what=f"{cfg} M={M} shared expert")
        snear = parity.nearest(to_np(ysh)[sel], ssref)
        sh = (snear[:, 0], parity.switch_bound(snear, snear, ssref.hscale)[:, 0])
    parity.combine_check(got[sel], near, parity.switch_bound(near, near, sref.hscale),
                         w16[sel], shared=sh, what=f"{cfg} M={M} combined")


def test_moe_combine_op_chain(gpu, oracle):
    """Combine against the numpy op chain, with and without the gated shared expert."""
    from fastmlx_amd import ops

    rng = np.random.default_rng(13)
    T, k, D = 7, 4, 96
    y = make_x(rng, T, k, D)
    w = oracle.f32_to_bf16(rng.uniform(0, 1, (T, k)).astype(np.float32))
    sh = make_x(rng, T, D)
    sg = make_x(rng, T)
    r16 = lambda v: oracle.bf16_to_f32(oracle.f32_to_bf16(v.astype(np.float32)))
    base = r16((r16(oracle.bf16_to_f32(y) * oracle.bf16_to_f32(w)[:, :, None])).sum(1))
    dev = lambda t: to_dev(t, gpu)
    announce("moe_combine")
    plain = to_np(ops.moe_combine(dev(y), dev(w)))
    gated = to_np(ops.moe_combine(dev(y), dev(w), dev(sh), dev(sg)))
    torch.cuda.synchronize()
    sig = r16(1 / (1 + np.exp(-oracle.bf16_to_f32(sg).astype(np.float64))))
    want_g = r16(base + r16(sig[:, None] * oracle.bf16_to_f32(sh)))
    # element by element: at most one bf16 ulp apart (a sum order or an exp that
    # lands on the other side of a rounding point)
    for got, want in ((plain, base), (gated, want_g)):
        g = oracle.bf16_to_f32(got).astype(np.float64)
        assert np.all(np.abs(g - want) <= 2.0 ** -7 * np.abs(want) + 1e-30)


# --- the segmented grouped product (int4 group 64, D and I multiples of 256) ---

@pytest.mark.parametrize("E,T,k", [
    (64, 5, 4),     # 20 slots over 64 experts: 16-slot windows, mostly one slot per segment
    (4, 40, 2),     # 80 slots over 4 experts: 32-slot windows, runs of several pieces
    (1, 37, 1),     # one expert: every segment a full window but the last
    (16, 64, 3),    # 192 slots, uniform
])
def test_switch_glu_segments(gpu, oracle, E, T, k):
    """Sorted slots cut into expert segments, gate and up fused with silu * up, down
    stored to each slot's own row: every slot equals the oracle's SwitchGLU row."""
    rng = np.random.default_rng(E * 31 + T * 7 + k)
    D, I = 256, 512
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, T, D)
    inds = topk_uniform(rng, T, E, k)
    announce(f"switch_glu segments E={E} T={T} k={k}")
    got = _run(gpu, x, inds, gate, up, down)
    _check(got, x, inds, gate, up, down)


def test_switch_glu_segments_hot_expert(gpu, oracle):
    """Zipf routing: one expert takes a large share of the slots (runs of many
    windows) while most experts get one or two."""
    from synth import topk_zipf

    rng = np.random.default_rng(77)
    E, T, k, D, I = 32, 96, 4, 512, 256
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, T, D)
    inds = topk_zipf(rng, T, E, k)
    announce("switch_glu segments zipf")
    got = _run(gpu, x, inds, gate, up, down)
    _check(got, x, inds, gate, up, down)


def test_switch_glu_segments_bad_expert_id(gpu, oracle):
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(13)
    E, D, I = 6, 256, 256
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, 30, D)
    inds = topk_uniform(rng, 30, E, 2)
    inds[3, 0] = 6
    inds[20, 1] = 1000
    announce("switch_glu segments out-of-range ids")
    got = _run(gpu, x, inds, gate, up, down)
    assert np.all(got[3, 0] == 0) and np.all(got[20, 1] == 0)
    with pytest.raises(FmxqError):
        ops.device_error()
    # every good slot, the good slot of each bad token included, matches the oracle
    keep = np.ones((30, 2), dtype=bool)
    keep[3, 0] = keep[20, 1] = False
    _check(got, x, np.where(inds >= E, 0, inds), gate, up, down, keep=keep)


def test_gather_qmm_segments_unsorted_lhs_and_bad_rows(gpu, oracle):
    """gather_qmm with one x row per item takes the sorted segment path whatever the
    order of rhs: explicit lhs, unsorted ids, a bad id and a bad x row (both give a
    zero row and a device error)."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(23)
    E, N, K, xb = 7, 200, 768, 11
    w, s, b = make_quant(rng, (E, N), K, 4, 64)
    x = make_x(rng, xb, 1, K)
    S = 90
    rhs = rng.integers(0, E, size=S).astype(np.uint32)
    lhs = rng.integers(0, xb, size=S).astype(np.uint32)
    rhs[17] = 9
    lhs[40] = xb + 3
    announce("gather_qmm segments, unsorted, lhs, bad id and row")
    y = ops.gather_qmm(to_dev(x, gpu), to_dev(w, gpu), to_dev(s, gpu), to_dev(b, gpu),
                       to_dev(rhs, gpu), to_dev(lhs, gpu), 1, True, 64, 4, False)
    torch.cuda.synchronize()
    got = to_np(y).reshape(S, N)
    bad = np.zeros(S, dtype=bool)
    bad[[17, 40]] = True
    assert np.all(got[bad] == 0)
    with pytest.raises(FmxqError):
        ops.device_error()
    ref = parity.gather_refs(x.reshape(xb, K), w, s, b, lhs[~bad].astype(np.int32),
                             rhs[~bad].astype(np.int32))
    parity.check_dense(got[~bad], ref, what="gather_qmm")


# --- few slots: no sort, every slot its own segment ---

@pytest.mark.parametrize("E,T,k,D,I", [
    (64, 1, 10, 256, 512),    # one decode token (configuration 3's top-10), MFMA walk
    (8, 2, 8, 256, 512),      # 16 slots, every expert twice
    (3, 5, 3, 256, 512),      # 15 slots over 3 experts: repeated experts in slot order
    (5, 17, 1, 256, 512),     # 17 slots: the sorted path, just past the limit
    (12, 1, 8, 2048, 2304),   # GEMV form: gate/up one 2048-deep slice, down two slices
    (6, 2, 3, 4608, 2048),    # GEMV form: gate/up four slices of 36 chunks
])
def test_switch_glu_few_slots(gpu, oracle, E, T, k, D, I):
    rng = np.random.default_rng(E * 13 + T * 5 + k)
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, T, D)
    inds = topk_uniform(rng, T, E, k)
    announce(f"switch_glu few slots E={E} T={T} k={k}")
    got = _run(gpu, x, inds, gate, up, down)
    _check(got, x, inds, gate, up, down)


def test_switch_glu_few_slots_bad_expert_id(gpu, oracle):
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(29)
    E, D, I, T, k = 9, 256, 256, 2, 4
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, T, D)
    inds = topk_uniform(rng, T, E, k)
    inds[1, 2] = 77
    announce("switch_glu few slots, out-of-range id")
    got = _run(gpu, x, inds, gate, up, down)
    assert np.all(got[1, 2] == 0)
    with pytest.raises(FmxqError):
        ops.device_error()
    keep = np.ones((T, k), dtype=bool)
    keep[1, 2] = False
    _check(got, x, np.where(inds >= E, 0, inds), gate, up, down, keep=keep)


@pytest.mark.parametrize("with_lhs,K", [(True, 512), (False, 512), (True, 4096), (False, 6144)])
def test_gather_qmm_few_items(gpu, oracle, with_lhs, K):
    """Up to 16 items: one segment per item in item order, with explicit lhs (one bad
    row) or the implicit item // lhs_div rows, and one bad expert id; K of 512 (MFMA
    walk) and of 4096 / 6144 (GEMV form with two and four K slices)."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(31 + with_lhs + K)
    E, N, xb, S = 6, 300, 5, 12
    w, s, b = make_quant(rng, (E, N), K, 4, 64)
    x = make_x(rng, xb, 1, K)
    rhs = rng.integers(0, E, size=S).astype(np.uint32)
    rhs[4] = 40
    if with_lhs:
        lhs = rng.integers(0, xb, size=S).astype(np.uint32)
        lhs[9] = xb
        lhs_div = 1
    else:
        lhs = None
        lhs_div = 3  # items 0..11 read rows 0..3
    announce(f"gather_qmm few items lhs={with_lhs} K={K}")
    y = ops.gather_qmm(to_dev(x, gpu), to_dev(w, gpu), to_dev(s, gpu), to_dev(b, gpu),
                       to_dev(rhs, gpu), None if lhs is None else to_dev(lhs, gpu), lhs_div,
                       True, 64, 4, False)
    torch.cuda.synchronize()
    got = to_np(y).reshape(S, N)
    bad = np.zeros(S, dtype=bool)
    bad[4] = True
    if with_lhs:
        bad[9] = True
    assert np.all(got[bad] == 0)
    with pytest.raises(FmxqError):
        ops.device_error()
    rows = lhs if with_lhs else (np.arange(S) // lhs_div).astype(np.uint32)
    ref = parity.gather_refs(x.reshape(xb, K), w, s, b, rows[~bad].astype(np.int32),
                             rhs[~bad].astype(np.int32))
    parity.check_dense(got[~bad], ref, what="gather_qmm")


def test_switch_glu_segments_short_and_long(gpu, oracle):
    """Sorted slots with K >= 2048: one-slot segments take the GEMV form, longer
    ones the MFMA walk; Zipf routing gives both, plus one out-of-range id."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(41)
    E, T, k, D, I = 24, 40, 4, 2048, 2304
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, T, D)
    inds = topk_zipf(rng, T, E, k)
    inds[7, 1] = E + 5
    counts = np.bincount(inds[inds < E].ravel(), minlength=E)
    assert counts.max() > 4 and ((counts > 0) & (counts <= 4)).any()
    announce("switch_glu segments, short and long, K >= 2048")
    got = _run(gpu, x, inds, gate, up, down)
    assert np.all(got[7, 1] == 0)
    with pytest.raises(FmxqError):
        ops.device_error()
    keep = np.ones((T, k), dtype=bool)
    keep[7, 1] = False
    _check(got, x, np.where(inds >= E, 0, inds), gate, up, down, keep=keep)


def test_gather_qmm_segments_short_and_long(gpu, oracle):
    """gather_qmm over 70 items, K = 4096: runs of one item (GEMV form) and of 2 to
    20 (MFMA walk), explicit lhs with a bad row, one bad id."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(43)
    E, N, K, xb = 10, 260, 4096, 9
    w, s, b = make_quant(rng, (E, N), K, 4, 64)
    x = make_x(rng, xb, 1, K)
    lens = [20, 1, 2, 3, 4, 5, 1, 14, 2, 18]
    rhs = np.concatenate([np.full(n, e, dtype=np.uint32) for e, n in enumerate(lens)])
    rng.shuffle(rhs)
    S = rhs.size
    lhs = rng.integers(0, xb, size=S).astype(np.uint32)
    rhs[11] = E
    lhs[50] = xb + 1
    announce("gather_qmm segments, short and long, K = 4096")
    y = ops.gather_qmm(to_dev(x, gpu), to_dev(w, gpu), to_dev(s, gpu), to_dev(b, gpu),
                       to_dev(rhs, gpu), to_dev(lhs, gpu), 1, True, 64, 4, False)
    torch.cuda.synchronize()
    got = to_np(y).reshape(S, N)
    bad = np.zeros(S, dtype=bool)
    bad[[11, 50]] = True
    assert np.all(got[bad] == 0)
    with pytest.raises(FmxqError):
        ops.device_error()
    ref = parity.gather_refs(x.reshape(xb, K), w, s, b, lhs[~bad].astype(np.int32),
                             rhs[~bad].astype(np.int32))
    parity.check_dense(got[~bad], ref, what="gather_qmm")


@pytest.mark.parametrize("E,lens,K", [
    # 600 slots over 8 experts (32-slot windows): runs of 1, odd lengths, runs one
    # slot short of or past a piece (31, 33), pieces of 17 to 32 slots (the walk that
    # dequantizes the weights) and of 1 to 16; grid 32 column tiles x 28 segments
    (8, [1, 3, 17, 31, 33, 64, 151, 300], 1024),
    # 232 slots over 64 experts (16-slot windows), runs of 1 to 6; grid 16 x 80
    (64, None, 1024),
    # one and three 256-value steps: the odd last step after the loop, and pipeline
    # loads past the end from the first step on
    (8, [1, 3, 17, 31, 33, 64, 151, 300], 256),
    (64, None, 768),
])
def test_gather_qmm_shared_x_walk(gpu, oracle, E, lens, K):
    """gather_qmm on grids of more than 512 blocks, where the MFMA walk shares each
    segment's x rows through LDS and DMAs only the rows inside the segment; K below
    2048, so every segment, one-slot ones included, takes the walk.  Explicit lhs
    with a bad x row and one bad expert id."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(59 + E)
    N, xb = 2048, 50
    w, s, b = make_quant(rng, (E, N), K, 4, 64)
    x = make_x(rng, xb, 1, K)
    if lens is None:
        lens = [int(v) for v in rng.integers(1, 7, size=E)]
    rhs = np.concatenate([np.full(n, e, dtype=np.uint32) for e, n in enumerate(lens)])
    rng.shuffle(rhs)
    S = rhs.size
    lhs = rng.integers(0, xb, size=S).astype(np.uint32)
    rhs[5] = E
    lhs[S // 2] = xb + 3
    announce(f"gather_qmm shared-x walk E={E} slots={S} K={K}")
    y = ops.gather_qmm(to_dev(x, gpu), to_dev(w, gpu), to_dev(s, gpu), to_dev(b, gpu),
                       to_dev(rhs, gpu), to_dev(lhs, gpu), 1, True, 64, 4, False)
    torch.cuda.synchronize()
    got = to_np(y).reshape(S, N)
    bad = np.zeros(S, dtype=bool)
    bad[[5, S // 2]] = True
    assert np.all(got[bad] == 0)
    with pytest.raises(FmxqError):
        ops.device_error()
    ref = parity.gather_refs(x.reshape(xb, K), w, s, b, lhs[~bad].astype(np.int32),
                             rhs[~bad].astype(np.int32))
    parity.check_dense(got[~bad], ref, what="gather_qmm")


def test_switch_glu_many_slots_per_expert_long_rows(gpu, oracle):
    """More than 8 slots per expert on average with K >= 2048: the MFMA walk alone."""
    rng = np.random.default_rng(47)
    E, T, k, D, I = 4, 40, 2, 2048, 2048
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, T, D)
    inds = topk_uniform(rng, T, E, k)
    announce("switch_glu 80 slots over 4 experts, K = 2048")
    got = _run(gpu, x, inds, gate, up, down)
    _check(got, x, inds, gate, up, down)


# --- long expert runs (>= 256 slots, batches of >= 4096 slots): the grouped GEMM ---

@pytest.mark.parametrize("E,T,k,D,I", [
    (2, 2100, 2, 256, 256),    # two runs of 2100 slots: 16 full tiles and a partial each
    (3, 2100, 2, 256, 512),    # three runs of ~1400
    (24, 1024, 4, 256, 256),   # Zipf: runs of 838 .. 281 grouped, 239 and below on the walk
    (2, 8200, 2, 256, 256),    # 16400 slots: more than the sort's LDS staging holds
])
def test_switch_glu_long_runs(gpu, oracle, E, T, k, D, I):
    rng = np.random.default_rng(E * 7 + T + k + D)
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, T, D)
    inds = topk_zipf(rng, T, E, k) if E >= 20 else topk_uniform(rng, T, E, k)
    counts = np.bincount(inds.ravel(), minlength=E)
    assert counts.max() >= 256 and T * k >= 4096
    announce(f"switch_glu long runs E={E} T={T} k={k} D={D} I={I} max run {counts.max()}")
    got = _run(gpu, x, inds, gate, up, down)
    _check(got, x, inds, gate, up, down)


def test_gather_qmm_long_runs_bad_row_and_id(gpu, oracle):
    """gather_qmm over 4096 items in runs of 2000, 1500, 300, 255 and 41 (three
    grouped-GEMM runs; 255 just below the threshold), N not a multiple of the
    256-column tile, a bad x row inside a long run and a bad expert id."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(53)
    E, N, K, xb = 5, 300, 512, 37
    w, s, b = make_quant(rng, (E, N), K, 4, 64)
    x = make_x(rng, xb, 1, K)
    lens = [2000, 1500, 300, 255, 41]
    rhs = np.concatenate([np.full(n, e, dtype=np.uint32) for e, n in enumerate(lens)])
    rng.shuffle(rhs)
    S = rhs.size
    lhs = rng.integers(0, xb, size=S).astype(np.uint32)
    i_bad_row = int(np.nonzero(rhs == 0)[0][17])
    lhs[i_bad_row] = xb + 4
    i_bad_id = int(np.nonzero(rhs == 4)[0][0])
    rhs[i_bad_id] = 11
    announce("gather_qmm long runs with bad row and id")
    y = ops.gather_qmm(to_dev(x, gpu), to_dev(w, gpu), to_dev(s, gpu), to_dev(b, gpu),
                       to_dev(rhs, gpu), to_dev(lhs, gpu), 1, True, 64, 4, False)
    torch.cuda.synchronize()
    got = to_np(y).reshape(S, N)
    bad = np.zeros(S, dtype=bool)
    bad[[i_bad_row, i_bad_id]] = True
    assert np.all(got[bad] == 0)
    with pytest.raises(FmxqError):
        ops.device_error()
    ref = parity.gather_refs(x.reshape(xb, K), w, s, b, lhs[~bad].astype(np.int32),
                             rhs[~bad].astype(np.int32))
    parity.check_dense(got[~bad], ref, what="gather_qmm")


# --- switch_glu_combine: one MoE layer's routed part in one call ---

@pytest.mark.parametrize("cfg,M", [("c3", 1), ("c3", 16), ("c3", 128), ("c3", 512), ("c4", 1),
                                   ("c4", 2), ("c4", 32)])
def test_switch_glu_combine_configs(gpu, oracle, cfg, M):
    """The fused layer at configurations 3 and 4, at every configuration 3 token
    count the bench times (qwen3next_forward.go:519-520).
    - Up to 16 slots, and up to 256 slots over at least twice as many experts
      (configuration 3 at M=16), run unsorted, the down projection and the
      weighted sum as one kernel.
    - Other batches run the sorted SwitchGLU, then the combine.
    - Configuration 4 adds its shared expert (computed by a one-expert SwitchGLU).
    Checked element by element against the oracle's op chain."""
    from fastmlx_amd import ops

    (gate, up, down), dstack, shared, dshared = _layer_weights(gpu, cfg)
    rng = np.random.default_rng(900 + M)
    E, D = gate[0].shape[0], down[0].shape[1]
    if cfg == "c3":
        k = 10
        inds = topk_uniform(rng, M, E, k)
        wts = rng.dirichlet(np.ones(k), size=M).astype(np.float32)
    else:
        k = 8
        inds = topk_zipf(rng, M, E, k)
        g = 1 / (1 + np.exp(-rng.standard_normal((M, k))))
        wts = (g / g.sum(1, keepdims=True)).astype(np.float32)
    x = make_x(rng, M, D)
    w16 = oracle.f32_to_bf16(wts)
    dx = to_dev(x, gpu)
    announce(f"switch_glu_combine {cfg} M={M} slots={M * k}")
    ysh = None
    if dshared is not None:
        ysh = ops.switch_glu(dx, torch.zeros(M, 1, dtype=torch.int32, device=gpu), *dshared, 64, 4)
    out = ops.switch_glu_combine(dx, to_dev(inds.astype(np.uint32), gpu), *dstack, to_dev(w16, gpu),
                                 None if ysh is None else ysh.view(M, D))
    torch.cuda.synchronize()
    got = to_np(out)
    sel = np.unique(np.concatenate([[0, M - 1], rng.choice(M, size=min(M, 3), replace=False)]))
    # From 4096 slots the sorted SwitchGLU can take the grouped GEMM (single-rounding
    # dequant): the combined rows must then match the combine of either definition.
    sref = parity.SwitchRef(x, inds, gate, up, down, token_sel=sel, fused=M * k >= 4096)
    sh = None
    if shared is not None:
        zi = np.zeros((M, 1), dtype=np.int32)
        ssref = parity.SwitchRef(x, zi, *shared, token_sel=sel, fused=False)
        parity.check_switch(to_np(ysh)[sel], ssref, what="shared expert")
        snear = parity.nearest(to_np(ysh)[sel], ssref)
        sh = (snear[:, 0], parity.switch_bound(snear, snear, ssref.hscale)[:, 0])
    errors = []
    for near in sref.refs:
        try:
            parity.combine_check(got[sel], near, parity.switch_bound(near, near, sref.hscale),
                                 w16[sel], shared=sh, what=f"switch_glu_combine {cfg} M={M}")
            break
        except AssertionError as e:
            errors.append(str(e))
    else:
        raise AssertionError(" | ".join(errors))


@pytest.mark.parametrize("I,gated,E,T,k", [(512, True, 9, 2, 6), (1024, False, 9, 2, 6),
                                           (4096, True, 9, 2, 6), (8192, False, 9, 2, 6),
                                           (512, True, 300, 12, 10)])
def test_switch_glu_combine_few_slots_shapes(gpu, oracle, I, gated, E, T, k):
    """The fused down/combine kernel's other row forms (32 lanes per 1024-value row,
    two and four chunks per lane at 4096 and 8192), a sigmoid-gated shared term, a bad expert id
    (its slot contributes zero and the flag is raised), and 120 slots over 300
    experts (unsorted beyond 16 slots)."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(I + gated + E)
    D = 512
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, T, D)
    inds = topk_uniform(rng, T, E, k)
    inds[1, 4] = E + 3
    wts = oracle.f32_to_bf16(rng.dirichlet(np.ones(k), size=T).astype(np.float32))
    sh = make_x(rng, T, D)
    sg = make_x(rng, T) if gated else None
    dev = lambda t: to_dev(t, gpu)
    announce(f"switch_glu_combine I={I} gated={gated} E={E} slots={T * k}")
    out = ops.switch_glu_combine(dev(x), dev(inds.astype(np.uint32)), tuple(map(dev, gate)),
                                 tuple(map(dev, up)), tuple(map(dev, down)), dev(wts), dev(sh),
                                 None if sg is None else dev(sg))
    torch.cuda.synchronize()
    got = to_np(out)
    with pytest.raises(FmxqError):
        ops.device_error()
    safe = np.where(inds >= E, 0, inds)
    sref = parity.SwitchRef(x, safe, gate, up, down, fused=False)
    near = sref.refs[0].copy()
    near[1, 4] = 0.0  # the bad slot's row is zero
    allow = parity.switch_bound(near, near, sref.hscale)
    allow[1, 4] = 0.0
    shv = oracle.bf16_to_f32(sh).astype(np.float64)
    if gated:
        r16 = lambda v: oracle.bf16_to_f32(oracle.f32_to_bf16(np.asarray(v, np.float32))).astype(np.float64)
        gt = r16(1 / (1 + np.exp(-oracle.bf16_to_f32(sg).astype(np.float64))))
        shv = r16(gt[:, None] * shv)
    parity.combine_check(got, near, allow, wts, shared=(shv, 2.0 ** -8 * np.abs(shv)),
                         what=f"switch_glu_combine I={I}")


# --- the one-token layer (gate/up, then down with the combine) ---

def _combine_ref_check(oracle, got, x, inds, gate, up, down, wts, E, sh=None, sg=None,
                       what="one-token layer"):
    """got [1, D] against the oracle's routed experts (bad ids contribute zero) plus
    an optional precomputed shared row sh (gated by sigmoid(sg))."""
    safe = np.where(inds >= E, 0, inds)
    sref = parity.SwitchRef(x, safe, gate, up, down, fused=False)
    near = sref.refs[0].copy()
    allow = parity.switch_bound(near, near, sref.hscale)
    bad = inds >= E
    near[bad] = 0.0
    allow[bad] = 0.0
    shared = None
    if sh is not None:
        shv = oracle.bf16_to_f32(sh).astype(np.float64)
        if sg is not None:
            r16 = lambda v: oracle.bf16_to_f32(oracle.f32_to_bf16(np.asarray(v, np.float32))).astype(np.float64)
            gt = r16(1 / (1 + np.exp(-oracle.bf16_to_f32(sg).astype(np.float64))))
            shv = r16(gt[:, None] * shv)
        shared = (shv, 2.0 ** -8 * np.abs(shv))
    parity.combine_check(got, near, allow, wts, shared=shared, what=what)


@pytest.mark.parametrize("I,D,E,k,gated,bad", [
    (512, 512, 9, 6, True, True),        # shallow rows: the segment walk
    (1024, 1024, 9, 6, False, False),    # 32 lanes per down row
    (2048, 4096, 12, 8, True, True),     # two chunks per lane on the gate/up rows
    (4096, 2048, 9, 6, False, True),     # two chunks per lane on the down rows
    (512, 7168, 20, 16, True, False),    # 16 slots, the most the unsorted path takes
    (512, 10240, 16, 16, False, True),   # every expert hit
])
def test_switch_glu_combine_one_token(gpu, oracle, I, D, E, k, gated, bad):
    """One token: the few-slot gate/up GEMV, then the down projection fused with the
    weighted top-k sum, at hidden sizes from 512 to 10240 (one to five chunks a lane
    on the gate/up rows), every down layout (16, 32 and 64 lanes per row, one or two
    chunks per lane), up to 16 slots, a gated or plain shared row and a bad expert
    id (its slot contributes zero, the flag is raised)."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(I + D + E + k)
    gate, up, down = _stack(rng, E, D, I)
    x = make_x(rng, 1, D)
    inds = topk_uniform(rng, 1, E, k)
    if bad:
        inds[0, k // 2] = E + 5
    wts = oracle.f32_to_bf16(rng.dirichlet(np.ones(k), size=1).astype(np.float32))
    sh = make_x(rng, 1, D)
    sg = make_x(rng, 1) if gated else None
    dev = lambda t: to_dev(t, gpu)
    announce(f"switch_glu_combine one token I={I} D={D} E={E} k={k} bad={bad}")
    out = ops.switch_glu_combine(dev(x), dev(inds.astype(np.uint32)), tuple(map(dev, gate)),
                                 tuple(map(dev, up)), tuple(map(dev, down)), dev(wts), dev(sh),
                                 None if sg is None else dev(sg))
    torch.cuda.synchronize()
    got = to_np(out)
    if bad:
        with pytest.raises(FmxqError):
            ops.device_error()
    else:
        ops.device_error()
    _combine_ref_check(oracle, got, x, inds, gate, up, down, wts, E, sh, sg,
                       what=f"one token I={I} D={D}")


def test_one_token_layer_back_to_back(gpu, oracle):
    """One-token layers in a row on one stream, with different slot counts and
    experts and no synchronization between them: each call's down/combine kernel
    must read its own call's h rows from the stream's scratch.  Every output is
    checked, and a second round of the same calls gives the same bits."""
    from fastmlx_amd import ops

    rng = np.random.default_rng(4242)
    E, D, I = 24, 2048, 512
    gate, up, down = _stack(rng, E, D, I)
    dev = lambda t: to_dev(t, gpu)
    dg, du, dd = tuple(map(dev, gate)), tuple(map(dev, up)), tuple(map(dev, down))
    calls = []
    for i, k in enumerate((10, 4, 16, 1, 10, 7)):
        x = make_x(rng, 1, D)
        inds = topk_uniform(rng, 1, E, k)
        wts = oracle.f32_to_bf16(rng.dirichlet(np.ones(k), size=1).astype(np.float32))
        calls.append((x, inds, wts, dev(x), dev(inds.astype(np.uint32)), dev(wts)))
    announce("one-token layer: six calls back to back")
    outs = [ops.switch_glu_combine(dx, di, dg, du, dd, dw) for _, _, _, dx, di, dw in calls]
    torch.cuda.synchronize()
    ops.device_error()
    for (x, inds, wts, *_), out in zip(calls, outs):
        _combine_ref_check(oracle, to_np(out), x, inds, gate, up, down, wts, E,
                           what=f"back-to-back k={inds.shape[1]}")
    # once more: the same calls repeated give the same bits
    again = [ops.switch_glu_combine(dx, di, dg, du, dd, dw) for _, _, _, dx, di, dw in calls]
    torch.cuda.synchronize()
    for a, b in zip(outs, again):
        assert np.array_equal(to_np(a), to_np(b))


# --- moe_layer: routed experts, weighted sum and the shared expert in one call ---

@pytest.mark.parametrize("M", [1, 3, 32, 256])
def test_moe_layer_shared_expert_c4(gpu, oracle, M):
    """Configuration 4 with its shared expert computed inside the call
    (deepseekv3_forward.go:436-440: routed sum + mlp(x)), up to M=256, the largest
    token count the bench times.  One token runs the
    shared expert as one more gate/up segment and one more down/combine wave; three
    tokens (24 slots, few sharing an expert) run it as a one-expert SwitchGLU first;
    sorted batches (32 and 256 tokens) sort it in as expert E, one slot per token,
    inside the routed launches.  Checked element by element against the oracle's
    routed experts and shared MLP."""
    from fastmlx_amd import ops

    (gate, up, down), dstack, shared, dshared = _layer_weights(gpu, "c4")
    rng = np.random.default_rng(950 + M)
    E, D = gate[0].shape[0], down[0].shape[1]
    k = 8
    inds = topk_zipf(rng, M, E, k)
    g = 1 / (1 + np.exp(-rng.standard_normal((M, k))))
    w16 = oracle.f32_to_bf16((g / g.sum(1, keepdims=True)).astype(np.float32))
    x = make_x(rng, M, D)
    announce(f"moe_layer c4 M={M} slots={M * k} + shared expert")
    out = ops.moe_layer(to_dev(x, gpu), to_dev(inds.astype(np.uint32), gpu), *dstack,
                        to_dev(w16, gpu), dshared)
    torch.cuda.synchronize()
    got = to_np(out)
    sel = np.unique(np.concatenate([[0, M - 1], rng.choice(M, size=min(M, 3), replace=False)]))
    sref = parity.SwitchRef(x, inds, gate, up, down, token_sel=sel, fused=False)
    near = sref.refs[0]
    zi = np.zeros((M, 1), dtype=np.int32)
    ssref = parity.SwitchRef(x, zi, *shared, token_sel=sel, fused=False)
    sv = ssref.refs[0]
    sa = parity.switch_bound(sv, sv, ssref.hscale)
    parity.combine_check(got[sel], near, parity.switch_bound(near, near, sref.hscale), w16[sel],
                         shared=(sv[:, 0], sa[:, 0]), what=f"moe_layer c4 M={M}")


@pytest.mark.parametrize("T,E,D,k", [(1, 300, 2048, 10), (2, 300, 2048, 10),
                                     (1, 64, 2048, 16), (1, 40, 512, 6),
                                     (24, 32, 2048, 6), (40, 16, 512, 4)])
def test_moe_layer_gated_shared_expert(gpu, oracle, T, E, D, k):
    """A Qwen3-Next-style layer (qwen3next_forward.go:519-524): the shared expert's
    output scaled by sigmoid(shared_gate) before it is added.  One token with up
    to 15 slots and D >= 2048 runs fused; two tokens, 16 slots (a block would need
    17 waves) and D = 512 (below the GEMV form's depth) run the one-expert
    SwitchGLU first; 24 and 40 tokens over few experts sort the shared expert in
    as expert E (16- and 32-slot segments; D = 512 walks its down projection with
    every load issued up front)."""
    from fastmlx_amd import ops

    rng = np.random.default_rng(960 + T + k + D)
    I = 512
    gate, up, down = _stack(rng, E, D, I)
    sh = _stack(rng, 1, D, I)
    x = make_x(rng, T, D)
    inds = topk_uniform(rng, T, E, k)
    w16 = oracle.f32_to_bf16(rng.dirichlet(np.ones(k), size=T).astype(np.float32))
    sg = make_x(rng, T)
    dev = lambda t: to_dev(t, gpu)
    announce(f"moe_layer gated shared T={T} E={E} D={D} k={k}")
    out = ops.moe_layer(dev(x), dev(inds.astype(np.uint32)), tuple(map(dev, gate)),
                        tuple(map(dev, up)), tuple(map(dev, down)), dev(w16),
                        tuple(tuple(map(dev, q)) for q in sh), dev(sg))
    torch.cuda.synchronize()
    got = to_np(out)
    sref = parity.SwitchRef(x, inds, gate, up, down, fused=False)
    near = sref.refs[0]
    ssref = parity.SwitchRef(x, np.zeros((T, 1), dtype=np.int32), *sh, fused=False)
    sv = ssref.refs[0][:, 0]
    sa = parity.switch_bound(ssref.refs[0], ssref.refs[0], ssref.hscale)[:, 0]
    r16 = lambda v: oracle.bf16_to_f32(oracle.f32_to_bf16(np.asarray(v, np.float32))).astype(np.float64)
    gt = r16(1 / (1 + np.exp(-oracle.bf16_to_f32(sg).astype(np.float64))))[:, None]
    shv = r16(gt * sv)
    parity.combine_check(got, near, parity.switch_bound(near, near, sref.hscale), w16,
                         shared=(shv, gt * sa + 2.0 ** -8 * np.abs(shv)),
                         what=f"moe_layer gated T={T}")


@pytest.mark.parametrize("T", [1, 20])
def test_moe_layer_bad_expert_id(gpu, oracle, T):
    """Bad routed ids: their slots contribute zero, the shared expert and the other
    slots still add up, and the flag is raised.  One token runs the fused one-token
    form; 20 tokens (120 slots over 40 experts) sort the shared expert in as
    expert E, where a routed id of exactly E must still count as bad, not as the
    shared expert."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(971 + T)
    E, D, I, k = 40, 2048, 512, 6
    gate, up, down = _stack(rng, E, D, I)
    sh = _stack(rng, 1, D, I)
    x = make_x(rng, T, D)
    inds = topk_uniform(rng, T, E, k)
    bad = [(0, 2, E + 7)] if T == 1 else [(0, 2, E + 7), (5, 1, E), (T - 1, 0, 2 ** 32 - 1)]
    inds = inds.astype(np.int64)
    for t, j, v in bad:
        inds[t, j] = v
    w16 = oracle.f32_to_bf16(rng.dirichlet(np.ones(k), size=T).astype(np.float32))
    dev = lambda t: to_dev(t, gpu)
    announce(f"moe_layer bad id T={T}")
    out = ops.moe_layer(dev(x), dev(inds.astype(np.uint32)), tuple(map(dev, gate)),
                        tuple(map(dev, up)), tuple(map(dev, down)), dev(w16),
                        tuple(tuple(map(dev, q)) for q in sh))
    torch.cuda.synchronize()
    got = to_np(out)
    with pytest.raises(FmxqError):
        ops.device_error()
    safe = np.where(inds >= E, 0, inds).astype(np.int32)
    sref = parity.SwitchRef(x, safe, gate, up, down, fused=False)
    near = sref.refs[0].copy()
    allow = parity.switch_bound(near, near, sref.hscale)
    for t, j, _ in bad:
        near[t, j] = 0.0
        allow[t, j] = 0.0
    ssref = parity.SwitchRef(x, np.zeros((T, 1), dtype=np.int32), *sh, fused=False)
    sv = ssref.refs[0]
    sa = parity.switch_bound(sv, sv, ssref.hscale)
    parity.combine_check(got, near, allow, w16, shared=(sv[:, 0], sa[:, 0]),
                         what="moe_layer bad id")


def test_moe_layer_graph_replay(gpu, oracle):
    """moe_layer under HIP graph capture: the one-token form, the few-slot form
    (whose shared expert ids come from a zero buffer filled once per buffer) and
    the sorted form (the shared expert sorted in as expert E) replay to the eager
    result every time, with eager calls of other sizes on the same stream in
    between."""
    from fastmlx_amd import ops

    (gate, up, down), dstack, shared, dshared = _layer_weights(gpu, "c4")
    rng = np.random.default_rng(990)
    E, D = gate[0].shape[0], down[0].shape[1]
    k = 8
    cases = []
    for T in (1, 4, 40):
        inds = topk_zipf(rng, T, E, k)
        g = 1 / (1 + np.exp(-rng.standard_normal((T, k))))
        w16 = oracle.f32_to_bf16((g / g.sum(1, keepdims=True)).astype(np.float32))
        cases.append((to_dev(make_x(rng, T, D), gpu), to_dev(inds.astype(np.uint32), gpu),
                      to_dev(w16, gpu), torch.empty(T, D, dtype=torch.bfloat16, device=gpu)))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())

    def step():
        for x, inds, w, out in cases:
            ops.moe_layer(x, inds, *dstack, w, dshared, out=out)

    announce("moe_layer graph capture")
    with torch.cuda.stream(side):
        step()
    torch.cuda.synchronize()
    eager = [to_np(c[-1]).copy() for c in cases]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        step()
    xo, io, wo, oo = cases[1]
    for rep in range(3):
        for c in cases:
            c[-1].zero_()
        g.replay()
        torch.cuda.synchronize()
        for c, e in zip(cases, eager):
            assert np.array_equal(to_np(c[-1]), e), f"replay {rep} differs from eager"
        with torch.cuda.stream(side):  # eager work of another size between replays
            ops.moe_layer(xo[:2], io[:2], *dstack, wo[:2], dshared)
        torch.cuda.synchronize()
