"""GPU parity: gather_qmm (flat ABI form) vs the oracle."""
import numpy as np
import pytest
import torch

from gpu_util import announce, to_dev, to_np
import parity
from synth import make_quant, make_x, topk_uniform

pytestmark = pytest.mark.gpu


def _run(gpu, x, w, s, b, rhs, lhs=None, lhs_div=1, group=64, bits=4, sorted_indices=False):
    from fastmlx_amd import ops

    y = ops.gather_qmm(to_dev(x, gpu), to_dev(w, gpu), to_dev(s, gpu), to_dev(b, gpu),
                       to_dev(rhs.astype(np.uint32), gpu),
                       None if lhs is None else to_dev(lhs.astype(np.uint32), gpu), lhs_div,
                       True, group, bits, sorted_indices)
    torch.cuda.synchronize()
    return to_np(y)


@pytest.mark.parametrize("bits", [4, 8])
def test_switchglu_broadcast_form(gpu, oracle, bits):
    """x [T,1,K] against top_k experts per token (lhs_div = top_k)."""
    rng = np.random.default_rng(11 + bits)
    T, k, E, N, K = 6, 3, 9, 192, 256
    w, s, b = make_quant(rng, (E, N), K, bits, 64)
    x = make_x(rng, T, 1, K)
    inds = topk_uniform(rng, T, E, k)
    announce(f"gather broadcast bits={bits}")
    got = _run(gpu, x, w, s, b, inds.reshape(-1), lhs_div=k, bits=bits)
    ref = parity.gather_refs(x.reshape(T, K), w, s, b, np.repeat(np.arange(T), k),
                            inds.reshape(-1), 64, bits)
    assert got.shape == (T * k, 1, N)
    parity.check_dense(got.reshape(T * k, N), ref, what="gather_qmm")


def _close_ulps(a, b, ulps=2):
    fa = (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    fb = (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return float(np.max(np.abs(fa - fb) / (np.abs(fb) * 2.0 ** -8 + 1e-6)))


def test_sorted_hint_does_not_change_result(gpu, oracle):
    """sorted_indices selects the grouped kernel; the values it produces agree with
    the per-slot kernel to within bf16 rounding (switch_glu.go:28-30: the sort is
    only a memory-access win) and both meet the oracle tolerance."""
    rng = np.random.default_rng(3)
    S, E, N, K = 80, 8, 128, 512
    w, s, b = make_quant(rng, (E, N), K, 4, 64)
    x = make_x(rng, S, 1, K)
    rhs = np.sort(rng.integers(0, E, size=S)).astype(np.uint32)
    announce("gather sorted vs unsorted")
    a = _run(gpu, x, w, s, b, rhs, sorted_indices=True)
    c = _run(gpu, x, w, s, b, rhs, sorted_indices=False)
    assert _close_ulps(a, c) <= 2.0
    ref = parity.gather_refs(x.reshape(S, K), w, s, b, np.arange(S), rhs.astype(np.int32))
    for got in (a, c):
        parity.check_dense(got.reshape(S, N), ref, what="gather_qmm")


@pytest.mark.parametrize("bits,group", [(4, 64), (4, 128), (8, 32), (8, 64)])
@pytest.mark.parametrize("runs", [[1] * 40, [5, 3, 32, 1, 40, 7], [100], [31, 33, 2]])
def test_grouped_kernel_runs(gpu, oracle, bits, group, runs):
    """Expert-sorted batches whose runs start and end inside and across 32-slot
    tiles, with ragged N; each slot must equal its own per-slot product."""
    rng = np.random.default_rng(sum(runs) * 13 + bits + group)
    E, N, K = len(runs) + 3, 72, 256
    w, s, b = make_quant(rng, (E, N), K, bits, group)
    experts = np.sort(rng.choice(E, size=len(runs), replace=False))
    rhs = np.concatenate([np.full(r, e) for r, e in zip(runs, experts)]).astype(np.uint32)
    S = len(rhs)
    x = make_x(rng, S, 1, K)
    announce(f"grouped gather bits={bits} group={group} runs={runs[:6]}")
    got = _run(gpu, x, w, s, b, rhs, group=group, bits=bits, sorted_indices=True)
    ref = parity.gather_refs(x.reshape(S, K), w, s, b, np.arange(S), rhs.astype(np.int32), group,
                            bits)
    parity.check_dense(got.reshape(S, N), ref, what="gather_qmm")


def test_grouped_kernel_lhs_multirow_and_bad_ids(gpu, oracle):
    """Grouped path with explicit lhs, Mx = 2 rows per item and an out-of-range id
    inside the sorted run: that item's rows are zero and the flag is raised."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(21)
    E, N, K, xb, Mx = 6, 64, 128, 9, 2
    w, s, b = make_quant(rng, (E, N), K, 4, 64)
    x = make_x(rng, xb, Mx, K)
    rhs = np.array([0, 0, 1, 1, 1, 2, 4, 4, 4, 4, 4, 5, 5, 9, 9, 5, 0, 1, 1, 3], dtype=np.uint32)
    lhs = rng.integers(0, xb, size=len(rhs)).astype(np.uint32)
    announce("grouped gather with lhs, Mx=2, bad ids")
    got = _run(gpu, x, w, s, b, rhs, lhs=lhs, sorted_indices=True)
    good = rhs < E
    assert np.all(got[~good] == 0)
    xrow = (lhs[:, None].astype(np.int64) * Mx + np.arange(Mx)[None, :])[good].reshape(-1)
    ref = parity.gather_refs(x.reshape(xb * Mx, K), w, s, b, xrow,
                            np.repeat(rhs[good], Mx).astype(np.int32))
    parity.check_dense(got[good].reshape(-1, N), ref, what="gather_qmm")
    with pytest.raises(FmxqError):
        ops.device_error()


def test_explicit_lhs_and_multi_row_items(gpu, oracle):
    rng = np.random.default_rng(4)
    xb, Mx, E, N, K = 5, 3, 4, 64, 128
    w, s, b = make_quant(rng, (E, N), K, 8, 32)
    x = make_x(rng, xb, Mx, K)
    lhs = np.array([4, 0, 0, 2, 3, 1, 4], dtype=np.uint32)
    rhs = np.array([1, 3, 0, 0, 2, 1, 3], dtype=np.uint32)
    announce("gather explicit lhs, Mx=3")
    got = _run(gpu, x, w, s, b, rhs, lhs=lhs, group=32, bits=8)
    xrow = (lhs[:, None].astype(np.int64) * Mx + np.arange(Mx)[None, :]).reshape(-1)
    ref = parity.gather_refs(x.reshape(xb * Mx, K), w, s, b, xrow,
                            np.repeat(rhs, Mx).astype(np.int32), 32, 8)
    parity.check_dense(got.reshape(-1, N), ref, what="gather_qmm")


def test_out_of_range_expert_zeroes_and_flags(gpu):
    """An expert id >= E never reads outside the stack: zeros plus a device error."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(5)
    E, N, K = 4, 64, 128
    w, s, b = make_quant(rng, (E, N), K, 4, 64)
    x = make_x(rng, 3, 1, K)
    rhs = np.array([1, 7, 2], dtype=np.uint32)  # 7 is out of range
    announce("gather out-of-range id")
    got = _run(gpu, x, w, s, b, rhs)
    assert np.all(got[1] == 0)
    assert np.any(got[0] != 0)
    with pytest.raises(FmxqError) as ei:
        ops.device_error()
    assert ei.value.code == 4
    ops.device_error()  # cleared


def test_index_flag_is_per_stream(gpu):
    """The out-of-range flag belongs to the stream whose kernel raised it: another
    stream's check neither reports nor clears it."""
    from fastmlx_amd import FmxqError, ops

    rng = np.random.default_rng(6)
    E, N, K = 4, 64, 128
    w, s, b = make_quant(rng, (E, N), K, 4, 64)
    x = make_x(rng, 3, 1, K)
    bad = np.array([1, 9, 2], dtype=np.uint32)
    good = np.array([0, 3, 2], dtype=np.uint32)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    announce("index flags of two streams")
    with torch.cuda.stream(sa):
        _run(gpu, x, w, s, b, bad)
    with torch.cuda.stream(sb):
        _run(gpu, x, w, s, b, good)
        ops.device_error()  # nothing on this stream
    with torch.cuda.stream(sa):
        with pytest.raises(FmxqError) as ei:
            ops.device_error()
        assert ei.value.code == 4
        ops.device_error()  # cleared


@pytest.mark.parametrize("M", [1, 16])
def test_config3_expert_projection(gpu, oracle, M):
    """Config 3 gate projection: 512 experts, 2048 -> 512, top-10 per token."""
    rng = np.random.default_rng(600 + M)
    E, N, K, k = 512, 512, 2048, 10
    w, s, b = make_quant(rng, (E, N), K, 4, 64)
    x = make_x(rng, M, 1, K)
    inds = topk_uniform(rng, M, E, k)
    announce(f"config3 gather M={M}")
    got = _run(gpu, x, w, s, b, inds.reshape(-1), lhs_div=k)
    ref = parity.gather_refs(x.reshape(M, K), w, s, b, np.repeat(np.arange(M), k),
                            inds.reshape(-1))
    parity.check_dense(got.reshape(-1, N), ref, what="gather_qmm")


@pytest.mark.parametrize("cfg,M", [("c3", 128), ("c3", 512), ("c4", 32), ("c4", 256)])
def test_sorted_switch_projection_full_size(gpu, oracle, cfg, M):
    """The sorted branch of switchGLUCore (switch_glu.go:135-148) at config 3/4 sizes:
    slots sorted by expert, x rows gathered by order // top_k.  The oracle checks a
    sample of slots."""
    from synth import topk_zipf

    rng = np.random.default_rng(700 + M)
    if cfg == "c3":
        E, N, K, k = 512, 512, 2048, 10
        inds = topk_uniform(rng, M, E, k)
    else:
        E, N, K, k = 256, 2048, 7168, 8
        inds = topk_zipf(rng, M, E, k)
    w, s, b = make_quant(rng, (E, N), K, 4, 64)
    x = make_x(rng, M, 1, K)
    flat = inds.reshape(-1)
    order = np.argsort(flat, kind="stable")
    rhs = flat[order].astype(np.uint32)
    lhs = (order // k).astype(np.uint32)
    announce(f"sorted switch projection {cfg} M={M}")
    got = _run(gpu, x, w, s, b, rhs, lhs=lhs, sorted_indices=True).reshape(-1, N)
    sel = np.unique(np.concatenate([[0, len(rhs) - 1],
                                    rng.choice(len(rhs), size=24, replace=False)]))
    ref = parity.gather_refs(x.reshape(M, K), w, s, b, lhs[sel].astype(np.int32),
                            rhs[sel].astype(np.int32))
    parity.check_dense(got[sel], ref, what="gather_qmm")
