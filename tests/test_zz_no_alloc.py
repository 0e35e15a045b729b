"""fmxq_switch_glu_noalloc through the C ABI against fmxq_switch_glu.

The allocation-free entry point runs the same kernels with its scratch in one
fixed __device__ buffer per GPU.  Its outputs must equal the allocating entry
point's bit for bit, on two calls in a row with the second one smaller (the
buffer keeps the first call's contents), and must meet the oracle's
per-element bound.  A call needing more scratch than the buffer holds is
refused before anything runs.
"""
import ctypes

import numpy as np
import pytest
import torch

import parity
from gpu_util import announce, to_dev, to_np
from synth import make_quant, make_x, topk_uniform

pytestmark = pytest.mark.gpu


def _call(lib, name, x, inds, gate, up, down, out, T, k, E, D, I, bits, stream=None):
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    return getattr(lib, name)(p(x), p(inds), *(p(t) for t in gate), *(p(t) for t in up),
                              *(p(t) for t in down), p(out), T, k, E, D, I, 64, bits, stream)


def _case(gpu, lib, seed, E, T, k, D, I, bits=4):
    rng = np.random.default_rng(seed)
    gate = make_quant(rng, (E, I), D, bits)
    up = make_quant(rng, (E, I), D, bits)
    down = make_quant(rng, (E, D), I, bits)
    x = make_x(rng, T, D)
    inds = topk_uniform(rng, T, E, k)
    dev = lambda q: tuple(to_dev(t, gpu) for t in q)
    dg, du, dd = dev(gate), dev(up), dev(down)
    dx, di = to_dev(x, gpu), to_dev(inds.astype(np.uint32), gpu)
    ya = torch.empty(T, k, D, dtype=torch.bfloat16, device=gpu)
    yb = torch.full((T, k, D), 7.0, dtype=torch.bfloat16, device=gpu)
    announce(f"switch_glu vs switch_glu_noalloc E={E} T={T} k={k} D={D} I={I} bits={bits}")
    assert _call(lib, "fmxq_switch_glu", dx, di, dg, du, dd, ya, T, k, E, D, I, bits) == 0
    assert _call(lib, "fmxq_switch_glu_noalloc", dx, di, dg, du, dd, yb, T, k, E, D, I,
                 bits) == 0, lib.fmxq_last_error()
    torch.cuda.synchronize()
    a, b = to_np(ya), to_np(yb)
    assert np.array_equal(a, b), f"{np.count_nonzero(a != b)} elements differ"
    sel = np.array([0, T - 1])
    sref = parity.SwitchRef(x, inds, gate, up, down, 64, bits, token_sel=sel, fused=False)
    parity.check_switch(b[sel], sref, what="switch_glu_noalloc")


def test_noalloc_matches_switch_glu_twice(gpu):
    """A sorted batch (config 3's experts at M = 48: 480 slots, 32-slot windows), then
    a smaller few-slot call (one decode token, 10 slots, no sort) and a small 8-bit
    call that takes the gather path: each equals fmxq_switch_glu exactly."""
    from fastmlx_amd import _lib

    lib = _lib.load()
    _case(gpu, lib, 1, E=512, T=48, k=10, D=2048, I=512)
    _case(gpu, lib, 2, E=512, T=1, k=10, D=2048, I=512)
    _case(gpu, lib, 3, E=8, T=40, k=2, D=256, I=256, bits=8)


def test_noalloc_refuses_oversized_scratch(gpu):
    """8192 slots at I = 2048 need about 100 MB of scratch: refused with a shape
    error before anything is enqueued; the next call on the same GPU still works.
    Every operand is allocated at full size all the same."""
    from fastmlx_amd import _lib

    lib = _lib.load()
    E, T, k, D, I = 4, 4096, 2, 256, 2048
    rng = np.random.default_rng(9)
    q = lambda n, kk: tuple(to_dev(t, gpu) for t in make_quant(rng, (E, n), kk))
    gate, up, down = q(I, D), q(I, D), q(D, I)
    x = to_dev(make_x(rng, T, D), gpu)
    inds = to_dev(topk_uniform(rng, T, E, k).astype(np.uint32), gpu)
    out = torch.empty(T, k, D, dtype=torch.bfloat16, device=gpu)
    announce("switch_glu_noalloc oversized call")
    rc = _call(lib, "fmxq_switch_glu_noalloc", x, inds, gate, up, down, out, T, k, E, D, I, 4)
    assert rc == 3, rc  # FMXQ_ERR_SHAPE
    msg = lib.fmxq_last_error().decode()
    assert "scratch" in msg and "allocation-free" in msg, msg
    torch.cuda.synchronize()
    _case(gpu, lib, 4, E=16, T=4, k=4, D=256, I=512)


def test_noalloc_first_call_inside_graph_capture(gpu):
    """The allocation-free entry point's very first call on a fresh stream, made
    inside graph capture: every allocating path (the per-stream scratch, the
    workspaces) refuses to grow while a stream is captured, so a capture that
    succeeds and replays to fmxq_switch_glu's output bit for bit shows that the
    fixed buffer served the call.  Replayed twice, with an eager call of another
    size in between."""
    from fastmlx_amd import _lib

    lib = _lib.load()
    rng = np.random.default_rng(21)
    E, T, k, D, I = 64, 6, 4, 512, 512
    q = lambda n, kk: tuple(to_dev(t, gpu) for t in make_quant(rng, (E, n), kk))
    gate, up, down = q(I, D), q(I, D), q(D, I)
    x = to_dev(make_x(rng, T, D), gpu)
    inds = to_dev(topk_uniform(rng, T, E, k).astype(np.uint32), gpu)
    yg = torch.zeros(T, k, D, dtype=torch.bfloat16, device=gpu)
    ya = torch.empty(T, k, D, dtype=torch.bfloat16, device=gpu)
    fresh = torch.cuda.Stream()
    fresh.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    announce("switch_glu_noalloc first call inside graph capture")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=fresh):
        rc = _call(lib, "fmxq_switch_glu_noalloc", x, inds, gate, up, down, yg, T, k, E, D, I, 4,
                   ctypes.c_void_p(fresh.cuda_stream))
    assert rc == 0, lib.fmxq_last_error()
    assert _call(lib, "fmxq_switch_glu", x, inds, gate, up, down, ya, T, k, E, D, I, 4) == 0
    torch.cuda.synchronize()
    want = to_np(ya)
    for rep in range(2):
        yg.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(to_np(yg), want), f"replay {rep} differs from fmxq_switch_glu"
        _case(gpu, lib, 30 + rep, E=16, T=3, k=2, D=256, I=256)  # other contents in the buffer
