"""GPU parity: the MoE routers (softmax top-k and DeepSeek's group-limited top-k)
against the oracle and the reference's own routing vectors.

The routers are fp32 on the device and fp64 in the oracle.  Picks must agree
exactly except where two candidates at the k-th place differ by less than fp32
can resolve (a near tie); weights agree to 1e-5 relative (fp32 output) or to
bf16 rounding (bf16 output).
"""
import json
import os

import numpy as np
import pytest
import torch

from gpu_util import announce

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def _picks_agree(got_i, want_i, key):
    """Same picks in the same order, or a swap at a near tie of `key`."""
    if np.array_equal(got_i, want_i):
        return True
    for g, w in zip(got_i, want_i):
        if g != w and abs(key[g] - key[w]) > 1e-5 * max(1.0, abs(key[w])):
            return False
    return set(got_i.tolist()) == set(want_i.tolist()) or abs(
        key[got_i[-1]] - key[want_i[-1]]) <= 1e-5


def _check_rows(gi, gw, oi, ow, key, wtol):
    bad = 0
    for t in range(gi.shape[0]):
        if not _picks_agree(gi[t], oi[t], key[t]):
            bad += 1
            continue
        if np.array_equal(gi[t], oi[t]):
            assert np.allclose(gw[t], ow[t], rtol=wtol, atol=wtol * 1e-3), (t, gw[t], ow[t])
    assert bad == 0, f"{bad} rows picked different experts"


def _w_np(w):
    return w.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("T,E,k,in_dtype,out_dtype", [
    (512, 512, 10, torch.bfloat16, torch.bfloat16),   # C3 routing: 512 experts, top-10
    (128, 512, 10, torch.float32, torch.float32),
    (5, 64, 1, torch.float32, torch.float32),         # ragged T (not a multiple of 4 rows)
    (33, 1000, 16, torch.bfloat16, torch.float32),    # E not a multiple of 64
    (8, 1024, 64, torch.float32, torch.float32),      # the largest supported E and k
])
def test_softmax_router(gpu, oracle, T, E, k, in_dtype, out_dtype):
    from fastmlx_amd import ops

    announce(f"route_softmax_topk T={T} E={E} k={k} {in_dtype}->{out_dtype}")
    g = torch.Generator().manual_seed(T * 7 + E)
    logits = torch.randn(T, E, generator=g).to(in_dtype)
    for norm in (True, False):
        inds, w = ops.route_softmax_topk(logits.to(gpu), k, norm, out_dtype)
        torch.cuda.synchronize()
        x = logits.float().numpy()
        oi, ow = oracle.route_softmax_topk(x, k, norm=norm)
        gi = inds.cpu().numpy()
        wtol = 1e-5 if out_dtype == torch.float32 else 2 ** -8
        _check_rows(gi, _w_np(w), oi, ow, x.astype(np.float64), wtol)


@pytest.mark.parametrize("T,E,k,ng,tg,in_dtype,out_dtype", [
    (256, 256, 8, 8, 4, torch.float32, torch.float32),    # C4 routing: DeepSeek-V3 shape
    (256, 256, 8, 8, 4, torch.bfloat16, torch.bfloat16),
    (37, 64, 6, 8, 3, torch.float32, torch.float32),
    (16, 128, 4, 1, 1, torch.float32, torch.float32),     # no group restriction
    (16, 96, 5, 32, 7, torch.float32, torch.float32),     # groups of three experts
    (9, 64, 2, 64, 5, torch.float32, torch.float32),      # one expert per group
])
def test_group_router(gpu, oracle, T, E, k, ng, tg, in_dtype, out_dtype):
    from fastmlx_amd import ops

    announce(f"route_group_topk T={T} E={E} k={k} groups={ng}/{tg} {in_dtype}->{out_dtype}")
    g = torch.Generator().manual_seed(T * 11 + E + ng)
    gates = torch.randn(T, E, generator=g).to(in_dtype)
    bias = (torch.randn(E, generator=g) * 0.1).float()
    for norm, scale in ((True, 2.5), (False, 1.0)):
        inds, w = ops.route_group_topk(gates.to(gpu), bias.to(gpu), k, ng, tg, scale, norm,
                                       out_dtype)
        torch.cuda.synchronize()
        x = gates.float().numpy()
        oi, ow = oracle.route_group_topk(x, bias.numpy(), k, ng, tg, scale, norm)
        sig = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
        key = sig + bias.numpy().astype(np.float64)
        wtol = 1e-5 if out_dtype == torch.float32 else 2 ** -8
        _check_rows(inds.cpu().numpy(), _w_np(w), oi, ow, key, wtol)


def test_group_router_reference_vectors(gpu):
    """The reference fixture of TestDeepseekV3GroupExpertSelectParity
    (compute/models/deepseekv3_test.go:130-163) through the HIP router."""
    from fastmlx_amd import ops

    with open(os.path.join(HERE, "golden", "deepseek_routing.json")) as f:
        cases = json.load(f)["routing"]
    for c in cases:
        announce(f"route_group_topk fixture {c['label']}")
        gates = torch.tensor([c["gates"]], dtype=torch.float32, device=gpu)
        bias = torch.tensor(c["bias"], dtype=torch.float32, device=gpu)
        inds, w = ops.route_group_topk(gates, bias, c["top_k"], c["n_group"], c["topk_group"],
                                       c["routed_scaling_factor"], c["norm_topk_prob"])
        torch.cuda.synchronize()
        got = dict(zip(inds[0].cpu().tolist(), w[0].cpu().tolist()))
        want = dict(zip(c["inds"], c["scores"]))
        assert set(got) == set(want), (c["label"], got, want)
        for e, v in want.items():
            assert abs(got[e] - v) <= 1e-5 * abs(v), (c["label"], e, got[e], v)


def test_router_feeds_switch_glu_combine(gpu, oracle):
    """Router output drives the MoE pieces directly: softmax top-k weights in bf16
    into moe_combine give the oracle's weighted sum of the expert outputs."""
    from fastmlx_amd import ops

    announce("router -> moe_combine")
    T, E, k, D = 16, 64, 4, 256
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16).to(gpu)
    inds, w = ops.route_softmax_topk(logits, k, True, torch.bfloat16)
    y = torch.randn(T, k, D, generator=g).to(torch.bfloat16).to(gpu)
    out = ops.moe_combine(y, w)
    torch.cuda.synchronize()
    ref = (y.float() * w.float()[:, :, None]).sum(dim=1)
    assert torch.allclose(out.float(), ref, rtol=2e-2, atol=2e-2)
    assert (inds >= 0).all() and (inds < E).all()
