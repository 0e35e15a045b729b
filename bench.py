"""Benchmark of the quantized-linear hot path on one MI355X.

Workload: the Llama-3-8B-shaped decode stack -- 32
layers of q/k/v/o (4096->4096, 4096->1024 x2, 4096->4096) and gate/up/down
(4096->14336 x2, 14336->4096) int4 group-64 quantized linears -- at M=1 token.
One step = one pass over all 224 projections, captured once in a HIP graph and
replayed.  Weights are seeded random tensors generated on the GPU (3.9 GB, so
the 256 MB MALL cannot hold them); x ~ N(0,1) bf16.

value = algorithmic HBM bytes of the step / measured step time (GB/s).
Also reported, as extra fields: the same stack at M in {4, 8, 16, 32}, the
north-star qmv points (4-bit 14336x4096 and 4096x14336 at M=1, rotating over
distinct weight copies), the qmm points (4-bit, M=2048 and M=512) and one MoE layer of
configs 3 and 4 (moe_c3_M*, moe_c4_M*).

The CPU baseline times the oracle's OpenMP routine (oracle/, kind "port") on a
bounded sample of the same stack.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

LLAMA_PROJ = [  # name, N (out), K (in)
    ("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
    ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336),
]
GROUP = 64


def gen_quant(torch, N, K, bits, gen, dev):
    """Packed words are uniform random bits, i.e. every q uniform on 0..2^bits-1."""
    words = torch.randint(0, 2 ** 32, (N, K * bits // 32), dtype=torch.int64, device=dev,
                          generator=gen).to(torch.int32)
    G = K // GROUP
    if bits == 4:
        s = torch.empty(N, G, device=dev).uniform_(0.002, 0.02, generator=gen).to(torch.bfloat16)
        noise = torch.randn(N, G, device=dev, generator=gen) * 1e-3
        b = (-8.0 * s.float() + noise).to(torch.bfloat16)
    else:
        s = torch.empty(N, G, device=dev).uniform_(1e-4, 2e-3, generator=gen).to(torch.bfloat16)
        b = (-128.0 * s.float()).to(torch.bfloat16)
    return words, s, b


def build_stack(torch, layers, bits, gen, dev):
    return [{name: gen_quant(torch, N, K, bits, gen, dev) for name, N, K in LLAMA_PROJ}
            for _ in range(layers)]


def stack_bytes(M, layers, bits):
    from fastmlx_amd.roofline import qmm_bytes

    return layers * sum(qmm_bytes(M, N, K, bits, GROUP) for _, N, K in LLAMA_PROJ)


QMV_UP_PMC = os.path.join(ROOT, "profiles", "qmv1_gate_up_14336x4096_M1_traffic.md")


def measured_traffic(path):
    """HBM bytes per launch of the roofline kernel from its committed rocprofv3 --pmc
    summary (FETCH_SIZE and WRITE_SIZE, each scaled by the copy-kernel calibration),
    or None when no summary is present."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def capture(torch, fn):
    """Warm up fn eagerly on a side stream, then capture it into a HIP graph."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    # capture on the warmed stream: the split-K workspace is kept per stream
    with torch.cuda.graph(g, stream=side):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, reps, warmup):
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        g.replay()
    t1.record()
    t1.synchronize()
    return t0.elapsed_time(t1) / reps  # ms per replay


def stack_step_fn(torch, ops, stack, xs, outs, bits):
    def step():
        for layer in stack:
            for name, N, K in LLAMA_PROJ:
                w, s, b = layer[name]
                ops.quantized_matmul(xs[K], w, s, b, True, GROUP, bits, out=outs[name])
    return step


def moe_points(torch, ops, gen, dev):
    """Configs 3 and 4: one MoE layer per step (SwitchGLU over the routed experts,
    the weighted top-k combine, and for config 4 the shared expert).  Each step of
    a replayed graph uses its own routing (and, for config 4, its own shared
    expert) so that consecutive steps do not find their experts in the 256 MB
    last-level cache."""
    from fastmlx_amd.roofline import HBM_PEAK_GBS, moe_bytes

    def stacks(E, N, K):
        return gen_quant_stack(torch, E, N, K, gen, dev)

    out = {}
    # config 3: 512 experts, 2048 -> 512 -> 2048, top-10 uniform, softmax weights
    E, D, I, k = 512, 2048, 512, 10
    gate, up, down = stacks(E, I, D), stacks(E, I, D), stacks(E, D, I)
    for M in (1, 16, 128, 512):
        R = 16 if M <= 16 else 4
        x = torch.randn(M, D, device=dev, generator=gen).to(torch.bfloat16)
        routes = []
        for _ in range(R):
            inds = torch.argsort(torch.rand(M, E, device=dev, generator=gen), dim=1)[:, :k]
            w = torch.softmax(torch.randn(M, k, device=dev, generator=gen), dim=1)
            routes.append((inds.to(torch.int32).contiguous(), w.to(torch.bfloat16)))
        ys = torch.empty(M, k, D, device=dev, dtype=torch.bfloat16)
        yo = torch.empty(M, D, device=dev, dtype=torch.bfloat16)

        def fn():
            for inds, w in routes:
                ops.switch_glu(x, inds, gate, up, down, GROUP, 4, out=ys)
                ops.moe_combine(ys, w, out=yo)
        g = capture(torch, fn)
        per = time_graph(torch, g, 10, 2) / R
        hit = sum(int(torch.unique(r[0]).numel()) for r in routes) / R
        by = moe_bytes(M, D, I, k, int(round(hit)), 4, GROUP)
        gbps = by / (per * 1e-3) / 1e9
        out[f"moe_c3_M{M}"] = {"us": round(per * 1e3, 2), "GBps": round(gbps, 1),
                               "frac_hbm": round(gbps / HBM_PEAK_GBS, 4),
                               "experts_hit": round(hit, 1), "distinct_routings": R}
    del gate, up, down
    # config 4: 256 routed experts + 1 shared, 7168 -> 2048 -> 7168, top-8 Zipf(1.1)
    E, D, I, k = 256, 7168, 2048, 8
    gate, up, down = stacks(E, I, D), stacks(E, I, D), stacks(E, D, I)
    R = 8
    shared = [(stacks(1, I, D), stacks(1, I, D), stacks(1, D, I)) for _ in range(R)]
    pz = torch.arange(1, E + 1, device=dev, dtype=torch.float64) ** -1.1
    for M in (1, 32, 256):
        x = torch.randn(M, D, device=dev, generator=gen).to(torch.bfloat16)
        routes = []
        for _ in range(R):
            # sequential draws without replacement; ids permuted per step so that the
            # hot ranks land on different experts from step to step
            ranks = torch.multinomial(pz.expand(M, E), k, replacement=False, generator=gen)
            perm = torch.randperm(E, device=dev, generator=gen)
            inds = perm[ranks]
            w = torch.sigmoid(torch.randn(M, k, device=dev, generator=gen))
            w = w / w.sum(dim=1, keepdim=True)
            routes.append((inds.to(torch.int32).contiguous(), w.to(torch.bfloat16)))
        zero = torch.zeros(M, 1, device=dev, dtype=torch.int32)
        ys = torch.empty(M, k, D, device=dev, dtype=torch.bfloat16)
        ysh = torch.empty(M, 1, D, device=dev, dtype=torch.bfloat16)
        yo = torch.empty(M, D, device=dev, dtype=torch.bfloat16)

        def fn():
            for (inds, w), (sg, su, sd) in zip(routes, shared):
                ops.switch_glu(x, inds, gate, up, down, GROUP, 4, out=ys)
                ops.switch_glu(x, zero, sg, su, sd, GROUP, 4, out=ysh)
                ops.moe_combine(ys, w, shared=ysh.view(M, D), out=yo)
        g = capture(torch, fn)
        per = time_graph(torch, g, 6, 1) / R
        hit = sum(int(torch.unique(r[0]).numel()) for r in routes) / R
        by = moe_bytes(M, D, I, k, int(round(hit)), 4, GROUP, shared_I=I)
        gbps = by / (per * 1e-3) / 1e9
        out[f"moe_c4_M{M}"] = {"us": round(per * 1e3, 2), "GBps": round(gbps, 1),
                               "frac_hbm": round(gbps / HBM_PEAK_GBS, 4),
                               "experts_hit": round(hit, 1), "distinct_routings": R}
    return out


def gen_quant_stack(torch, E, N, K, gen, dev):
    """Stacked experts [E, N, K/8] with the same value distributions as gen_quant."""
    w, s, b = gen_quant(torch, E * N, K, 4, gen, dev)
    return w.view(E, N, -1), s.view(E, N, -1), b.view(E, N, -1)


def cpu_baseline(torch, stack, xs, M, bits, target_s=10.0):
    """Oracle CPU routine on the first layers of the same stack (same bytes)."""
    import numpy as np

    import oracle

    def host(t):
        t = t.detach().cpu()
        if t.dtype == torch.bfloat16:
            t = t.view(torch.int16)
        a = t.numpy()
        return np.ascontiguousarray(a.view(np.uint16 if a.dtype == np.int16 else np.uint32))

    xh = {K: host(x) for K, x in xs.items()}
    hosted = {}
    done_bytes, elapsed, passes = 0, 0.0, 0
    # cycle over the layers (3.9 GB in all, far beyond the host caches) until
    # about target_s seconds of CPU work have been timed
    while elapsed < target_s and passes < 64 * len(stack):
        i = passes % len(stack)
        if i not in hosted:
            hosted[i] = {name: tuple(host(t) for t in stack[i][name]) for name, _, _ in LLAMA_PROJ}
        hl = hosted[i]
        t0 = time.perf_counter()
        for name, N, K in LLAMA_PROJ:
            w, s, b = hl[name]
            oracle.qmm_cpu_fast(xh[K], w, s, b, GROUP, bits)
        elapsed += time.perf_counter() - t0
        done_bytes += stack_bytes(M, 1, bits)
        passes += 1
    return {
        "value": round(done_bytes / elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": oracle.num_threads(),
        "kind": "port",
        "sample": f"{passes} layer passes over the first {len(hosted)} layers of the same int4 "
                  f"stack at M={M} ({done_bytes / 1e6:.0f} MB algorithmic traffic in "
                  f"{elapsed:.1f} s), oracle_qmm_cpu_fast (OpenMP, fp32 accumulate)",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="skip the secondary points")
    ap.add_argument("--no-moe", action="store_true", help="skip the MoE layer points")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the path has no "
              f"multi-GPU mode in this build", file=sys.stderr)
        sys.exit(2)

    import torch

    from fastmlx_amd import ops
    from fastmlx_amd.roofline import (BF16_MFMA_PEAK_TFLOPS, HBM_PEAK_GBS, qmm_bytes,
                                      qmm_flops)

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1001)
    bits = 4
    L = args.layers
    stack = build_stack(torch, L, bits, gen, dev)
    torch.cuda.synchronize()

    def run_stack(M, reps, warmup):
        xs = {K: torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
              for K in (4096, 14336)}
        outs = {name: torch.empty(M, N, device=dev, dtype=torch.bfloat16)
                for name, N, _ in LLAMA_PROJ}
        g = capture(torch, stack_step_fn(torch, ops, stack, xs, outs, bits))
        ms = time_graph(torch, g, reps, warmup)
        return ms, xs

    # headline: M = 1
    ms, xs1 = run_stack(1, args.steps, args.warmup)
    total_bytes = stack_bytes(1, L, bits)
    value = total_bytes / (ms * 1e-3) / 1e9

    extra = {}
    roof = None
    if not args.quick:
        for M in (4, 8, 16, 32):
            msM, _ = run_stack(M, max(10, args.steps // 5), 2)
            extra[f"stack_M{M}_GBps"] = round(stack_bytes(M, L, bits) / (msM * 1e-3) / 1e9, 1)
            extra[f"stack_M{M}_ms"] = round(msM, 4)

        # north-star qmv points, rotating over the stack's distinct weight copies
        def qmv_rotation(names, N, K):
            x = torch.randn(1, K, device=dev, generator=gen).to(torch.bfloat16)
            y = torch.empty(1, N, device=dev, dtype=torch.bfloat16)
            mats = [layer[n] for layer in stack for n in names]
            # at least 128 launches per graph (the distinct copies in turn, repeated):
            # the graph's own start-up then adds little to the per-launch time
            seq = mats * -(-128 // len(mats))

            def fn():
                for w, s, b in seq:
                    ops.quantized_matmul(x, w, s, b, True, GROUP, bits, out=y)
            g = capture(torch, fn)
            ms_all = time_graph(torch, g, 10, 2)
            per = ms_all / len(seq)
            by = qmm_bytes(1, N, K, bits, GROUP)
            return per, by, len(mats), len(seq)

        per_up, by_up, n_up, l_up = qmv_rotation(("gate", "up"), 14336, 4096)
        per_dn, by_dn, n_dn, l_dn = qmv_rotation(("down",), 4096, 14336)
        gbps_up = by_up / (per_up * 1e-3) / 1e9
        gbps_dn = by_dn / (per_dn * 1e-3) / 1e9
        extra["qmv_14336x4096_M1"] = {"us": round(per_up * 1e3, 3), "GBps": round(gbps_up, 1),
                                      "frac_hbm": round(gbps_up / HBM_PEAK_GBS, 4),
                                      "distinct_copies": n_up, "launches_per_graph": l_up}
        extra["qmv_4096x14336_M1"] = {"us": round(per_dn * 1e3, 3), "GBps": round(gbps_dn, 1),
                                      "frac_hbm": round(gbps_dn / HBM_PEAK_GBS, 4),
                                      "distinct_copies": n_dn, "launches_per_graph": l_dn}
        roof = {"bound": "hbm", "achieved": round(gbps_up, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(gbps_up / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(QMV_UP_PMC),
                "kernel": "fmxq::qmv1_kernel<4,1,4,4,2,4,1> (gate/up 14336x4096, M=1)",
                "bytes_per_launch": by_up,
                "timing": "HIP events over a graph of %d back-to-back launches cycling over %d "
                          "distinct weight copies (%.0f MB, beyond the 256 MB last-level "
                          "cache); per-launch = total / launches" % (l_up, n_up, n_up * by_up / 1e6)}

        # qmm points: M = 2048 (north star) and 512 (config 2)
        for Mq in (2048, 512):
            for (N, K) in ((14336, 4096), (4096, 14336)):
                w, s, b = stack[0]["gate" if N == 14336 else "down"]
                x = torch.randn(Mq, K, device=dev, generator=gen).to(torch.bfloat16)
                y = torch.empty(Mq, N, device=dev, dtype=torch.bfloat16)

                def fn():
                    for _ in range(5):
                        ops.quantized_matmul(x, w, s, b, True, GROUP, bits, out=y)
                g = capture(torch, fn)
                per = time_graph(torch, g, 4, 1) / 5
                tf = qmm_flops(Mq, N, K) / (per * 1e-3) / 1e12
                extra[f"qmm_{N}x{K}_M{Mq}"] = {"us": round(per * 1e3, 2), "TFLOPs": round(tf, 1),
                                               "frac_mfma": round(tf / BF16_MFMA_PEAK_TFLOPS, 4)}

        if not args.no_moe:
            extra.update(moe_points(torch, ops, gen, dev))

    result = {
        "metric": "qmv HBM GB/s (% peak) at M=1; qmm TFLOP/s (% MFMA) at M=2048; vs CPU",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 x int4 (fp32 accumulate)",
        "data": "synthetic (seeded torch generator on the GPU; random-init int4 weights)",
        "config": {"workload": "Llama-3-8B-shaped decode stack of int4 group-64 quantized "
                               "linears (BASELINE configs[1]), M=1",
                   "layers": L, "projections_per_layer": len(LLAMA_PROJ), "M": 1,
                   "bits": bits, "group_size": GROUP, "bytes_per_step": total_bytes,
                   "graph": "one HIP graph per step (224 launches)"},
        "roofline": roof,
    }
    result.update(extra)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch, stack, xs1, 1, bits)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
