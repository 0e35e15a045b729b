"""Benchmark of the quantized-linear hot path on one MI355X.

Headline workload: the Llama-3-8B-shaped decode stack.
- 32 layers of int4 group-64 quantized linears: q/k/v/o (4096->4096, 4096->1024
  twice, 4096->4096) and gate/up/down (4096->14336 twice, 14336->4096).
- M=1 token.
- One step is one pass over all 224 projections, captured once in a HIP graph
  and replayed.
- Weights are seeded random tensors generated on the GPU. At 3.9 GB they do not
  fit in the 256 MB last-level cache. x ~ N(0,1) in bf16.

value = algorithmic HBM bytes of the step / measured step time (GB/s).

Extra fields cover every other point of BASELINE.json:
- the stack at M in {4, 8, 16, 32};
- configuration 0 (2048x2048, M=1);
- the north-star decode GEMV (4096x14336, M=1) and its transpose;
- configuration 2 at M in {5, 64, 512, 2048}, 4-bit and 8-bit, both
  orientations;
- one MoE layer of configuration 3 at M in {1, 16, 128, 512};
- one MoE layer of configuration 4 at M in {1, 32, 256}.
Decode- and verify-sized points rotate over distinct weight copies, so every
launch streams its weights from HBM.

`roofline` describes the north-star kernel, the M=1 GEMV on 4096x14336.
- `achieved` = its algorithmic bytes per launch / its HIP-event time per launch,
  over a graph of back-to-back launches.
- `traffic` = its rocprofv3 FETCH_SIZE + WRITE_SIZE bytes per launch, read from
  the committed summary in profiles/.

`cpu_baseline` times the oracle's OpenMP routine (oracle/, kind "port") on a
bounded sample of the same stack. The qmm M=2048 point and one MoE point get
CPU timings of their own (cpu_points), and `host` states the host's sockets and
cores.

`python bench.py --probe CASE` runs one workload for a profiler and prints one
line (see PROBES).
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

LLAMA_PROJ = [  # name, N (out), K (in): llama.go:403-428
    ("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
    ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336),
]
GROUP = 64
PROFILES = os.path.join(ROOT, "profiles")
ROOF_PMC = os.path.join(PROFILES, "qmv1_down_4096x14336_M1_traffic.md")
QMM_PMC = os.path.join(PROFILES, "qmm_wide_14336x4096_M2048_counters.md")


def gen_quant(torch, N, K, bits, gen, dev):
    """Packed words are uniform random bits, i.e. every q uniform on 0..2^bits-1;
    scales and biases follow BASELINE.json (int4: s ~ U[0.002, 0.02], b = -8 s +
    N(0, 1e-3); int8: s ~ U[1e-4, 2e-3], b = -128 s)."""
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


def gen_quant_stack(torch, E, N, K, gen, dev):
    """Stacked experts [E, N, K/8] with the same value distributions as gen_quant."""
    w, s, b = gen_quant(torch, E * N, K, 4, gen, dev)
    return w.view(E, N, -1), s.view(E, N, -1), b.view(E, N, -1)


def build_stack(torch, layers, bits, gen, dev):
    return [{name: gen_quant(torch, N, K, bits, gen, dev) for name, N, K in LLAMA_PROJ}
            for _ in range(layers)]


def stack_bytes(M, layers, bits):
    from fastmlx_amd.roofline import qmm_bytes

    return layers * sum(qmm_bytes(M, N, K, bits, GROUP) for _, N, K in LLAMA_PROJ)


def profile_value(path, key):
    """A `key: value` line of a committed rocprofv3 summary, or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return float(line.split(":", 1)[1].strip())
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
    # capture on the warmed stream: the library's scratch is kept per stream
    with torch.cuda.graph(g, stream=side):
        fn()
    torch.cuda.synchronize()
    return g


def time_graph(torch, g, reps, warmup):
    """ms per replay: `warmup` untimed replays, then `reps` replays between two
    events on the replaying stream, synchronized on both sides."""
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / reps


def host_facts():
    """nproc and lscpu's sockets / cores, for the CPU baselines."""
    facts = {"nproc": os.cpu_count()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = dict(line.split(":", 1) for line in out.splitlines() if ":" in line)
        kv = {k.strip(): v.strip() for k, v in kv.items()}
        sockets = int(kv.get("Socket(s)", "0") or 0)
        cps = int(kv.get("Core(s) per socket", "0") or 0)
        facts.update(model=kv.get("Model name"), sockets=sockets, cores_per_socket=cps,
                     threads_per_core=int(kv.get("Thread(s) per core", "0") or 0),
                     physical_cores=sockets * cps)
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    try:
        facts["affinity_cpus"] = len(os.sched_getaffinity(0))
    except AttributeError:
        pass
    return facts


def host_np(torch, t):
    import numpy as np

    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    a = t.numpy()
    return np.ascontiguousarray(a.view(np.uint16 if a.dtype == np.int16 else np.uint32))


def cpu_baseline(torch, stack, xs, M, bits, target_s=10.0):
    """Oracle CPU routine on the first layers of the same stack (same bytes)."""
    import oracle

    xh = {K: host_np(torch, x) for K, x in xs.items()}
    hosted = {}
    done_bytes, elapsed, passes = 0, 0.0, 0
    # cycle over the layers (3.9 GB in all, far beyond the host caches) until
    # about target_s seconds of CPU work have been timed
    while elapsed < target_s and passes < 64 * len(stack):
        i = passes % len(stack)
        if i not in hosted:
            hosted[i] = {name: tuple(host_np(torch, t) for t in stack[i][name])
                         for name, _, _ in LLAMA_PROJ}
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


def cpu_qmm_point(torch, w, s, b, M, K, bits):
    """One quantized_matmul at M on the host (a single rep: ~0.24 TFLOP)."""
    import numpy as np

    import oracle
    from fastmlx_amd.roofline import qmm_flops

    rng = np.random.default_rng(5)
    x = oracle.f32_to_bf16(rng.standard_normal((M, K), dtype=np.float32))
    wh, sh, bh = (host_np(torch, t) for t in (w, s, b))
    N = wh.shape[0]
    t0 = time.perf_counter()
    oracle.qmm_cpu_fast(x, wh, sh, bh, GROUP, bits)
    dt = time.perf_counter() - t0
    return {"value": round(qmm_flops(M, N, K) / dt / 1e12, 4), "unit": "TFLOP/s",
            "cores": oracle.num_threads(), "kind": "port", "seconds": round(dt, 2),
            "sample": f"one {M}x{N}x{K} int4 product (single rep), oracle_qmm_cpu_fast"}


def cpu_moe_point(torch, gate, up, down, x, inds, weights):
    """One configuration-3 MoE layer on the host: per distinct expert, its slots'
    gate/up products, silu * up and the down product (oracle_qmm_cpu_fast), then
    the weighted combine; the same op chain and the same bytes as the GPU point."""
    import numpy as np

    import oracle

    gh = [host_np(torch, t) for t in gate]
    uh = [host_np(torch, t) for t in up]
    dh = [host_np(torch, t) for t in down]
    xh = host_np(torch, x)
    ih = inds.detach().cpu().numpy().astype(np.int64)
    wf = weights.detach().float().cpu().numpy()
    M, k = ih.shape
    D = xh.shape[1]
    r16 = lambda v: oracle.bf16_to_f32(oracle.f32_to_bf16(v.astype(np.float32)))
    t0 = time.perf_counter()
    flat = ih.reshape(-1)
    ys = np.zeros((M * k, D), dtype=np.float32)
    for e in np.unique(flat):
        slots = np.nonzero(flat == e)[0]
        xe = np.ascontiguousarray(xh[slots // k])
        g = oracle.bf16_to_f32(oracle.qmm_cpu_fast(xe, gh[0][e], gh[1][e], gh[2][e], GROUP, 4))
        u = oracle.bf16_to_f32(oracle.qmm_cpu_fast(xe, uh[0][e], uh[1][e], uh[2][e], GROUP, 4))
        sig = r16(1.0 / (1.0 + np.exp(-g)))
        h = oracle.f32_to_bf16(r16(r16(g * sig) * u))
        ys[slots] = oracle.bf16_to_f32(oracle.qmm_cpu_fast(h, dh[0][e], dh[1][e], dh[2][e],
                                                            GROUP, 4))
    r16((ys.reshape(M, k, D) * wf[:, :, None]).sum(1))
    dt = time.perf_counter() - t0
    return dt, int(np.unique(flat).size)


# ---------------------------------------------------------------------- points

def rotation_point(torch, ops, mats, M, N, K, bits, gen, dev, min_launches=128):
    """quantized_matmul at (M, N, K) over distinct weight copies in turn, at least
    min_launches per graph; returns ms per launch."""
    x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
    y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
    seq = mats * -(-min_launches // len(mats))

    def fn():
        for w, s, b in seq:
            ops.quantized_matmul(x, w, s, b, True, GROUP, bits, out=y)
    g = capture(torch, fn)
    reps = 10 if M <= 64 else 2
    return time_graph(torch, g, reps, 2) / len(seq), len(seq)


def dense_point(torch, ops, mats, M, N, K, bits, gen, dev):
    from fastmlx_amd.roofline import (BF16_MFMA_PEAK_TFLOPS, HBM_PEAK_GBS, qmm_bytes,
                                      qmm_flops, roofline_time_s)

    launches = 128 if M <= 64 else 16
    ms, n = rotation_point(torch, ops, mats, M, N, K, bits, gen, dev, launches)
    by, fl = qmm_bytes(M, N, K, bits, GROUP), qmm_flops(M, N, K)
    gbps = by / (ms * 1e-3) / 1e9
    tf = fl / (ms * 1e-3) / 1e12
    hbm_bound = by / (HBM_PEAK_GBS * 1e9) >= fl / (BF16_MFMA_PEAK_TFLOPS * 1e12)
    return {"us": round(ms * 1e3, 3), "GBps": round(gbps, 1), "TFLOPs": round(tf, 2),
            "frac_hbm": round(gbps / HBM_PEAK_GBS, 4),
            "frac_mfma": round(tf / BF16_MFMA_PEAK_TFLOPS, 4),
            "bound": "hbm" if hbm_bound else "mfma",
            "frac_roofline": round(roofline_time_s(by, fl) / (ms * 1e-3), 4),
            "distinct_copies": len(mats), "launches_per_graph": n}


def ingest_points(torch, ops, gen, dev, cpu):
    """quantize and dequantize at one DeepSeek-V3 kv_b_proj band: [128 heads x 256,
    512] bf16, int4 group 64 (the requantize and the dequantize of absorbKVB,
    deepseekv3.go:633,662-669), over 16 distinct copies (a graph of 64 launches).
    HBM bytes per call: the bf16 values, the packed words and the scale/bias pairs."""
    from fastmlx_amd.roofline import HBM_PEAK_GBS

    rows, K, bits = 32768, 512, 4
    by = rows * K * 2 + rows * K * bits // 8 + rows * (K // GROUP) * 4
    src = [(torch.randn(rows, K, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
           for _ in range(16)]
    trips = [ops.quantize(t, GROUP, bits) for t in src]
    deq = torch.empty(rows, K, device=dev, dtype=torch.bfloat16)
    seq = list(range(len(src))) * 4

    def fq():
        for i in seq:
            ops.quantize(src[i], GROUP, bits, out=trips[i])

    def fd():
        for i in seq:
            ops.dequantize(*trips[i], GROUP, bits, out=deq)
    out, cpu_out = {}, {}
    for name, fn in (("quantize", fq), ("dequantize", fd)):
        ms = time_graph(torch, capture(torch, fn), 10, 2) / len(seq)
        gbps = by / (ms * 1e-3) / 1e9
        out[f"ingest_{name}_32768x512_4bit"] = {
            "us": round(ms * 1e3, 3), "GBps": round(gbps, 1),
            "frac_hbm": round(gbps / HBM_PEAK_GBS, 4), "bytes_per_call": by,
            "distinct_copies": len(src), "launches_per_graph": len(seq)}
    if cpu:
        import oracle

        h = host_np(torch, src[0])
        t0 = time.perf_counter()
        oracle.quantize(h, GROUP, bits)
        dt = time.perf_counter() - t0
        cpu_out["ingest_quantize_32768x512_4bit"] = {
            "value": round(by / dt / 1e9, 3), "unit": "GB/s", "cores": oracle.num_threads(),
            "kind": "port", "sample": "one 32768x512 band, oracle_quantize (OpenMP)"}
    return out, cpu_out


def moe_points(torch, ops, gen, dev, cpu):
    """Configs 3 and 4: one MoE layer per step.
    - Configuration 3's step is switch_glu_combine: SwitchGLU over the routed
      experts and the weighted top-k combine in one call.  Configuration 4's is
      moe_layer: the same plus its shared expert MLP, computed inside the call.
    - Each step of a replayed graph has its own routing, and for configuration 4
      its own shared expert, so consecutive steps do not find their experts in
      the 256 MB last-level cache."""
    from fastmlx_amd.roofline import HBM_PEAK_GBS, moe_bytes

    out, cpu_out = {}, {}
    # config 3: 512 experts, 2048 -> 512 -> 2048, top-10 uniform, softmax weights
    E, D, I, k = 512, 2048, 512, 10
    gate, up, down = (gen_quant_stack(torch, E, I, D, gen, dev),
                      gen_quant_stack(torch, E, I, D, gen, dev),
                      gen_quant_stack(torch, E, D, I, gen, dev))
    for M in (1, 16, 128, 512):
        R = 16 if M <= 16 else 4
        x = torch.randn(M, D, device=dev, generator=gen).to(torch.bfloat16)
        routes = []
        for _ in range(R):
            inds = torch.argsort(torch.rand(M, E, device=dev, generator=gen), dim=1)[:, :k]
            w = torch.softmax(torch.randn(M, k, device=dev, generator=gen), dim=1)
            routes.append((inds.to(torch.int32).contiguous(), w.to(torch.bfloat16)))
        yo = torch.empty(M, D, device=dev, dtype=torch.bfloat16)

        def fn():
            for inds, w in routes:
                ops.switch_glu_combine(x, inds, gate, up, down, w, out=yo)
        g = capture(torch, fn)
        per = time_graph(torch, g, 10, 2) / R
        hit = sum(int(torch.unique(r[0]).numel()) for r in routes) / R
        by = moe_bytes(M, D, I, k, int(round(hit)), 4, GROUP)
        gbps = by / (per * 1e-3) / 1e9
        out[f"moe_c3_M{M}"] = {"us": round(per * 1e3, 2), "GBps": round(gbps, 1),
                               "frac_hbm": round(gbps / HBM_PEAK_GBS, 4),
                               "experts_hit": round(hit, 1), "distinct_routings": R}
        if cpu and M == 128:
            dt, hit0 = cpu_moe_point(torch, gate, up, down, x, routes[0][0], routes[0][1])
            by0 = moe_bytes(M, D, I, k, hit0, 4, GROUP)
            import oracle

            cpu_out[f"moe_c3_M{M}"] = {
                "value": round(by0 / dt / 1e9, 3), "unit": "GB/s", "cores": oracle.num_threads(),
                "kind": "port", "seconds": round(dt, 3),
                "sample": f"one routing of the same layer ({hit0} experts hit), per-expert "
                          f"oracle_qmm_cpu_fast products and the op chain in numpy"}
    del gate, up, down
    # config 4: 256 routed experts + 1 shared, 7168 -> 2048 -> 7168, top-8 Zipf(1.1)
    E, D, I, k = 256, 7168, 2048, 8
    gate, up, down = (gen_quant_stack(torch, E, I, D, gen, dev),
                      gen_quant_stack(torch, E, I, D, gen, dev),
                      gen_quant_stack(torch, E, D, I, gen, dev))
    R = 8
    shared = [(gen_quant_stack(torch, 1, I, D, gen, dev), gen_quant_stack(torch, 1, I, D, gen, dev),
               gen_quant_stack(torch, 1, D, I, gen, dev)) for _ in range(R)]
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
        yo = torch.empty(M, D, device=dev, dtype=torch.bfloat16)

        def fn():
            for (inds, w), sh in zip(routes, shared):
                ops.moe_layer(x, inds, gate, up, down, w, sh, out=yo)
        g = capture(torch, fn)
        per = time_graph(torch, g, 6, 1) / R
        hit = sum(int(torch.unique(r[0]).numel()) for r in routes) / R
        by = moe_bytes(M, D, I, k, int(round(hit)), 4, GROUP, shared_I=I)
        gbps = by / (per * 1e-3) / 1e9
        out[f"moe_c4_M{M}"] = {"us": round(per * 1e3, 2), "GBps": round(gbps, 1),
                               "frac_hbm": round(gbps / HBM_PEAK_GBS, 4),
                               "experts_hit": round(hit, 1), "distinct_routings": R}
    return out, cpu_out


# ---------------------------------------------------------------------- probes

PROBES = {
    # name: (M, N, K, bits) dense products over rotating weight copies
    "qmv_down": (1, 4096, 14336, 4), "qmv_up": (1, 14336, 4096, 4),
    "qmv_c0": (1, 2048, 2048, 4), "tied_head": (1, 128256, 4096, 4),
    "qmvx4_up": (4, 14336, 4096, 4), "qmvx8_up": (8, 14336, 4096, 4),
    "skinny16_up": (16, 14336, 4096, 4), "skinny32_up": (32, 14336, 4096, 4),
    "skinny16_down": (16, 4096, 14336, 4), "skinny32_down": (32, 4096, 14336, 4),
    "skinny64_up": (64, 14336, 4096, 4), "skinny64_down": (64, 4096, 14336, 4),
    "qmm_up": (2048, 14336, 4096, 4), "qmm_down": (2048, 4096, 14336, 4),
    "qmm512_up": (512, 14336, 4096, 4), "qmm512_down": (512, 4096, 14336, 4),
}


def probe(args):
    """One workload for a profiler to observe: --launches launches of the case.

    Dense cases rotate --copies weight copies (16 copies of a 29 MB matrix exceed
    the 256 MB last-level cache); moe_c3 / moe_c4 run one SwitchGLU per launch at
    --tokens (with --combine, switch_glu_combine with softmax routing weights, the
    call the bench times); quantize / dequantize run one DeepSeek-V3 kv_b_proj band
    (32768 x 512, int4 group 64) per launch; copy is a plain device copy of --mib MiB, which reads
    and writes exactly that many bytes per dispatch (the byte counters'
    calibration)."""
    import torch

    from fastmlx_amd import ops
    from fastmlx_amd.roofline import moe_bytes, qmm_bytes

    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    info = {"case": args.probe}
    if args.probe == "copy":
        n = args.mib * (1 << 20)
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(args.launches):
            dst.copy_(src)
        info.update(read_bytes=n, write_bytes=n)
    elif args.probe in ("quantize", "dequantize"):
        rows, K, bits = 32768, 512, 4
        src = [(torch.randn(rows, K, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
               for _ in range(args.copies)]
        trips = [ops.quantize(t, GROUP, bits) for t in src]
        deq = torch.empty(rows, K, device=dev, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        for i in range(args.launches):
            j = i % args.copies
            if args.probe == "quantize":
                ops.quantize(src[j], GROUP, bits, out=trips[j])
            else:
                ops.dequantize(*trips[j], GROUP, bits, out=deq)
        info.update(rows=rows, K=K, bits=bits, copies=args.copies,
                    algorithmic_bytes=rows * K * 2 + rows * K * bits // 8 + rows * (K // GROUP) * 4)
    elif args.probe in ("moe_c3", "moe_c4"):
        c3 = args.probe == "moe_c3"
        E, D, I, k = (512, 2048, 512, 10) if c3 else (256, 7168, 2048, 8)
        M, R = args.tokens, 8
        gate = gen_quant_stack(torch, E, I, D, gen, dev)
        up = gen_quant_stack(torch, E, I, D, gen, dev)
        down = gen_quant_stack(torch, E, D, I, gen, dev)
        x = torch.randn(M, D, device=dev, generator=gen).to(torch.bfloat16)
        routes = []
        pz = torch.arange(1, E + 1, device=dev, dtype=torch.float64) ** -1.1
        for _ in range(R):
            if c3:
                r = torch.argsort(torch.rand(M, E, device=dev, generator=gen), dim=1)[:, :k]
            else:
                ranks = torch.multinomial(pz.expand(M, E), k, replacement=False, generator=gen)
                r = torch.randperm(E, device=dev, generator=gen)[ranks]
            routes.append(r.to(torch.int32).contiguous())
        ws = [torch.softmax(torch.randn(M, k, device=dev, generator=gen), dim=1).to(torch.bfloat16)
              for _ in range(R)]
        ys = torch.empty(M, k, D, device=dev, dtype=torch.bfloat16)
        yo = torch.empty(M, D, device=dev, dtype=torch.bfloat16)
        # configuration 4's layer call carries its shared expert (moe_layer)
        sh = None if c3 or not args.combine else tuple(
            gen_quant_stack(torch, 1, n, kk, gen, dev) for n, kk in ((I, D), (I, D), (D, I)))
        torch.cuda.synchronize()
        for i in range(args.launches):
            if sh is not None:
                ops.moe_layer(x, routes[i % R], gate, up, down, ws[i % R], sh, out=yo)
            elif args.combine:
                ops.switch_glu_combine(x, routes[i % R], gate, up, down, ws[i % R], out=yo)
            else:
                ops.switch_glu(x, routes[i % R], gate, up, down, GROUP, 4, out=ys)
        hit = sum(int(torch.unique(r).numel()) for r in routes) / R
        info.update(algorithmic_bytes=moe_bytes(M, D, I, k, int(round(hit)), 4, GROUP,
                                                **({} if sh is None else {"shared_I": I})),
                    experts_hit=hit, combine=bool(args.combine), shared_expert=sh is not None)
    else:
        M, N, K, bits = PROBES[args.probe]
        copies = args.copies if M <= 32 else 1
        mats = [gen_quant(torch, N, K, bits, gen, dev) for _ in range(copies)]
        x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
        y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        for i in range(args.launches):
            w, s, b = mats[i % copies]
            ops.quantized_matmul(x, w, s, b, True, GROUP, bits, out=y)
        info.update(M=M, N=N, K=K, bits=bits, copies=copies,
                    algorithmic_bytes=qmm_bytes(M, N, K, bits, GROUP))
    torch.cuda.synchronize()
    info["launches"] = args.launches
    print(json.dumps(info), flush=True)


# ---------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--quick", action="store_true", help="skip the secondary points")
    ap.add_argument("--no-moe", action="store_true", help="skip the MoE layer points")
    ap.add_argument("--probe", choices=sorted(PROBES) + ["moe_c3", "moe_c4", "copy", "quantize",
                                                         "dequantize"],
                    help="run one workload for a profiler instead of the benchmark")
    ap.add_argument("--launches", type=int, default=64)
    ap.add_argument("--copies", type=int, default=16)
    ap.add_argument("--mib", type=int, default=512)
    ap.add_argument("--tokens", type=int, default=128)
    ap.add_argument("--combine", action="store_true",
                    help="moe probes: switch_glu_combine (the bench's call) instead of switch_glu")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the path has no "
              f"multi-GPU mode in this build", file=sys.stderr)
        sys.exit(2)
    if args.probe:
        probe(args)
        return

    import torch

    from fastmlx_amd import ops
    from fastmlx_amd.roofline import HBM_PEAK_GBS, qmm_bytes

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

        def step():
            for layer in stack:
                for name, N, K in LLAMA_PROJ:
                    w, s, b = layer[name]
                    ops.quantized_matmul(xs[K], w, s, b, True, GROUP, bits, out=outs[name])
        g = capture(torch, step)
        return time_graph(torch, g, reps, warmup), xs

    # headline: M = 1
    ms, xs1 = run_stack(1, args.steps, args.warmup)
    total_bytes = stack_bytes(1, L, bits)
    value = total_bytes / (ms * 1e-3) / 1e9

    extra, cpu_points = {}, {}
    roof = None
    if not args.quick:
        for M in (4, 8, 16, 32):
            msM, _ = run_stack(M, max(10, args.steps // 5), 2)
            extra[f"stack_M{M}_GBps"] = round(stack_bytes(M, L, bits) / (msM * 1e-3) / 1e9, 1)
            extra[f"stack_M{M}_ms"] = round(msM, 4)
            extra[f"stack_M{M}_frac_hbm"] = round(extra[f"stack_M{M}_GBps"] / HBM_PEAK_GBS, 4)

        # labelled comparison: the same stack at M = 1 with q|k|v and gate|up each in one
        # fmxq_quantized_matmul_group call (4 launches a layer instead of 7, same weights)
        x4 = xs1[4096]
        yq = {name: torch.empty(1, N, device=dev, dtype=torch.bfloat16)
              for name, N, _ in LLAMA_PROJ}

        def grouped_step():
            for layer in stack:
                ops.quantized_matmul_group(x4, [layer["q"], layer["k"], layer["v"]], GROUP, bits,
                                           outs=[yq["q"], yq["k"], yq["v"]])
                ops.quantized_matmul(x4, *layer["o"], True, GROUP, bits, out=yq["o"])
                ops.quantized_matmul_group(x4, [layer["gate"], layer["up"]], GROUP, bits,
                                           outs=[yq["gate"], yq["up"]])
                ops.quantized_matmul(xs1[14336], *layer["down"], True, GROUP, bits,
                                     out=yq["down"])
        msg = time_graph(torch, capture(torch, grouped_step), args.steps, args.warmup)
        extra["stack_M1_grouped_qkv_gateup"] = {
            "ms": round(msg, 4), "GBps": round(total_bytes / (msg * 1e-3) / 1e9, 1),
            "frac_hbm": round(total_bytes / (msg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "launches_per_step": 4 * L,
            "note": "q|k|v and gate|up each through one fmxq_quantized_matmul_group call on "
                    "the same separate weights (4 launches a layer instead of 7); not the "
                    "reference's call pattern, a comparison of the launch count only"}

        ups = [layer[n] for layer in stack for n in ("gate", "up")]
        downs = [layer["down"] for layer in stack]
        # north-star GEMV and its transpose; configuration 0 over 128 copies
        extra["qmv_4096x14336_M1"] = dense_point(torch, ops, downs, 1, 4096, 14336, 4, gen, dev)
        extra["qmv_14336x4096_M1"] = dense_point(torch, ops, ups, 1, 14336, 4096, 4, gen, dev)
        c0 = [gen_quant(torch, 2048, 2048, 4, gen, dev) for _ in range(128)]
        extra["c0_qmv_2048x2048_M1"] = dense_point(torch, ops, c0, 1, 2048, 2048, 4, gen, dev)
        del c0
        # the tied lm_head (llama.go:433-437): qlinear on the 128256 x 4096 embedding
        # triple, the largest single decode product; two copies (2 x 279 MB) so
        # every launch streams from HBM
        head = [gen_quant(torch, 128256, 4096, 4, gen, dev) for _ in range(2)]
        extra["tied_head_128256x4096_M1"] = dense_point(torch, ops, head, 1, 128256, 4096, 4, gen, dev)
        del head
        nd = extra["qmv_4096x14336_M1"]
        by_dn = qmm_bytes(1, 4096, 14336, 4, GROUP)
        # The same kernel on taller matrices of the same 14336-deep shape: the
        # increment between 16384 and 32768 rows is its steady-state streaming
        # rate, and what the 4096-row launch takes beyond its bytes at that rate is
        # the per-launch cost that does not scale with the bytes.
        sweep = {}
        for rows, copies in ((16384, 4), (32768, 2)):
            big = [gen_quant(torch, rows, 14336, 4, gen, dev) for _ in range(copies)]
            sweep[rows] = dense_point(torch, ops, big, 1, rows, 14336, 4, gen, dev)
            del big
        by16, by32 = qmm_bytes(1, 16384, 14336, 4, GROUP), qmm_bytes(1, 32768, 14336, 4, GROUP)
        dt = (sweep[32768]["us"] - sweep[16384]["us"]) * 1e-6
        marginal = (by32 - by16) / dt / 1e9 if dt > 0 else None
        extra["qmv_K14336_size_sweep"] = {
            "rows": [4096, 16384, 32768],
            "us": [nd["us"], sweep[16384]["us"], sweep[32768]["us"]],
            "frac_hbm": [nd["frac_hbm"], sweep[16384]["frac_hbm"], sweep[32768]["frac_hbm"]],
            "marginal_GBps": None if marginal is None else round(marginal, 1),
            "marginal_frac_hbm": None if marginal is None else round(marginal / HBM_PEAK_GBS, 4),
            "fixed_us_per_launch": None if marginal is None else
            round(nd["us"] - by_dn / (marginal * 1e9) * 1e6, 3)}
        traffic = profile_value(ROOF_PMC, "traffic_bytes_per_launch")
        roof = {"bound": "hbm", "achieved": nd["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": nd["frac_hbm"], "traffic": None if traffic is None else int(traffic),
                "kernel": "fmxq::qmv1_slice_kernel<16,7,1> (4-bit 4096x14336, M=1: the "
                          "north-star decode GEMV, the C1 down projection)",
                "bytes_per_launch": by_dn, "us_per_launch": nd["us"],
                "timing": "HIP events around a graph of %d back-to-back launches cycling over "
                          "%d distinct weight copies (%.0f MB, beyond the 256 MB last-level "
                          "cache); per launch = total / launches"
                          % (nd["launches_per_graph"], nd["distinct_copies"],
                             nd["distinct_copies"] * by_dn / 1e6)}

        # configuration 2: both orientations, 4- and 8-bit, M in {5, 64, 512, 2048}
        mats = {(14336, 4096, 4): ups, (4096, 14336, 4): downs}
        for (N, K) in ((14336, 4096), (4096, 14336)):
            mats[(N, K, 8)] = [gen_quant(torch, N, K, 8, gen, dev) for _ in range(10)]
        for bb in (4, 8):
            for (N, K) in ((14336, 4096), (4096, 14336)):
                for Mq in (5, 64, 512, 2048):
                    extra[f"c2_{bb}bit_{N}x{K}_M{Mq}"] = dense_point(
                        torch, ops, mats[(N, K, bb)], Mq, N, K, bb, gen, dev)
        del mats
        qm = extra["c2_4bit_14336x4096_M2048"]
        busy = profile_value(QMM_PMC, "mfma_busy")
        extra["qmm_M2048_mfma_busy_rocprof"] = busy
        # The qmm headline: the hand-written MFMA kernel that quantized_matmul runs
        # at prefill sizes (dequantization in registers, no vendor GEMM, no
        # workspace the size of W); both Config 2 orientations, int4 group 64.
        qd = extra["c2_4bit_4096x14336_M2048"]
        extra["qmm_M2048"] = {
            "kernel": "fmxq::qmm_wide_kernel<4,8,256> (hand-written HIP, bf16 MFMA 32x32x16)",
            "us": {"14336x4096": qm["us"], "4096x14336": qd["us"]},
            "TFLOPs": {"14336x4096": qm["TFLOPs"], "4096x14336": qd["TFLOPs"]},
            "frac_mfma": {"14336x4096": qm["frac_mfma"], "4096x14336": qd["frac_mfma"]},
            "peak_TFLOPs": 2500.0}
        if not args.no_cpu:
            w, s, b = stack[0]["gate"]
            cpu_points["c2_4bit_14336x4096_M2048"] = cpu_qmm_point(torch, w, s, b, 2048, 4096, 4)
            cpu_points["c2_4bit_14336x4096_M2048"]["gpu_over_cpu"] = round(
                qm["TFLOPs"] / max(cpu_points["c2_4bit_14336x4096_M2048"]["value"], 1e-9), 1)
        ing, ing_cpu = ingest_points(torch, ops, gen, dev, not args.no_cpu)
        extra.update(ing)
        cpu_points.update(ing_cpu)
        if not args.no_moe:
            moe, moe_cpu = moe_points(torch, ops, gen, dev, not args.no_cpu)
            extra.update(moe)
            cpu_points.update(moe_cpu)

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
        result["cpu_points"] = cpu_points
        result["host"] = host_facts()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
