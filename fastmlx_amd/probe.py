"""Run one quantized-linear workload for a profiler to observe.

    python -m fastmlx_amd.probe --case qmv_up --launches 64

Cases (4-bit, group 64 unless noted):
  qmv_up     y[1,14336] = x[1,4096] . deq(W)^T over distinct weight copies
  qmv_down   y[1,4096]  = x[1,14336] . deq(W)^T over distinct weight copies
  qmm_up     M=2048, 14336x4096;  qmm_down  M=2048, 4096x14336
  skinny16   M=16, 14336x4096 over distinct copies
  moe_c3     config-3 MoE layer (512 experts, top-10) at --tokens M
  moe_c4     config-4 routed experts (256 experts, 7168 -> 2048 -> 7168, top-8
             Zipf(1.1)) at --tokens M; 8 routings rotate from launch to launch
  copy       a plain device copy of --mib MiB (calibrates byte counters: it
             reads and writes exactly that many bytes per dispatch)

Weight copies rotate so every launch streams its weights from HBM (16 copies
of a 29 MB matrix exceed the 256 MB last-level cache).  Prints one line per
case with the launch count and the algorithmic bytes per launch, which is what
a FETCH_SIZE / WRITE_SIZE reading is compared against.
"""
from __future__ import annotations

import argparse
import json


def _quant(torch, N, K, bits, gen, dev):
    words = torch.randint(0, 2 ** 32, (N, K * bits // 32), dtype=torch.int64, device=dev,
                          generator=gen).to(torch.int32)
    s = torch.empty(N, K // 64, device=dev).uniform_(0.002, 0.02, generator=gen)
    b = (-8.0 * s + 1e-3 * torch.randn(N, K // 64, device=dev, generator=gen))
    return words, s.to(torch.bfloat16), b.to(torch.bfloat16)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--case", required=True,
                    choices=["qmv_up", "qmv_down", "qmm_up", "qmm_down", "skinny16", "moe_c3",
                             "moe_c4", "copy"])
    ap.add_argument("--launches", type=int, default=64)
    ap.add_argument("--copies", type=int, default=16)
    ap.add_argument("--mib", type=int, default=512)
    ap.add_argument("--tokens", type=int, default=128)
    args = ap.parse_args()

    import torch

    from . import ops
    from .roofline import moe_bytes, qmm_bytes

    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    info = {"case": args.case}
    if args.case == "copy":
        n = args.mib * (1 << 20)
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(args.launches):
            dst.copy_(src)
        info.update(read_bytes=n, write_bytes=n)
    elif args.case == "moe_c3":
        E, D, I, k, M = 512, 2048, 512, 10, args.tokens
        mats = [(_quant(torch, E * I, D, 4, gen, dev), _quant(torch, E * I, D, 4, gen, dev),
                 _quant(torch, E * D, I, 4, gen, dev))]
        trip = lambda q, o, i: (q[0].view(E, o, -1), q[1].view(E, o, -1), q[2].view(E, o, -1))
        g, u, d = mats[0]
        gate, up, down = trip(g, I, D), trip(u, I, D), trip(d, D, I)
        x = torch.randn(M, D, device=dev, generator=gen).to(torch.bfloat16)
        inds = torch.stack([torch.randperm(E, device=dev, generator=gen)[:k] for _ in range(M)])
        inds = inds.to(torch.int32)
        for _ in range(args.launches):
            ops.switch_glu(x, inds, gate, up, down, 64, 4)
        hit = int(torch.unique(inds).numel())
        info.update(algorithmic_bytes=moe_bytes(M, D, I, k, hit, 4, 64), experts_hit=hit)
    elif args.case == "moe_c4":
        E, D, I, k, M, R = 256, 7168, 2048, 8, args.tokens, 8
        gate = [t.view(E, I, -1) for t in _quant(torch, E * I, D, 4, gen, dev)]
        up = [t.view(E, I, -1) for t in _quant(torch, E * I, D, 4, gen, dev)]
        down = [t.view(E, D, -1) for t in _quant(torch, E * D, I, 4, gen, dev)]
        x = torch.randn(M, D, device=dev, generator=gen).to(torch.bfloat16)
        pz = torch.arange(1, E + 1, device=dev, dtype=torch.float64) ** -1.1
        routes = []
        for _ in range(R):
            ranks = torch.multinomial(pz.expand(M, E), k, replacement=False, generator=gen)
            routes.append(torch.randperm(E, device=dev, generator=gen)[ranks].to(torch.int32))
        ys = torch.empty(M, k, D, device=dev, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        for i in range(args.launches):
            ops.switch_glu(x, routes[i % R], gate, up, down, 64, 4, out=ys)
        hit = sum(int(torch.unique(r).numel()) for r in routes) / R
        info.update(algorithmic_bytes=moe_bytes(M, D, I, k, int(round(hit)), 4, 64),
                    experts_hit=hit)
    else:
        shapes = {"qmv_up": (1, 14336, 4096), "qmv_down": (1, 4096, 14336),
                  "qmm_up": (2048, 14336, 4096), "qmm_down": (2048, 4096, 14336),
                  "skinny16": (16, 14336, 4096)}
        M, N, K = shapes[args.case]
        copies = args.copies if M <= 32 else 1
        mats = [_quant(torch, N, K, 4, gen, dev) for _ in range(copies)]
        x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
        y = torch.empty(M, N, device=dev, dtype=torch.bfloat16)
        torch.cuda.synchronize()
        for i in range(args.launches):
            w, s, b = mats[i % copies]
            ops.quantized_matmul(x, w, s, b, True, 64, 4, out=y)
        info.update(M=M, N=N, K=K, copies=copies, algorithmic_bytes=qmm_bytes(M, N, K, 4, 64))
    torch.cuda.synchronize()
    info["launches"] = args.launches
    print(json.dumps(info), flush=True)


if __name__ == "__main__":
    main()
