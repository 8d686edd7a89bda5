"""Headline benchmark: Cl(8,0) geometric product, forward + backward, fp32,
batch 262144, one MI355X (BASELINE.json metric "multivector-pairs/s fwd+bwd,
Cl(8,0) fp32, 1 MI355X; % FP32 VALU/MFMA peak").

One step = ``c = cl.geom_prod(a, b)`` + ``torch.autograd.grad(c, (a, b), gc)``
with gc all-ones, inputs resident in HBM. Prints ONE JSON line.

The JSON carries a ``roofline`` object for the dominant kernel (the fused
backward) timed with HIP events on the stream it runs on, and a
``cpu_baseline`` object: the oracle's einsum restatement (torch fp32) timed on
this host's cores on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_TFLOPS = 157.3   # MI355X FP32 (vector packed / matrix) peak
PEAK_HBM_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--batch", type=int, default=262144)
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


def cpu_baseline(n: int, budget_s: float):
    """Oracle einsum restatement (fp32 torch, all host threads) on a bounded
    sample: fwd + bwd (autograd) of the Cl(n,0) geometric product."""
    import torch
    from oracle import clifford_oracle as O
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    rows = 256
    g = torch.Generator().manual_seed(0)
    a = torch.randn(rows, 1 << n, generator=g).requires_grad_()
    b = torch.randn(rows, 1 << n, generator=g).requires_grad_()
    gc = torch.ones(rows, 1 << n)
    done, t0 = 0, time.perf_counter()
    times = []
    while True:
        t1 = time.perf_counter()
        c = O.einsum_product("geom", a, b)
        torch.autograd.grad(c, (a, b), gc)
        times.append(time.perf_counter() - t1)
        done += rows
        if time.perf_counter() - t0 > budget_s or len(times) >= 50:
            break
    times.sort()
    med = times[len(times) // 2]
    return {"value": rows / med, "unit": "multivector-pairs/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{len(times)} chunks x {rows} rows of Cl({n},0) geom_prod fwd+bwd (oracle einsum "
                      f"restatement, torch fp32 CPU, median chunk time)"}


def load_traffic():
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 (sharding is designed, not built)"}))
        sys.exit(2)
    import torch
    import cliffordcuda_amd as cc
    from cliffordcuda_amd import _lib

    n, B = 8, args.batch
    D = 1 << n
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    g = torch.Generator().manual_seed(0)
    a = torch.randn(B, D, generator=g).to(dev).requires_grad_()
    b = torch.randn(B, D, generator=g).to(dev).requires_grad_()
    gc = torch.ones(B, D, device=dev)
    cl = cc.CliffordAlgebra([1] * n, device=dev)

    def step():
        c = cl.geom_prod(a, b)
        return torch.autograd.grad(c, (a, b), gc)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps

    # per-kernel average durations with HIP events on the launch stream
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    c = torch.empty_like(a)
    ga = torch.empty_like(a)
    gb = torch.empty_like(a)
    reps = max(5, args.steps)

    def time_kernel(fn):
        fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / reps

    fwd_ms = time_kernel(lambda: lib.clf_product_fwd(0, n, 0, 0, a.data_ptr(), b.data_ptr(), c.data_ptr(), B, sp))
    bwd_ms = time_kernel(lambda: lib.clf_product_bwd(0, n, 0, 0, a.data_ptr(), b.data_ptr(), gc.data_ptr(),
                                                     ga.data_ptr(), gb.data_ptr(), B, sp))
    n_terms = D * D                       # nonzero sigma terms per row (Cl(8,0))
    bwd_flops = 4.0 * n_terms * B         # two gradient sums, FMA = 2 flops
    fwd_flops = 2.0 * n_terms * B
    achieved = bwd_flops / (bwd_ms * 1e-3) / 1e12
    traffic = load_traffic().get("prod_bwd_blk<GEOM> Cl(8,0) B=262144")
    out = {
        "metric": "multivector-pairs/s fwd+bwd, Cl(8,0) fp32, 1 MI355X; % FP32 VALU/MFMA peak",
        "value": B / (ms * 1e-3),
        "unit": "multivector-pairs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic N(0,1) a, b (seed 0), gc = ones",
        "config": {"workload": "headline: Cl(8,0) geom_prod fwd+bwd", "batch": B, "n": n, "dim": D,
                   "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "valu", "kernel": "prod_bwd_blk<GEOM>", "achieved": achieved,
                     "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s", "frac": achieved / PEAK_FP32_TFLOPS,
                     "traffic": traffic, "kernel_ms": bwd_ms,
                     "algorithmic_flops_per_launch": bwd_flops},
        "kernels": {"prod_fwd_blk<GEOM>": {"ms": fwd_ms, "tflops": fwd_flops / (fwd_ms * 1e-3) / 1e12},
                    "prod_bwd_blk<GEOM>": {"ms": bwd_ms, "tflops": achieved},
                    "step_tflops_algorithmic": (fwd_flops + bwd_flops) / (ms * 1e-3) / 1e12},
        "cpu_baseline": None if args.no_cpu else cpu_baseline(n, args.cpu_seconds),
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
