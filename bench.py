"""Benchmarks of the product & rotor hot path on one MI355X.

Default (the driver's contract): the headline workload of BASELINE.json's
metric, "multivector-pairs/s fwd+bwd, Cl(8,0) fp32, 1 MI355X; % FP32 VALU/MFMA
peak": Cl(8,0) geometric product, batch 262144, forward + backward, inputs
resident in HBM. One step = ``c = cl.geom_prod(a, b)`` +
``torch.autograd.grad(c, (a, b), gc)`` with gc all-ones. Prints ONE JSON line
with a ``roofline`` object for the dominant kernel (timed with HIP events on
the stream it runs on) and a ``cpu_baseline`` object (the oracle's einsum
restatement timed on this host's cores on a bounded sample).

``--workload all`` (or c1..c5) additionally measures the other BASELINE
configurations, one JSON line each, for the results table.
"""
from __future__ import annotations

import argparse
import contextlib
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_TFLOPS = 157.3   # MI355X FP32 peak (vector and matrix)
PEAK_HBM_GBS = 8000.0
METRIC = "multivector-pairs/s fwd+bwd, Cl(8,0) fp32, 1 MI355X; % FP32 VALU/MFMA peak"


@contextlib.contextmanager
def path_switch(name, value):
    """Set a CLF_* path switch for the block (the library reads the switches
    once per process, so each change is followed by a reload)."""
    from cliffordcuda_amd import _lib
    os.environ[name] = value
    _lib.reload_options()
    try:
        yield
    finally:
        del os.environ[name]
        _lib.reload_options()


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", default="headline",
                   choices=["headline", "c1", "c2", "c3", "c4", "c5", "all", "copycal", "published"])
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    return p.parse_args()


def n_terms(op: str, metric) -> int:
    """Nonzero sigma terms per row (counts of the reference's algorithmic flops)."""
    n = len(metric)
    r = sum(1 for m in metric if m == 0)
    return {"geom": 4 ** (n - r) * 3 ** r, "wedge": 3 ** n, "lc": 3 ** (n - r) * 2 ** r,
            "rc": 3 ** (n - r) * 2 ** r, "inner": 2 * 3 ** (n - r) * 2 ** r - 2 ** (n - r),
            "regressive": 3 ** n}[op]


def cpu_model() -> str:
    """The host CPU's model name (first 'model name' line of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(n: int, budget_s: float):
    """Oracle einsum restatement (fp32 torch, all host threads) on a bounded
    sample: fwd + bwd (autograd) of the Cl(n,0) geometric product."""
    import torch
    from oracle import clifford_oracle as O
    torch.set_num_threads(os.cpu_count() or 1)
    rows = 256
    g = torch.Generator().manual_seed(0)
    a = torch.randn(rows, 1 << n, generator=g).requires_grad_()
    b = torch.randn(rows, 1 << n, generator=g).requires_grad_()
    gc = torch.ones(rows, 1 << n)
    t0 = time.perf_counter()
    times = []
    while True:
        t1 = time.perf_counter()
        c = O.einsum_product("geom", a, b)
        torch.autograd.grad(c, (a, b), gc)
        times.append(time.perf_counter() - t1)
        if time.perf_counter() - t0 > budget_s or len(times) >= 50:
            break
    times.sort()
    med = times[len(times) // 2]
    return {"value": rows / med, "unit": "multivector-pairs/s", "cores": torch.get_num_threads(),
            "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(), "kind": "port",
            "sample": f"{len(times)} chunks x {rows} rows of Cl({n},0) geom_prod fwd+bwd (oracle einsum "
                      f"restatement, torch fp32 on the host CPU, median chunk time)"}


def cpu_rate(work, rows: int, budget_s: float, label: str, dtype: str = "fp32"):
    """Rows per second of work() (one chunk of `rows` rows through the oracle
    restatement on the host CPU, all threads), median over a bounded sample."""
    import torch
    torch.set_num_threads(os.cpu_count() or 1)
    times = []
    t0 = time.perf_counter()
    while True:
        t1 = time.perf_counter()
        work()
        times.append(time.perf_counter() - t1)
        if time.perf_counter() - t0 > budget_s or len(times) >= 20:
            break
    times.sort()
    return {"value": rows / times[len(times) // 2], "unit": "rows/s", "cores": torch.get_num_threads(),
            "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count(), "kind": "port",
            "sample": f"{len(times)} chunks x {rows} rows: {label} (oracle restatement, torch {dtype} on the "
                      f"host CPU, median chunk time)"}


# CPU baselines of --workload c1..c5 / all run after every GPU measurement of
# the invocation (host threads spinning after the oracle's parallel regions
# would otherwise slow the launches of the GPU steps): (dict, key, thunk).
CPU_JOBS = []


def cpu_product(op, metric, rows, fwd_only, budget_s):
    import torch
    from oracle import clifford_oracle as O
    n = len(metric)
    g = torch.Generator().manual_seed(0)
    a = torch.randn(rows, 1 << n, generator=g).requires_grad_(not fwd_only)
    b = torch.randn(rows, 1 << n, generator=g).requires_grad_(not fwd_only)

    def work():
        c = O.einsum_product(op, a, b, list(metric))
        if not fwd_only:
            torch.autograd.grad(c, (a, b), torch.ones_like(c))

    return cpu_rate(work, rows, budget_s, f"{op} {'fwd' if fwd_only else 'fwd+bwd'} {metric}")


class Clock:
    """Mean engine clock over a stretch of GPU work: clf_clock_sample launches
    one-wave workgroups that read the shader-clock counter (s_memtime) and the
    constant-rate counter (s_memrealtime) with their XCD index; a sample on the
    launch stream before the work and one after give, per XCD, cycles over
    real time."""

    SLOTS = 4096

    def __init__(self, torch, lib, stream):
        from cliffordcuda_amd import _lib
        self.torch, self.lib, self.stream = torch, lib, stream
        info = _lib.device_info(0)
        self.info = info
        self.buf = torch.zeros(2, 3 * self.SLOTS, dtype=torch.int64, device="cuda")

    def sample(self, k):
        from cliffordcuda_amd import _lib
        _lib.check(self.lib.clf_clock_sample(self.buf[k].data_ptr(), self.SLOTS, self.stream.cuda_stream),
                   "clf_clock_sample")

    def ghz(self):
        """Median over compute units (seen in both samples) of the mean clock
        between the two samples, and the per-XCD medians (None if the counters
        do not give a plausible value)."""
        h = self.buf.cpu().view(2, self.SLOTS, 3).tolist()
        first = [{}, {}]
        for k in range(2):
            for loc, cyc, rt in h[k]:
                if loc not in first[k] or cyc < first[k][loc][0]:
                    first[k][loc] = (cyc, rt)
        rate = self.info.wall_clock_khz * 1e3
        per_cu, per_xcd = [], {}
        for loc in set(first[0]) & set(first[1]):
            (c0, r0), (c1, r1) = first[0][loc], first[1][loc]
            if r1 <= r0 or c1 <= c0 or rate <= 0:
                continue
            v = (c1 - c0) / ((r1 - r0) / rate) / 1e9
            per_cu.append(v)
            per_xcd.setdefault(loc & 15, []).append(v)
        per_cu.sort()
        xcd = [sorted(v)[len(v) // 2] for _, v in sorted(per_xcd.items())]
        if not per_cu or not 0.3 < per_cu[len(per_cu) // 2] < 4.0:
            return None, xcd
        return per_cu[len(per_cu) // 2], xcd

    def device(self, ghz, vals, what):
        return {"compute_units": self.info.compute_units, "max_engine_clock_mhz": self.info.clock_khz / 1e3,
                "measured_engine_clock_ghz": ghz,
                "measured_engine_clock_ghz_per_xcd": [round(v, 3) for v in vals],
                "clock_method": f"clf_clock_sample before and after {what} on its stream: shader-clock cycles "
                                f"(s_memtime) over real time (s_memrealtime, {self.info.wall_clock_khz} kHz) "
                                f"per compute unit, median over compute units (per-XCD medians listed)"}


class Timer:
    def __init__(self, torch, stream, reps):
        self.torch, self.stream, self.reps = torch, stream, reps
        self.clock = None
        self.last_clock = (None, [])

    def kernel_ms(self, fn):
        """Average duration of fn() over `reps` back-to-back calls, HIP events on the launch stream,
        after at least 20 ms and max(10, reps / 4) calls of untimed work: the first calls after an
        idle GPU run slower (C2's first-timed kernels read 20 % slow after one warmup call)."""
        torch = self.torch
        t0 = time.perf_counter()
        calls = 0
        while calls < max(10, self.reps // 4) or time.perf_counter() - t0 < 0.02:
            fn()
            calls += 1
            if calls % 10 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        if self.clock is not None:
            self.clock.sample(0)
        e0.record(self.stream)
        for _ in range(self.reps):
            fn()
        e1.record(self.stream)
        if self.clock is not None:
            self.clock.sample(1)
        e1.synchronize()
        if self.clock is not None:
            self.last_clock = self.clock.ghz()
        return e0.elapsed_time(e1) / self.reps

    def step_ms(self, fn, warmup, steps):
        """Wall time per step of `steps` autograd steps after `warmup` untimed ones."""
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps


# Sub-millisecond steps (C3, C4) are timed over at least this many steps (0.15-
# 0.25 s of work): the first steps after an idle synchronize run up to 30 %
# slower, which dominates a 20-step window of 0.15 ms steps and still shows in a
# 200-step one.
MIN_SHORT_STEPS, MIN_SHORT_WARMUP = 1000, 50


def load_traffic():
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        return json.load(f)


def headline(args, torch, cc, lib, T):
    n, B = 8, 262144
    D = 1 << n
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(0)
    a = torch.randn(B, D, generator=g).to(dev).requires_grad_()
    b = torch.randn(B, D, generator=g).to(dev).requires_grad_()
    gc = torch.ones(B, D, device=dev)
    cl = cc.CliffordAlgebra([1] * n, device=dev)

    def step():
        c = cl.geom_prod(a, b)
        return torch.autograd.grad(c, (a, b), gc)

    ms = T.step_ms(step, args.warmup, args.steps)
    sp = T.stream.cuda_stream
    c = torch.empty_like(a)
    ga = torch.empty_like(a)
    gb = torch.empty_like(a)

    def fwd():
        lib.clf_product_fwd(0, n, 0, 0, a.data_ptr(), b.data_ptr(), c.data_ptr(), B, sp)

    def bwd():
        lib.clf_product_bwd(0, n, 0, 0, a.data_ptr(), b.data_ptr(), gc.data_ptr(), ga.data_ptr(), gb.data_ptr(), B, sp)

    # served path: Cl(8,0) is the real matrix algebra M_16(R), so the library
    # runs the matrix-representation kernels (rep16_fwd_kernel / rep16_bwd_kernel)
    fwd_ms = T.kernel_ms(fwd)
    bwd_ms = T.kernel_ms(bwd)
    bwd_clock = T.last_clock
    # the per-term kernels (the path of every other signature and product),
    # forced for comparison at the same shape
    with path_switch("CLF_GEOM_PATH", "direct"):
        dfwd_ms = T.kernel_ms(fwd)
        dbwd_ms = T.kernel_ms(bwd)
    # the same byte patterns without the arithmetic (clf_stream_probe over the
    # same buffers, nontemporal as the kernels stream): the rate this memory
    # system gives 3 reads + 2 writes (backward) and 2 reads + 1 write (forward)
    sfwd_ms = T.kernel_ms(lambda: lib.clf_stream_probe(2, 1, a.data_ptr(), b.data_ptr(), 0, c.data_ptr(), 0,
                                                       B * D, 1, sp))
    sbwd_ms = T.kernel_ms(lambda: lib.clf_stream_probe(3, 2, a.data_ptr(), b.data_ptr(), gc.data_ptr(), ga.data_ptr(),
                                                       gb.data_ptr(), B * D, 1, sp))
    nt = D * D
    bwd_flops = 4.0 * nt * B       # reference term-sum count: 2 products of 4^n multiply-adds
    fwd_flops = 2.0 * nt * B
    fwd_bytes = 12.0 * D * B       # read a, b; write c
    bwd_bytes = 20.0 * D * B       # read a, b, gc; write ga, gb
    achieved = bwd_bytes / (bwd_ms * 1e-3) / 1e9
    return {
        "metric": METRIC,
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
        "data": "synthetic: a, b ~ N(0,1) seed 0, gc = ones",
        "config": {"workload": "headline: Cl(8,0) geom_prod fwd+bwd, batch 262144, upstream gradient all-ones", "batch": B,
                   "n": n, "dim": D, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "kernel": "rep16_bwd_kernel", "achieved": achieved,
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS,
                     "traffic": load_traffic().get("rep16_bwd_kernel Cl(8,0) B=262144"),
                     "kernel_ms": bwd_ms, "algorithmic_bytes_per_launch": bwd_bytes,
                     "device": T.clock.device(*bwd_clock, "the rep16_bwd_kernel timing loop") if T.clock else None,
                     "stream_ceiling": {
                         "pattern": "clf_stream_probe: the same 3 reads + 2 writes of 268 MB, nontemporal, "
                                    "no arithmetic", "achieved": bwd_bytes / (sbwd_ms * 1e-3) / 1e9, "unit": "GB/s",
                         "kernel_ms": sbwd_ms, "frac_of_ceiling": sbwd_ms / bwd_ms}},
        "kernels": {
            "rep16_fwd_kernel": {"ms": fwd_ms, "gbs": fwd_bytes / (fwd_ms * 1e-3) / 1e9,
                                 "hbm_frac": fwd_bytes / (fwd_ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                                 "stream_ceiling_gbs": fwd_bytes / (sfwd_ms * 1e-3) / 1e9,
                                 "frac_of_stream_ceiling": sfwd_ms / fwd_ms},
            "rep16_bwd_kernel": {"ms": bwd_ms, "gbs": achieved, "hbm_frac": achieved / PEAK_HBM_GBS,
                                 "stream_ceiling_gbs": bwd_bytes / (sbwd_ms * 1e-3) / 1e9,
                                 "frac_of_stream_ceiling": sbwd_ms / bwd_ms},
            # per-term kernels: FP32 VALU bound, 4^n multiply-adds per product
            "prod_fwd_blk<GEOM> (per-term path)": {
                "ms": dfwd_ms, "tflops": fwd_flops / (dfwd_ms * 1e-3) / 1e12,
                "valu_frac": fwd_flops / (dfwd_ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS},
            "prod_bwd_blk<GEOM> (per-term path)": {
                "ms": dbwd_ms, "tflops": bwd_flops / (dbwd_ms * 1e-3) / 1e12,
                "valu_frac": bwd_flops / (dbwd_ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS},
        },
        # the reference's term count (4^n multiply-adds per product, 3 products
        # per step) over the step time: how fast the per-term formulation would
        # have to run to match this step. Not a utilisation: the matrix path does
        # 16^3 multiply-adds per product on the matrix cores.
        "term_count_equivalent_tflops": (fwd_flops + bwd_flops) / (ms * 1e-3) / 1e12,
        "cpu_baseline": None if args.no_cpu else cpu_baseline(n, args.cpu_seconds),
    }


def products_config(args, torch, cc, lib, T, name, metric, B, ops, fwd_only=False):
    n = len(metric)
    D = 1 << n
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(0)
    a = torch.randn(B, D, generator=g).to(dev)
    b = torch.randn(B, D, generator=g).to(dev)
    gc = torch.ones(B, D, device=dev)
    neg = sum(1 << k for k, m in enumerate(metric) if m == -1)
    nul = sum(1 << k for k, m in enumerate(metric) if m == 0)
    sp = T.stream.cuda_stream
    c = torch.empty_like(a)
    ga = torch.empty_like(a)
    gb = torch.empty_like(a)
    res = {}
    for op in ops:
        code = {"geom": 0, "wedge": 1, "inner": 2, "lc": 3, "rc": 4, "regressive": 5}[op]
        fms = T.kernel_ms(lambda: lib.clf_product_fwd(code, n, neg, nul, a.data_ptr(), b.data_ptr(), c.data_ptr(),
                                                      B, sp))
        entry = {"fwd_ms": fms}
        nt = n_terms(op, metric)
        flops = 2.0 * nt * B
        byts = 12.0 * D * B
        if not fwd_only:
            bms = T.kernel_ms(lambda: lib.clf_product_bwd(code, n, neg, nul, a.data_ptr(), b.data_ptr(),
                                                          gc.data_ptr(), ga.data_ptr(), gb.data_ptr(), B, sp))
            entry["bwd_ms"] = bms
            flops += 4.0 * nt * B
            byts += 20.0 * D * B
        t = (entry["fwd_ms"] + entry.get("bwd_ms", 0.0)) * 1e-3
        # The reference's nonzero sigma terms over the time. The masked products
        # run per-term kernels, so there it is their VALU rate (with its
        # fraction of the FP32 peak). The geometric product is served by the
        # matrix-representation kernels where the signature has one, which do
        # other (fewer or more) multiply-adds: there the figure only says how
        # fast the per-term formulation would have to run, and gets no
        # fraction of peak; the per-term kernels' own rate is per_term_path.
        entry.update({"pairs_per_s": B / t, "hbm_gbs_algorithmic": byts / t / 1e9,
                      "frac_hbm": byts / t / 1e9 / PEAK_HBM_GBS})
        if op == "geom":
            entry["term_count_equivalent_tflops"] = flops / t / 1e12
        else:
            entry.update({"tflops_algorithmic": flops / t / 1e12, "frac_fp32_peak": flops / t / 1e12 / PEAK_FP32_TFLOPS})
        if op == "geom":
            # the per-term kernels at the same shape (the path of every other op)
            with path_switch("CLF_GEOM_PATH", "direct"):
                dfms = T.kernel_ms(lambda: lib.clf_product_fwd(code, n, neg, nul, a.data_ptr(), b.data_ptr(),
                                                               c.data_ptr(), B, sp))
                dbms = 0.0
                if not fwd_only:
                    dbms = T.kernel_ms(lambda: lib.clf_product_bwd(code, n, neg, nul, a.data_ptr(), b.data_ptr(),
                                                                   gc.data_ptr(), ga.data_ptr(), gb.data_ptr(), B,
                                                                   sp))
            dt = (dfms + dbms) * 1e-3
            entry["per_term_path"] = {"fwd_ms": dfms, "bwd_ms": dbms, "pairs_per_s": B / dt,
                                      "valu_frac": flops / dt / 1e12 / PEAK_FP32_TFLOPS}
        if not args.no_cpu:
            rows = max(1, min(256, (1 << 16) >> n))  # bounded: 256 rows at n = 8, 64 at n = 10
            CPU_JOBS.append((entry, "cpu_baseline",
                             lambda op=op, rows=rows: cpu_product(op, metric, rows, fwd_only, args.cpu_seconds / 5)))
        res[op] = entry
    return {"workload": name, "metric": metric, "batch": B, "results": res}


def c3_layer(args, torch, cc, lib, T):
    n, B = 8, 262144
    D = 1 << n
    dev = torch.device("cuda", 0)
    cl = cc.CliffordAlgebra([1] * n, device=dev)
    layer = cc.GeometricProductLayer(cl)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, D, generator=g).to(dev).requires_grad_()
    with torch.no_grad():
        layer.weight.copy_((0.25 * torch.randn(1, D, generator=g)).to(dev))
    gy = torch.ones(B, D, device=dev)

    def step():
        y = layer(x)
        return torch.autograd.grad(y, (x, layer.weight), gy)

    steps = max(args.steps, MIN_SHORT_STEPS)
    ms = T.step_ms(step, max(args.warmup, MIN_SHORT_WARMUP), steps)
    flops = 6.0 * D * D * B
    byts = 20.0 * D * B
    sp = T.stream.cuda_stream
    nb = lib.clf_product_bcast_ws_bytes(n, B)
    ws = torch.empty(nb // 4, device=dev)
    y = torch.empty_like(x)
    gx = torch.empty_like(x)
    gw = torch.empty(D, device=dev)
    w = layer.weight.detach()
    def fwd():
        lib.clf_product_bcast_fwd(0, 0, n, 0, 0, x.data_ptr(), w.data_ptr(), y.data_ptr(), B, ws.data_ptr(), nb, sp)

    def bwd():
        lib.clf_product_bcast_bwd(0, 0, n, 0, 0, x.data_ptr(), w.data_ptr(), gy.data_ptr(), gx.data_ptr(),
                                  gw.data_ptr(), B, ws.data_ptr(), nb, sp)

    # served path: Cl(8,0) = M_16(R), phi(y) = phi(x) phi(w) per row
    # (rep16_bcast_* kernels); the GEMM against the weight's 256 x 256 matrix
    # (the path of the other layer ops and signatures) forced for comparison
    fms, bms = T.kernel_ms(fwd), T.kernel_ms(bwd)
    with path_switch("CLF_GEOM_PATH", "direct"):
        gfms, gbms = T.kernel_ms(fwd), T.kernel_ms(bwd)
    fwd_bytes, bwd_bytes = 8.0 * D * B, 12.0 * D * B  # x, y; x, gy, gx
    return {"workload": "c3: GeometricProductLayer Cl(8,0) fwd+bwd (x and weight grads)", "batch": B,
            "ms_per_step": ms, "timed_steps": steps, "rows_per_s": B / (ms * 1e-3),
            "path": "matrix representation (rep16_bcast_fwd/bwd_kernel), HBM-bound",
            "bcast_fwd_ms": fms, "bcast_bwd_ms": bms,
            "bcast_fwd_frac_hbm": fwd_bytes / (fms * 1e-3) / 1e9 / PEAK_HBM_GBS,
            "bcast_bwd_frac_hbm": bwd_bytes / (bms * 1e-3) / 1e9 / PEAK_HBM_GBS,
            # the dense-contraction count (2 D^2 flops per row forward, 4 D^2
            # backward) over the step: an equivalent rate, not a utilisation
            "dense_contraction_equivalent_tflops": flops / (ms * 1e-3) / 1e12,
            "gemm_path": {"fwd_ms": gfms, "bwd_ms": gbms,
                          "fwd_frac_mfma": 2.0 * D * D * B / (gfms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS,
                          "bwd_frac_mfma": 4.0 * D * D * B / (gbms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS,
                          "frac_mfma": 6.0 * D * D * B / ((gfms + gbms) * 1e-3) / 1e12 / PEAK_FP32_TFLOPS},
            "hbm_gbs_algorithmic": byts / (ms * 1e-3) / 1e9, "cpu_baseline": None}


# The reference's published table (NVIDIA A100, figures/tables.md:6-54; the
# minimum over its kernel variants per cell), for context beside the MI355X
# numbers measured the same way: {op: {n: us}} at batch 64, and the geometric
# product at batch 1 and 16.
A100_US = {
    "fwd": {64: {"geom": [17.3, 21.0, 34.3, 79.8, 254.9, 970.7], "wedge": [14.5, 18.0, 24.1, 41.3, 90.6, 245.5],
                 "inner": [14.7, 18.2, 24.4, 44.1, 104.8, 286.9], "lc": [14.2, 17.2, 22.0, 36.8, 79.5, 228.3],
                 "rc": [14.1, 18.7, 21.6, 36.6, 81.2, 225.9],
                 "regressive": [23.9, 28.3, 38.1, 72.0, 163.8, 275.6],
                 "rotor_apply": [24.8, 28.9, 34.6, 45.0, 49.3, 102.9]},
            1: {"geom": [15.5, 15.7, 16.1, 19.6, 31.8, 55.8]}, 16: {"geom": [16.0, 17.1, 20.7, 32.2, 74.1, 242.1]}},
    "bwd": {64: {"geom": [71.4, 72.3, 81.4, 159.7, 528.8, 1983.6], "wedge": [79.0, 82.1, 85.1, 137.2, 371.9, 1331.2],
                 "inner": [78.9, 77.7, 89.9, 178.6, 466.2, 1638.8], "lc": [77.1, 78.9, 84.9, 143.7, 403.1, 1334.3],
                 "rc": [78.1, 53.7, 83.2, 143.5, 401.9, 1330.8],
                 "regressive": [89.1, 89.1, 93.8, 166.9, 429.3, 1374.7]},
            1: {"geom": [72.5, 72.0, 72.5, 72.9, 69.7, 132.5]}, 16: {"geom": [72.0, 71.5, 72.1, 81.0, 153.9, 514.5]}},
}


def published(args, torch, cc, lib, T):
    """The reference's published latency table, measured the way its harness
    does (benchmark/_harness.py:41-50,98-145): Cl(n,0), n = 7..12, batch 1, 16,
    64, a, b ~ N(0,1) on the GPU; the clock warmed with 2 s of matmuls; every
    call synchronised before and after and timed with the wall clock; 25
    untimed calls, then the median over 10 trials of the mean of 10 calls.
    Forward rows time the product call; backward rows build the forward graph
    outside the timer and time torch.autograd.grad(c, (a, b), gc) with a seeded
    N(0,1) gc (bench_geom_prod_bwd.py); the rotor row times apply_rotor(cs, x)
    with cs compiled outside the timer (bench_rotor_apply.py). Each cell also
    carries the device time of the same call (HIP events over 100 back-to-back
    calls). A control row times torch's own elementwise `a * b` the same way
    (forward and autograd.grad): at these sizes every cell is bounded below by
    the host's synchronisation and autograd-engine hand-off costs, which vary
    from box to box, and the control measures them in the same run."""
    import statistics
    dev = torch.device("cuda", 0)
    a0 = torch.randn(4096, 4096, device=dev)
    b0 = torch.randn(4096, 4096, device=dev)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < 2.0:
        a0 = a0 @ b0
    torch.cuda.synchronize()
    del a0, b0

    def harness_us(time_one, warmup=25, iters=10, trials=10):
        for _ in range(warmup):
            time_one()
        ts = []
        for _ in range(trials):
            acc = 0.0
            for _ in range(iters):
                acc += time_one()
            ts.append(acc / iters * 1e6)
        return statistics.median(ts)

    def sync_timed(fn):
        def one():
            torch.cuda.synchronize()
            t = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            return time.perf_counter() - t
        return one

    def bwd_timed(fwd, inputs, gc):
        def one():
            torch.cuda.synchronize()
            c = fwd()
            torch.cuda.synchronize()
            t = time.perf_counter()
            torch.autograd.grad(c, inputs, gc)
            torch.cuda.synchronize()
            return time.perf_counter() - t
        return one

    def device_us(fn, reps=100):
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(T.stream)
        for _ in range(reps):
            fn()
        e1.record(T.stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3

    ops = ["geom", "wedge", "inner", "lc", "rc", "regressive", "torch_mul"]
    table = {"fwd": {}, "bwd": {}}
    g = torch.Generator().manual_seed(0)
    for n in range(7, 13):
        D = 1 << n
        cl = cc.CliffordAlgebra([1] * n, device=dev)
        meth = {"geom": cl.geom_prod, "wedge": cl.wedge_prod, "inner": cl.inner_prod, "lc": cl.left_contraction,
                "rc": cl.right_contraction, "regressive": cl.regressive_prod, "torch_mul": lambda x, y: x * y}
        for B in (1, 16, 64):
            a = torch.randn(B, D, generator=g).to(dev).requires_grad_()
            b = torch.randn(B, D, generator=g).to(dev).requires_grad_()
            gc = torch.randn(B, D, generator=g).to(dev)
            for op in ops:
                f = meth[op]
                cell_f = table["fwd"].setdefault(op, {}).setdefault(str(n), {})
                cell_b = table["bwd"].setdefault(op, {}).setdefault(str(n), {})
                with torch.no_grad():
                    fus = harness_us(sync_timed(lambda: f(a, b)))
                    fdev = device_us(lambda: f(a, b))
                bus = harness_us(bwd_timed(lambda: f(a, b), (a, b), gc))
                c = f(a, b)
                bdev = device_us(lambda: torch.autograd.grad(c, (a, b), gc, retain_graph=True))
                cell_f[str(B)] = {"us": round(fus, 2), "device_us": round(fdev, 2)}
                cell_b[str(B)] = {"us": round(bus, 2), "device_us": round(bdev, 2)}
            biv = torch.randn(1, n * (n - 1) // 2, generator=g).to(dev)
            x = torch.randn(B, D, generator=g).to(dev)
            with torch.no_grad():
                cs = cl.compile_bivector(biv)
                rus = harness_us(sync_timed(lambda: cl.apply_rotor(cs, x)))
                rdev = device_us(lambda: cl.apply_rotor(cs, x))
            table["fwd"].setdefault("rotor_apply", {}).setdefault(str(n), {})[str(B)] = {
                "us": round(rus, 2), "device_us": round(rdev, 2)}
        print(f"[published] n={n} done", file=sys.stderr, flush=True)
    return {"workload": "published: the reference's latency table (Cl(n,0), n = 7..12, batch 1/16/64), "
                        "harness-style sync-timed wall clock, median of 10 x 10 after 25 warmups",
            "unit": "us", "table": table,
            "reference_a100_us_context": {"note": "NVIDIA A100 numbers published by the reference "
                                                  "(figures/tables.md:6-54), different hardware: context only",
                                          "n": list(range(7, 13)), **A100_US}}


def cpu_layer(budget_s):
    import torch
    from oracle import clifford_oracle as O
    rows = 256
    g = torch.Generator().manual_seed(0)
    x = torch.randn(rows, 256, generator=g).requires_grad_()
    w = (0.25 * torch.randn(1, 256, generator=g)).requires_grad_()

    def work():
        y = O.layer_forward("geom", x, w, [1] * 8)
        torch.autograd.grad(y, (x, w), torch.ones_like(y))

    return cpu_rate(work, rows, budget_s, "GeometricProductLayer Cl(8,0) fwd+bwd (x and weight grads)")


def cpu_rotor(budget_s):
    import torch
    from oracle import clifford_oracle as O
    rows = 256
    g = torch.Generator().manual_seed(0)
    biv = ((0.1 ** 0.5) * torch.randn(1, 28, generator=g)).double().requires_grad_()
    x = torch.randn(rows, 256, generator=g).double().requires_grad_()

    def work():
        y = O.apply_bivector(biv, x, 8)
        torch.autograd.grad(y, (x, biv), torch.ones_like(y))

    return cpu_rate(work, rows, budget_s, "RotorLayer n = 8 fwd+bwd, rotor recompiled per chunk", "fp64")


def c4_rotor(args, torch, cc, lib, T):
    n, B = 8, 131072
    D = 1 << n
    dev = torch.device("cuda", 0)
    cl = cc.CliffordAlgebra([1] * 7 + [-1], device=dev)
    layer = cc.RotorLayer(cl).train()
    g = torch.Generator().manual_seed(0)
    with torch.no_grad():
        layer.bivector.copy_(((0.1 ** 0.5) * torch.randn(1, 28, generator=g)).to(dev))
    x = torch.randn(B, D, generator=g).to(dev).requires_grad_()
    gy = torch.ones(B, D, device=dev)

    def step():
        y = layer(x)
        return torch.autograd.grad(y, (x, layer.bivector), gy)

    steps = max(args.steps, MIN_SHORT_STEPS)
    ms = T.step_ms(step, max(args.warmup, MIN_SHORT_WARMUP), steps)
    sp = T.stream.cuda_stream
    from cliffordcuda_amd import rotor as rotor_mod
    state = rotor_mod._compile_fwd(layer.bivector.detach().reshape(-1), n)
    y = torch.empty_like(x)
    gx = torch.empty_like(x)
    gs = torch.empty_like(state)
    nb = lib.clf_rotor_apply_ws_bytes(n, B)
    ws = torch.empty(max(4, nb) // 4, device=dev)
    biv = layer.bivector.detach()
    cms = T.kernel_ms(lambda: lib.clf_rotor_compile_fwd(n, biv.data_ptr(), state.data_ptr(), None, sp))
    fms = T.kernel_ms(lambda: lib.clf_rotor_apply_fwd(n, state.data_ptr(), x.data_ptr(), y.data_ptr(), B, sp))
    bms = T.kernel_ms(lambda: lib.clf_rotor_apply_bwd(n, state.data_ptr(), x.data_ptr(), gy.data_ptr(),
                                                      gx.data_ptr(), gs.data_ptr(), B, ws.data_ptr(), nb, sp))
    # the same entry points on the register plane-rotation chain (the n = 8
    # default is the Cl(8,0) representation on the matrix cores)
    with path_switch("CLF_ROTOR_PATH", "chain"):
        cfms = T.kernel_ms(lambda: lib.clf_rotor_apply_fwd(n, state.data_ptr(), x.data_ptr(), y.data_ptr(), B, sp))
        cbms = T.kernel_ms(lambda: lib.clf_rotor_apply_bwd(n, state.data_ptr(), x.data_ptr(), gy.data_ptr(),
                                                           gx.data_ptr(), gs.data_ptr(), B, ws.data_ptr(), nb, sp))
    byts = 20.0 * D * B
    return {"workload": "c4: RotorLayer train Cl(7,1) fwd+bwd (rotor recompiled each step)", "batch": B,
            "path": "Cl(8,0) representation, MFMA (rotor16 kernels)",
            "chain_path": {"apply_fwd_ms": cfms, "apply_bwd_ms": cbms},
            "ms_per_step": ms, "timed_steps": steps, "rows_per_s": B / (ms * 1e-3),
            "hbm_gbs_algorithmic": byts / (ms * 1e-3) / 1e9, "frac_hbm": byts / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
            "compile_fwd_ms": cms, "apply_fwd_ms": fms, "apply_bwd_ms": bms,
            "apply_fwd_frac_hbm": 8.0 * D * B / (fms * 1e-3) / 1e9 / PEAK_HBM_GBS,
            "apply_bwd_frac_hbm": 12.0 * D * B / (bms * 1e-3) / 1e9 / PEAK_HBM_GBS, "cpu_baseline": None}


def c5_degenerate(args, torch, cc, lib, T):
    metric = (1,) * 9 + (0,)
    B = 16384
    out = products_config(args, torch, cc, lib, T, "c5: Cl(9,0,1) geom + lc fwd+bwd", metric, B, ["geom", "lc"])
    dev = torch.device("cuda", 0)
    n = 10
    x = torch.randn(B, 1 << n, device=dev)
    o = torch.empty(B, device=dev)
    y = torch.empty_like(x)
    sp = T.stream.cuda_stream
    ns = T.kernel_ms(lambda: lib.clf_norm_sq_fwd(n, 0, 1 << 9, x.data_ptr(), o.data_ptr(), B, sp))
    gp = T.kernel_ms(lambda: lib.clf_graded(3, n, 0, 1 << 9, 2, x.data_ptr(), y.data_ptr(), B, sp))
    D = 1 << n
    out["norm_sq_fwd"] = {"ms": ns, "frac_hbm": (4.0 * D + 4) * B / (ns * 1e-3) / 1e9 / PEAK_HBM_GBS}
    out["grade_projection_fwd"] = {"ms": gp, "frac_hbm": 8.0 * D * B / (gp * 1e-3) / 1e9 / PEAK_HBM_GBS}
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1. The multi-GPU design "
                                   "(batch sharding + one small all-reduce) is described, not built."}))
        sys.exit(2)
    import torch
    import cliffordcuda_amd as cc
    from cliffordcuda_amd import _lib
    torch.cuda.set_device(0)
    lib = _lib.load()
    T = Timer(torch, torch.cuda.current_stream(0), max(5, args.steps))
    T.clock = Clock(torch, lib, T.stream)
    if args.workload == "headline":
        print(json.dumps(headline(args, torch, cc, lib, T)))
        return
    if args.workload == "copycal":
        # plain device copy of a known size: calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE
        nbytes = 256 << 20
        x = torch.ones(nbytes // 4, device="cuda")
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        ms = T.kernel_ms(lambda: y.copy_(x))
        # torch's elementwise add over the headline shape: the byte pattern of
        # the forward product (read two 256 MiB operands, write one)
        z = torch.empty_like(x)
        ams = T.kernel_ms(lambda: torch.add(x, y, out=z))
        # the same add at the per-operand sizes of C2 (32 MiB) and C5 (64 MiB):
        # three such arrays fit in the 256 MB last-level cache (MALL), so the
        # back-to-back launches run above the HBM rate
        by_size = {}
        for mib in (32, 64, 128, 256):
            k = (mib << 20) // 4
            xs, ys, zs = x[:k], y[:k], z[:k]
            t = T.kernel_ms(lambda: torch.add(xs, ys, out=zs))
            by_size[str(mib)] = {"add_us": t * 1e3, "add_gbs": 3.0 * (mib << 20) / (t * 1e-3) / 1e9}
        # clf_stream_probe: the product kernels' byte patterns without their
        # arithmetic, plain and nontemporal, 256 MiB per operand
        w = torch.empty_like(x)
        v = torch.empty_like(x)
        sp = T.stream.cuda_stream
        probe = {}
        for nin, nout, label in ((3, 2, "backward 3r+2w"), (2, 1, "forward 2r+1w"), (1, 1, "copy 1r+1w")):
            for ntv in (1, 0):
                t = T.kernel_ms(lambda: lib.clf_stream_probe(nin, nout, x.data_ptr(), y.data_ptr(), z.data_ptr(),
                                                             w.data_ptr(), v.data_ptr(), nbytes // 4, ntv, sp))
                probe[f"{label} {'nontemporal' if ntv else 'plain'}"] = {
                    "us": t * 1e3, "gbs": (nin + nout) * nbytes / (t * 1e-3) / 1e9}
        print(json.dumps({"workload": "copycal", "bytes_read_per_copy": nbytes, "bytes_written_per_copy": nbytes,
                          "stream_probe_256mib": probe,
                          "copy_ms": ms, "copy_gbs": 2.0 * nbytes / (ms * 1e-3) / 1e9,
                          "add_ms": ams, "add_gbs": 3.0 * nbytes / (ams * 1e-3) / 1e9,
                          "add_by_operand_mib": by_size}))
        return
    if args.workload == "published":
        print(json.dumps(published(args, torch, cc, lib, T)))
        return
    runs = ["c1", "c2", "c3", "c4", "c5"] if args.workload == "all" else [args.workload]
    out = []
    for w in runs:
        if w == "c1":
            r = products_config(args, torch, cc, lib, T, "c1: Cl(5,0) geom fwd", (1,) * 5, 1024, ["geom"], True)
        elif w == "c2":
            r = products_config(args, torch, cc, lib, T, "c2: Cl(6,1) six products fwd+bwd", (1,) * 6 + (-1,), 65536,
                                ["geom", "wedge", "inner", "lc", "rc", "regressive"])
        elif w == "c3":
            r = c3_layer(args, torch, cc, lib, T)
            if not args.no_cpu:
                CPU_JOBS.append((r, "cpu_baseline", lambda: cpu_layer(args.cpu_seconds / 3)))
        elif w == "c4":
            r = c4_rotor(args, torch, cc, lib, T)
            if not args.no_cpu:
                CPU_JOBS.append((r, "cpu_baseline", lambda: cpu_rotor(args.cpu_seconds / 3)))
        else:
            r = c5_degenerate(args, torch, cc, lib, T)
        out.append(r)
    for d, key, job in CPU_JOBS:
        d[key] = job()
    for r in out:
        print(json.dumps(r), flush=True)


if __name__ == "__main__":
    main()
