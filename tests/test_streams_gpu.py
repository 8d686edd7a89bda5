"""Stream and thread behaviour of the ops: every launch goes to the caller's
current stream (a side stream that is still busy with a long matmul when the
inputs are written and the op is called gives the right answer only if the op
runs after them on that stream), and concurrent callers on their own streams
in several threads get the same results as serial calls (the C ABI's tables
are built once under a lock and are read-only afterwards)."""
import threading

import pytest
import torch

import cliffordcuda_amd as cc

pytestmark = pytest.mark.gpu


def _ops(cl, n):
    """(name, fn(x, y) -> tuple of tensors) over the hot path's op families."""
    layer = cc.GeometricProductLayer(cl).cuda()
    with torch.no_grad():
        layer.weight.copy_(torch.linspace(-1.0, 1.0, 1 << n, device="cuda").view(1, -1))
    biv = torch.linspace(-0.3, 0.4, n * (n - 1) // 2, device="cuda").view(1, -1)

    def products(x, y):
        xr, yr = x.clone().requires_grad_(), y.clone().requires_grad_()
        outs = [cl.geom_prod(xr, yr), cl.wedge_prod(xr, yr), cl.inner_prod(xr, yr), cl.left_contraction(xr, yr)]
        gx, gy = torch.autograd.grad(sum(o.sum() for o in outs), (xr, yr))
        return tuple(o.detach() for o in outs) + (gx, gy)

    def graded(x, y):
        return cl.reverse(x), cl.grade_projection(y, 2), cl.norm_sq(x)

    def layer_fn(x, y):
        return (layer(x).detach(),)

    def rotor(x, y):
        return (cl.apply_bivector(biv, x),) if n >= 7 else ()

    return [("products", products), ("graded", graded), ("layer", layer_fn), ("rotor", rotor)]


@pytest.mark.parametrize("metric", [(1,) * 8, (1,) * 6 + (-1,), (1,) * 4 + (0,)],
                         ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[v] for v in m))
def test_ops_follow_the_current_stream(metric):
    n = len(metric)
    cl = cc.CliffordAlgebra(metric, device="cuda")
    g = torch.Generator().manual_seed(7)
    src_x = torch.randn(4099, 1 << n, generator=g).cuda()
    src_y = torch.randn(4099, 1 << n, generator=g).cuda()
    big = torch.randn(4096, 4096, device="cuda")
    for name, fn in _ops(cl, n):
        ref = fn(src_x, src_y)
        torch.cuda.synchronize()
        print(f"[case] stream metric={metric} op={name}", flush=True)
        side = torch.cuda.Stream()
        x = torch.zeros_like(src_x)
        y = torch.zeros_like(src_y)
        torch.cuda.synchronize()
        with torch.cuda.stream(side):
            for _ in range(4):  # keeps the side stream busy for milliseconds
                big = (big @ big) * 1e-3
            x.copy_(src_x)
            y.copy_(src_y)
            got = fn(x, y)
        side.synchronize()
        for u, v in zip(got, ref):
            assert torch.equal(u, v), name


def test_concurrent_callers_on_their_own_streams():
    metrics = [(1,) * 8, (1,) * 6 + (-1,), (1,) * 9 + (0,), (1, 1, 1, 1, 0, -1)]
    jobs = []
    for k, metric in enumerate(metrics):
        n = len(metric)
        g = torch.Generator().manual_seed(k)
        a = torch.randn(1031, 1 << n, generator=g).cuda()
        b = torch.randn(1031, 1 << n, generator=g).cuda()
        jobs.append((metric, a, b))

    def run(metric, a, b):
        cl = cc.CliffordAlgebra(metric, device="cuda")
        ar, br = a.clone().requires_grad_(), b.clone().requires_grad_()
        c = cl.geom_prod(ar, br) + cl.left_contraction(ar, br)
        ga, gb = torch.autograd.grad(c.sum(), (ar, br))
        return c.detach(), ga, gb

    refs = [run(*j) for j in jobs]
    torch.cuda.synchronize()
    results = [None] * len(jobs)
    errors = []

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                outs = [run(*jobs[i]) for _ in range(5)]
            s.synchronize()
            results[i] = outs
        except Exception as e:  # reported below, on the main thread
            errors.append(repr(e))

    print("[case] concurrent callers", flush=True)
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(jobs))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    for i, outs in enumerate(results):
        assert outs is not None
        for out in outs:
            for u, v in zip(out, refs[i]):
                assert torch.equal(u, v), metrics[i]
