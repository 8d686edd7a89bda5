"""HIP graph capture: the library issues no allocation, memset or host sync
inside its calls, so a training-like step (product layer, geometric product,
rotor layer, forward and backward) can be captured with torch.cuda.graph and
replayed. Every replay, with eager work and synchronizations between the
replays, equals the eager step on the same inputs. The loss gradient is passed
in as a tensor (no reduction kernel in the captured region)."""
import pytest
import torch

import cliffordcuda_amd as cc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("metric", [(1,) * 8, (1,) * 7 + (-1,)], ids=["cl80", "cl71"])
def test_graph_replays_match_eager(metric):
    n = len(metric)
    cl = cc.CliffordAlgebra(metric, device="cuda")
    layer = cc.GeometricProductLayer(cl).cuda()
    rot = cc.RotorLayer(cl).cuda().train()
    g = torch.Generator().manual_seed(3)
    with torch.no_grad():
        layer.weight.copy_((0.25 * torch.randn(1, 1 << n, generator=g)).cuda())
        rot.bivector.copy_((0.3 * torch.randn(1, n * (n - 1) // 2, generator=g)).cuda())
    B = 1031
    x = torch.randn(B, 1 << n, generator=g).cuda()
    y = torch.randn(B, 1 << n, generator=g).cuda()
    gout = torch.randn(B, 1 << n, generator=g).cuda()
    inputs = [(torch.randn(B, 1 << n, generator=g).cuda(), torch.randn(B, 1 << n, generator=g).cuda())
              for _ in range(3)]

    def step():
        a = x.detach().requires_grad_()
        out = layer(a) + cl.geom_prod(a, y) + rot(a)
        ga, gw, gbv = torch.autograd.grad(out, (a, layer.weight, rot.bivector), gout)
        return out.detach(), ga, gw, gbv

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step()
    for k, (nx, ny) in enumerate(inputs * 2):
        print(f"[case] graph metric={metric} replay={k}", flush=True)
        x.copy_(nx)
        y.copy_(ny)
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in static]
        eager = step()
        torch.cuda.synchronize()
        for u, v in zip(got, eager):
            assert torch.equal(u, v), k
