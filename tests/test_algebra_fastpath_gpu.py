"""CliffordAlgebra's product methods test the usual call (plain 2-D
contiguous fp32 tensors of the algebra's row length, device and one shape) in
one expression and then launch with a plan cached per op. After the first call
has cached the plan: results and gradients equal the generic entry's bit for
bit, other tensors (a Parameter, a batch of rows from a larger tensor) still
work, and every bad argument raises the reference's exception with its message
(the same checks in the same order as the first call)."""
import pytest
import torch

import cliffordcuda_amd as cc
from cliffordcuda_amd import products as P

pytestmark = pytest.mark.gpu

OPS = [("geom_prod", "geom"), ("wedge_prod", "wedge"), ("inner_prod", "inner"), ("left_contraction", "lc"),
       ("right_contraction", "rc"), ("regressive_prod", "regressive")]


@pytest.mark.parametrize("meth,op", OPS)
def test_fast_path_equals_generic_entry(meth, op):
    metric = (1,) * 6 + (-1,)
    cl = cc.CliffordAlgebra(list(metric), device="cuda")
    f = getattr(cl, meth)
    g = torch.Generator().manual_seed(7)
    a, b, gc = [torch.randn(37, 128, generator=g).cuda() for _ in range(3)]
    print(f"[case] fast path {op}", flush=True)
    f(a, b)  # first call: full checks, caches the plan
    assert op in cl._plans
    with torch.no_grad():
        assert torch.equal(f(a, b), P.product(op, a, b, metric))
    x = a.clone().requires_grad_()
    y = b.clone().requires_grad_()
    c = f(x, y)
    ga, gb = torch.autograd.grad(c, (x, y), gc)
    x2 = a.clone().requires_grad_()
    y2 = b.clone().requires_grad_()
    c2 = P.product(op, x2, y2, metric)
    ga2, gb2 = torch.autograd.grad(c2, (x2, y2), gc)
    for u, v in ((c, c2), (ga, ga2), (gb, gb2)):
        assert torch.equal(u.detach(), v.detach())
    # a Parameter and rows of a larger tensor
    p = torch.nn.Parameter(a.clone())
    assert torch.equal(f(p, b).detach(), P.product(op, a, b, metric))
    big = torch.randn(80, 128, generator=g).cuda()
    assert torch.equal(f(big[5:42], b), P.product(op, big[5:42].contiguous(), b, metric))


def test_bad_arguments_after_cached_plan_raise_reference_errors():
    cl = cc.CliffordAlgebra([1] * 7, device="cuda")
    a = torch.randn(4, 128, device="cuda")
    cl.geom_prod(a, a)
    assert "geom" in cl._plans
    cases = [
        ((a.double(), a), "a dtype"),
        ((a, a[:, :64]), "b last dim"),
        ((a.reshape(2, 2, 128), a), "a must be 2D"),
        ((a.cpu(), a), "a on device"),
        ((a, torch.randn(128, 4, device="cuda").t()), "b must be contiguous"),
        ((a, [1.0] * 128), "b must be a torch.Tensor"),
    ]
    for (x, y), msg in cases:
        with pytest.raises(ValueError, match=msg):
            cl.geom_prod(x, y)
    with pytest.raises(RuntimeError, match="shapes differ"):
        cl.geom_prod(a, a[:3])
    cl0 = cc.CliffordAlgebra([1] * 6 + [0], device="cuda")
    z = torch.randn(2, 128, device="cuda")
    for _ in range(2):
        with pytest.raises(ValueError, match="regressive_prod is undefined for degenerate metrics"):
            cl0.regressive_prod(z, z)
    assert "regressive" not in cl0._plans
