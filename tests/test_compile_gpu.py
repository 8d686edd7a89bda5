"""torch.compile over the public API: with fullgraph=True any graph break is an
error, so these tests show that products, graded ops, norm_sq, the product
layers and the rotor layer trace as single graphs (through the operators of
cliffordcuda_amd/_ops.py); values and gradients equal the eager path. The
aot_eager backend generates no code of its own, so only this library's
kernels run. torch.library.opcheck checks each operator's schema, fake
implementation and autograd registration."""
import pytest
import torch

import cliffordcuda_amd as cc

pytestmark = pytest.mark.gpu
TOL = 1e-5


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = float(ref.abs().max())
    return float((got - ref).abs().max()) / (den if den > 0 else 1.0)


def test_compile_products_and_graded_fullgraph():
    torch._dynamo.reset()
    cl = cc.CliffordAlgebra((1,) * 7 + (-1,), device="cuda")
    g = torch.Generator().manual_seed(0)
    a0 = torch.randn(33, 256, generator=g).cuda()
    b0 = torch.randn(33, 256, generator=g).cuda()

    def f(a, b):
        c = cl.geom_prod(a, b)
        d = cl.wedge_prod(c, b) + cl.left_contraction(a, c)
        return (cl.norm_sq(d) + cl.reverse(c).sum(-1) + cl.grade_projection(d, 2).sum(-1)).sum()

    cf = torch.compile(f, backend="aot_eager", fullgraph=True)
    outs = []
    for fn in (f, cf):
        a = a0.clone().requires_grad_()
        b = b0.clone().requires_grad_()
        loss = fn(a, b)
        loss.backward()
        outs.append((loss.detach(), a.grad, b.grad))
    for u, v in zip(*outs):
        assert rel_err(v, u) <= TOL


def test_compile_layers_fullgraph():
    torch._dynamo.reset()
    cl = cc.CliffordAlgebra((1,) * 8, device="cuda")
    model = torch.nn.Sequential(cc.GeometricProductLayer(cl), cc.RotorLayer(cl), cc.WedgeProductLayer(cl)).train()
    with torch.no_grad():
        model[0].weight.mul_(0.25)
        model[1].bivector.mul_(0.3)
    g = torch.Generator().manual_seed(1)
    x0 = torch.randn(70, 256, generator=g).cuda()
    cm = torch.compile(model, backend="aot_eager", fullgraph=True)
    res = []
    for m in (model, cm):
        model.zero_grad()
        x = x0.clone().requires_grad_()
        y = m(x)
        y.square().sum().backward()
        res.append([y.detach(), x.grad] + [p.grad.clone() for p in model.parameters()])
    for u, v in zip(*res):
        assert rel_err(v, u) <= TOL


def test_compile_rotor_cs_fullgraph():
    """The reference's explicit composition apply_rotor(compile_bivector(b), x)
    traces as one graph (the cs operators) and gives the eager values and
    gradients to the bivector and x."""
    cl = cc.CliffordAlgebra([1] * 8, device="cuda")
    g = torch.Generator().manual_seed(5)
    b0 = (0.3 * torch.randn(1, 28, generator=g)).cuda()
    x0 = torch.randn(33, 256, generator=g).cuda()
    gy = torch.randn(33, 256, generator=g).cuda()   # (a rotation-invariant loss would have no bivector gradient)

    def f(b, x):
        return cl.apply_rotor(cl.compile_bivector(b), x)

    res = []
    for fn in (f, torch.compile(f, fullgraph=True)):
        b = b0.clone().requires_grad_()
        x = x0.clone().requires_grad_()
        y = fn(b, x)
        y.backward(gy)
        res.append([y.detach(), b.grad, x.grad])
    for u, v in zip(*res):
        assert rel_err(v, u) <= TOL


@pytest.mark.parametrize("case", ["product", "graded", "norm_sq", "bcast_product", "rotor", "rotor_cs"])
def test_opcheck(case):
    ops = torch.ops.cliffordcuda_amd
    g = torch.Generator().manual_seed(2)
    x = torch.randn(9, 256, generator=g).cuda().requires_grad_()
    y = torch.randn(9, 256, generator=g).cuda().requires_grad_()
    w = torch.randn(1, 256, generator=g).cuda().requires_grad_()
    if case == "product":
        torch.library.opcheck(ops.product.default, (x, y, 0, 8, 0, 0))
    elif case == "graded":
        torch.library.opcheck(ops.graded.default, (x, 4, 8, 0, 0, 0))   # dual
    elif case == "norm_sq":
        torch.library.opcheck(ops.norm_sq.default, (x, 8, 0, 0))
    elif case == "bcast_product":
        torch.library.opcheck(ops.bcast_product.default, (x, w, 2, 0, 8, 0, 0))
    elif case == "rotor":
        biv = (0.3 * torch.randn(28, generator=g)).cuda().requires_grad_()
        torch.library.opcheck(ops.rotor_compile.default, (biv, 8))
        state = ops.rotor_compile(biv.detach(), 8)
        torch.library.opcheck(ops.rotor_apply.default, (state.requires_grad_(), x, 8))
    else:
        biv = (0.3 * torch.randn(28, generator=g)).cuda().requires_grad_()
        torch.library.opcheck(ops.rotor_compile_cs.default, (biv, 8))
        cs = ops.rotor_compile_cs(biv.detach(), 8)
        torch.library.opcheck(ops.rotor_cs_apply.default, (cs.requires_grad_(), x, 8))
