"""64-bit row offsets: batches whose last rows start past float index 2**31
(8 GiB per operand) on every kernel family of the hot path -- the Cl(8,0)
matrix representation, the n = 7 representation, the split representation
(n = 10 with a null generator), the balanced and blocked per-term kernels and
the graded ops. Rows are independent, so the rows of the large batch (first,
middle and last ones) must equal, bit for bit, the same rows computed as a
batch of their own, forward and backward."""
import pytest
import torch

import cliffordcuda_amd as cc

pytestmark = pytest.mark.gpu

# (metric, op, CLF_GEOM_PATH or None); batch = 2**31 / 2**n + 3 rows
CASES = [
    ((1,) * 8, "geom_prod", None),     # rep16 kernels
    ((1,) * 8, "geom_prod", "direct"),  # blocked per-term kernels
    ((1,) * 8, "left_contraction", None),  # balanced kernels
    ((1,) * 6 + (-1,), "geom_prod", None),  # n = 7 representation
    ((1,) * 9 + (0,), "geom_prod", None),  # split representation, fused kernels
]


def _rows(B):
    """The first, middle and last rows plus 2048 more: a sample batch of at
    least 2048 rows runs the same kernels as the large batch (below that the
    n = 8 forward takes the small-batch kernel, which sums a row's partner
    blocks in another order, so its results differ in the last bits)."""
    edge = torch.tensor([0, 1, B // 2, B - 3, B - 2, B - 1])
    return torch.cat([edge, torch.arange(2, 2050)]).cuda()


@pytest.mark.parametrize("metric,op,path", CASES, ids=lambda v: str(v))
def test_rows_past_2_31_floats(metric, op, path, clf_env):
    n = len(metric)
    D = 1 << n
    B = (1 << (31 - n)) + 3
    free, _ = torch.cuda.mem_get_info()
    if free < 7 * B * D * 4 + (4 << 30):
        pytest.skip("needs about 56 GiB of free device memory")
    if path is not None:
        clf_env.setenv("CLF_GEOM_PATH", path)
    print(f"[case] large batch metric={metric} op={op} path={path} B={B}", flush=True)
    cl = cc.CliffordAlgebra(metric, device="cuda")
    fn = getattr(cl, op)
    g = torch.Generator(device="cuda").manual_seed(5)
    a = torch.randn(B, D, device="cuda", generator=g).requires_grad_()
    b = torch.randn(B, D, device="cuda", generator=g).requires_grad_()
    gc = torch.randn(B, D, device="cuda", generator=g)
    rows = _rows(B)
    assert (B - 1) * D >= 1 << 31
    c = fn(a, b)
    ga, gb = torch.autograd.grad(c, (a, b), gc)
    big = [t.detach()[rows].clone() for t in (c, ga, gb)]
    del c, ga, gb
    a_s = a.detach()[rows].clone().requires_grad_()
    b_s = b.detach()[rows].clone().requires_grad_()
    c_s = fn(a_s, b_s)
    ga_s, gb_s = torch.autograd.grad(c_s, (a_s, b_s), gc[rows].clone())
    for name, u, v in zip(("c", "ga", "gb"), big, (c_s, ga_s, gb_s)):
        assert torch.equal(u, v.detach()), name
    if path is None and op == "geom_prod" and n == 8:
        # graded ops on the same 8 GiB operand
        x = a.detach()
        rev = cl.reverse(x)[rows]
        nsq = cl.norm_sq(x)[rows]
        xs = x[rows].clone()
        assert torch.equal(rev, cl.reverse(xs))
        assert torch.equal(nsq, cl.norm_sq(xs))
    del a, b, gc
    torch.cuda.empty_cache()


# (layer class, metric): the Cl(8,0) representation layer, the GEMM layer path,
# the rotor on the Cl(8,0) representation and the register plane-rotation chain
LAYER_CASES = [
    ("GeometricProductLayer", (1,) * 8),
    ("WedgeProductLayer", (1,) * 8),
    ("RotorLayer", (1,) * 7 + (-1,)),
    ("RotorLayer", (1,) * 9),
]


@pytest.mark.parametrize("cls,metric", LAYER_CASES, ids=lambda v: str(v))
def test_layer_rows_past_2_31_floats(cls, metric):
    """Layer outputs and input gradients of the large batch's rows equal those
    of the same rows as a batch of their own (the parameter gradients sum over
    the batch and are not compared)."""
    n = len(metric)
    D = 1 << n
    B = (1 << (31 - n)) + 3
    free, _ = torch.cuda.mem_get_info()
    if free < 6 * B * D * 4 + (4 << 30):
        pytest.skip("needs about 52 GiB of free device memory")
    print(f"[case] large batch layer={cls} metric={metric} B={B}", flush=True)
    cl = cc.CliffordAlgebra(metric, device="cuda")
    layer = getattr(cc, cls)(cl).cuda()
    g = torch.Generator(device="cuda").manual_seed(6)
    with torch.no_grad():
        for p in layer.parameters():
            p.copy_(0.2 * torch.randn(p.shape, device="cuda", generator=g))
    x = torch.randn(B, D, device="cuda", generator=g).requires_grad_()
    gy = torch.randn(B, D, device="cuda", generator=g)
    rows = _rows(B)
    y = layer(x)
    (gx,) = torch.autograd.grad(y, (x,), gy)
    big = [t.detach()[rows].clone() for t in (y, gx)]
    del y, gx
    xs = x.detach()[rows].clone().requires_grad_()
    ys = layer(xs)
    (gxs,) = torch.autograd.grad(ys, (xs,), gy[rows].clone())
    for name, u, v in zip(("y", "gx"), big, (ys, gxs)):
        assert torch.equal(u, v.detach()), name
    del x, gy
    torch.cuda.empty_cache()
