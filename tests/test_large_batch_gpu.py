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
    return torch.tensor([0, 1, B // 2, B - 3, B - 2, B - 1], device="cuda")


@pytest.mark.parametrize("metric,op,path", CASES, ids=lambda v: str(v))
def test_rows_past_2_31_floats(metric, op, path, monkeypatch):
    n = len(metric)
    D = 1 << n
    B = (1 << (31 - n)) + 3
    free, _ = torch.cuda.mem_get_info()
    if free < 7 * B * D * 4 + (4 << 30):
        pytest.skip("needs about 56 GiB of free device memory")
    if path is not None:
        monkeypatch.setenv("CLF_GEOM_PATH", path)
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
