"""The rotor chain with one wave per row (2^(n-6) floats per lane; n = 9 up
to 12288 rows, n = 10 and 11 always, n = 12 above 768 rows). Every element
gets the same operations in every layout (y_I = fma(c, x_I, (-+s) x_J), exact
identities on the lanes a plane does not touch), so the same rows equal, bit
for bit, across layouts: at n = 9 rows alone (wave rows) against a batch of
12300 (64 floats on 8 lanes per row), at n = 12 rows alone (the LDS-staged
chain) against a batch of 1100 (wave rows). At n = 10, 11 both batches run on
wave rows: rows alone equal their rows in the batch (other grid) bit for bit,
and the fp64 oracle chain within 1e-5. Forward and transposed (the x gradient
through a rotor that needs no gradient)."""
import pytest
import torch

import cliffordcuda_amd as cc
from oracle import clifford_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-5


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = float(ref.abs().max())
    return float((got - ref).abs().max()) / (den if den > 0 else 1.0)


@pytest.mark.parametrize("n,B", [(9, 12300), (10, 1100), (11, 1100), (12, 1100)])
def test_wave_row_chain_across_layouts(n, B):
    cl = cc.CliffordAlgebra([1] * (n - 1) + [-1], device="cuda")
    g = torch.Generator().manual_seed(40 + n)
    biv = (0.3 * torch.randn(1, n * (n - 1) // 2, generator=g)).cuda()
    x = torch.randn(B, 1 << n, generator=g).cuda()
    gy = torch.randn(B, 1 << n, generator=g).cuda()
    rows = torch.tensor([0, 1, 517, B - 1], device="cuda")
    print(f"[case] rotor wave rows n={n} B={B}", flush=True)
    with torch.no_grad():
        cs = cl.compile_bivector(biv)
        y_big = cl.apply_rotor(cs, x)
        y_small = cl.apply_rotor(cs, x[rows].contiguous())
    assert torch.equal(y_big[rows], y_small)
    xb = x.clone().requires_grad_()
    (gx_big,) = torch.autograd.grad(cl.apply_rotor(cs, xb), (xb,), gy)
    xs = x[rows].clone().requires_grad_()
    (gx_small,) = torch.autograd.grad(cl.apply_rotor(cs, xs), (xs,), gy[rows].contiguous())
    assert torch.equal(gx_big[rows], gx_small)
    if n in (10, 11):
        cs64 = cs.detach().double().cpu()
        x64 = x[rows].double().cpu().requires_grad_()
        y64 = O.givens_chain_apply(cs64, x64, n)
        (gx64,) = torch.autograd.grad(y64, (x64,), gy[rows].double().cpu())
        assert rel_err(y_small, y64) <= TOL
        assert rel_err(gx_small, gx64) <= TOL
