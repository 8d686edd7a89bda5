"""GPU parity of the rotor path (compile + sandwich, forward and backward to the
bivector and to x) against the fp64 oracle (Euclidean ~R x R, reference
algebra.py:343-373 semantics). Tolerance 1e-5 normwise, values and gradients."""
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


def oracle_step(biv, x, gy, n):
    b64 = biv.double().requires_grad_()
    x64 = x.double().requires_grad_()
    y64 = O.apply_bivector(b64, x64, n)
    y64.backward(gy.double())
    return y64, b64.grad, x64.grad


@pytest.mark.parametrize("n,metric", [(7, (1,) * 7), (8, (1,) * 7 + (-1,)), (9, (1,) * 9), (10, (1,) * 9 + (0,))])
def test_apply_bivector_parity(n, metric):
    cl = cc.CliffordAlgebra(metric, device="cuda")
    g = torch.Generator().manual_seed(n)
    B = 24 if n < 10 else 6
    biv = (0.1 ** 0.5) * torch.randn(1, n * (n - 1) // 2, generator=g)
    x = torch.randn(B, 1 << n, generator=g)
    gy = torch.randn(B, 1 << n, generator=g)
    bd = biv.cuda().requires_grad_()
    xd = x.cuda().requires_grad_()
    print(f"[case] rotor n={n} B={B}", flush=True)
    y = cl.apply_bivector(bd, xd)
    y.backward(gy.cuda())
    y64, gb64, gx64 = oracle_step(biv, x, gy, n)
    assert rel_err(y, y64) <= TOL
    assert rel_err(xd.grad, gx64) <= TOL
    assert rel_err(bd.grad, gb64) <= TOL


def test_rotor_layer_c4_shape():
    """RotorLayer train mode on Cl(7,1), bivector ~ N(0, 0.1),
    x (131072, 256): full-batch forward + backward against the fp64 oracle.
    The upstream gradient is all ones and y = ~R x R is linear in x, so with
    S = sum_b x_b (fp64): the full-batch bivector gradient equals the oracle's
    bivector gradient on the single row S, sum_b y_b equals the oracle's
    sandwich of S, and every row of the x gradient equals the oracle's x
    gradient of one row (it does not depend on x)."""
    n = 8
    cl = cc.CliffordAlgebra([1] * 7 + [-1], device="cuda")
    layer = cc.RotorLayer(cl).train()
    g = torch.Generator().manual_seed(0)
    biv = (0.1 ** 0.5) * torch.randn(1, 28, generator=g)
    with torch.no_grad():
        layer.bivector.copy_(biv.cuda())
    B = 131072
    x = torch.randn(B, 256, generator=g)
    xd = x.cuda().requires_grad_()
    y = layer(xd)
    y.sum().backward()
    rows = torch.tensor([0, 1, 77, 4096, 65536, B - 1])
    y64, _, gx64 = oracle_step(biv, x[rows], torch.ones(len(rows), 256), n)
    assert rel_err(y[rows.cuda()], y64) <= TOL
    assert rel_err(xd.grad[rows.cuda()], gx64) <= TOL
    S = x.double().sum(0, keepdim=True)
    yS, gbS, gx1 = oracle_step(biv, S, torch.ones(1, 256), n)
    assert rel_err(y.detach().double().sum(0, keepdim=True), yS) <= TOL
    assert rel_err(layer.bivector.grad, gbS) <= TOL
    assert rel_err(xd.grad, gx1.expand(B, 256)) <= TOL


def test_compile_then_apply_eval_cache_and_properties():
    n = 8
    cl = cc.CliffordAlgebra([1] * n, device="cuda")
    layer = cc.RotorLayer(cl).eval()
    x = torch.randn(64, 256, device="cuda")
    with torch.no_grad():
        y1 = layer(x)
        layer.bivector.mul_(0.5)          # in-place edit must invalidate the eval cache
        y2 = layer(x)
        cs = cl.compile_bivector(layer.bivector)
        y3 = cl.apply_rotor(cs, x)
    assert not torch.allclose(y1, y2)
    torch.testing.assert_close(y2, y3)
    # norm and grade preservation of the sandwich
    torch.testing.assert_close(cl.norm_sq(y3), cl.norm_sq(x), rtol=1e-5, atol=1e-4)
    for k in range(n + 1):
        torch.testing.assert_close(cl.grade_projection(y3, k),
                                   cl.apply_rotor(cs, cl.grade_projection(x, k)), rtol=1e-5, atol=1e-5)


def test_large_and_equal_angles():
    """Equal plane angles (where the reference's eigh pair pick is fragile) and a
    large bivector (scaling and squaring)."""
    n = 8
    cl = cc.CliffordAlgebra([1] * n, device="cuda")
    biv = torch.zeros(1, 28)
    # two commuting planes (0,1) and (2,3) with the same angle, and a big one
    biv[0, 0] = 0.7
    biv[0, 13] = 0.7     # pair (2,3): index of (2,3) in lex order is 7+6 = 13
    g = torch.Generator().manual_seed(5)
    x = torch.randn(8, 256, generator=g)
    for scale in (1.0, 25.0):
        b = biv * scale
        bd = b.cuda().requires_grad_()
        y = cl.apply_bivector(bd, x.cuda())
        y.sum().backward()
        y64, gb64, _ = oracle_step(b, x, torch.ones(8, 256), n)
        assert rel_err(y, y64) <= 5e-5, scale
        assert rel_err(bd.grad, gb64) <= 5e-4, scale


def test_rotor_errors():
    cl = cc.CliffordAlgebra([1] * 6, device="cuda")
    with pytest.raises(ValueError, match="n >= 7"):
        cl.compile_bivector(torch.zeros(1, 15, device="cuda"))
    cl8 = cc.CliffordAlgebra([1] * 8, device="cuda")
    with pytest.raises(ValueError, match="first dim must be 1"):
        cl8.compile_bivector(torch.zeros(2, 28, device="cuda"))
    with pytest.raises(ValueError, match="rotor state"):
        cl8.apply_rotor(torch.zeros(5, device="cuda"), torch.zeros(2, 256, device="cuda"))


def _rotor_step(cl, biv, x, gy, need_biv=True, need_x=True):
    bd = biv.cuda().requires_grad_(need_biv)
    xd = x.cuda().requires_grad_(need_x)
    y = cl.apply_bivector(bd, xd)
    y.backward(gy.cuda())
    return y.detach(), (bd.grad if need_biv else None), (xd.grad if need_x else None)


@pytest.mark.parametrize("B", [1, 3, 16, 27, 1000, 40001])
def test_rotor8_matrix_path_matches_chain_and_oracle(B, monkeypatch):
    """n = 8 runs through the Cl(8,0) representation by default; the register
    chain (CLF_ROTOR_PATH=chain) and the oracle give the same values and
    gradients, for batches that leave partial row groups (rows past the end
    must not enter the bivector-gradient sums), and for the gx-only and
    bivector-only backward variants."""
    cl = cc.CliffordAlgebra([1] * 7 + [-1], device="cuda")
    g = torch.Generator().manual_seed(B)
    biv = 0.6 * torch.randn(1, 28, generator=g)
    x = torch.randn(B, 256, generator=g)
    gy = torch.randn(B, 256, generator=g)
    print(f"[case] rotor8 matrix vs chain B={B}", flush=True)
    ym, gbm, gxm = _rotor_step(cl, biv, x, gy)
    _, gb_only, _ = _rotor_step(cl, biv, x, gy, need_x=False)
    _, _, gx_only = _rotor_step(cl, biv, x, gy, need_biv=False)
    monkeypatch.setenv("CLF_ROTOR_PATH", "chain")
    yc, gbc, gxc = _rotor_step(cl, biv, x, gy)
    monkeypatch.delenv("CLF_ROTOR_PATH")
    assert rel_err(ym, yc) <= TOL
    assert rel_err(gxm, gxc) <= TOL
    assert rel_err(gbm, gbc) <= TOL
    assert torch.equal(gb_only, gbm)
    assert torch.equal(gx_only, gxm)
    if B <= 1000:
        rows = torch.arange(B)
        y64, gb64, gx64 = oracle_step(biv, x[rows], gy[rows], 8)
        assert rel_err(ym, y64) <= TOL
        assert rel_err(gxm, gx64) <= TOL
        assert rel_err(gbm, gb64) <= TOL


def test_rotor8_state_spin_block():
    """The n = 8 state ends with the 16 x 16 spin matrix U = phi(R): orthogonal,
    and unchanged in sign convention by large angles (c < 0 planes)."""
    cl = cc.CliffordAlgebra([1] * 8, device="cuda")
    for scale in (0.05, 1.0, 3.0):
        biv = scale * torch.randn(1, 28, generator=torch.Generator().manual_seed(11))
        state = cl.compile_bivector(biv.cuda())
        assert state.numel() == 8 * 8 + 56 + 256
        U = state[120:].double().view(16, 16).cpu()
        torch.testing.assert_close(U @ U.T, torch.eye(16, dtype=torch.float64), atol=2e-6, rtol=0)
