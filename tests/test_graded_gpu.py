"""GPU parity of the graded ops and norm_sq (forward + backward) against the
oracle, plus the reference's identity tests (tests/correctness/test_dual.py,
test_norm_sq.py)."""
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


METRICS = [(1, 1, 1), (1, -1), (1,) * 5, (1, 1, -1, -1, 0), (-1, 1, 1, -1, 1, -1, 1, 1), (1,) * 9 + (0,)]


@pytest.mark.parametrize("metric", METRICS)
def test_graded_ops(metric):
    n = len(metric)
    cl = cc.CliffordAlgebra(metric, device="cuda")
    g = torch.Generator().manual_seed(1)
    x = torch.randn(33, 1 << n, generator=g)
    gy = torch.randn(33, 1 << n, generator=g)
    cases = [("reverse", cl.reverse, O.reverse), ("involution", cl.grade_involution, O.grade_involution),
             ("conjugation", cl.clifford_conjugation, O.clifford_conjugation)]
    for k in range(n + 1):
        cases.append((f"proj{k}", lambda t, k=k: cl.grade_projection(t, k), lambda t, k=k: O.grade_projection(t, k)))
    if 0 not in metric:
        cases.append(("dual", cl.dual, lambda t: O.dual(t, metric)))
        cases.append(("dual_c", lambda t: cl.dual(t, compile=True), lambda t: O.dual(t, metric)))
    for name, fn, ref_fn in cases:
        xd = x.cuda().requires_grad_()
        y = fn(xd)
        y.backward(gy.cuda())
        x64 = x.double().requires_grad_()
        y64 = ref_fn(x64)
        y64.backward(gy.double())
        assert rel_err(y, y64) == 0.0 or rel_err(y, y64) <= TOL, name
        assert rel_err(xd.grad, x64.grad) <= TOL, name
    # norm_sq
    xd = x.cuda().requires_grad_()
    ns = cl.norm_sq(xd)
    gns = torch.randn(33, generator=g)
    ns.backward(gns.cuda())
    x64 = x.double().requires_grad_()
    ns64 = O.norm_sq(x64, metric)
    ns64.backward(gns.double())
    assert rel_err(ns, ns64) <= TOL
    assert rel_err(xd.grad, x64.grad) <= TOL


@pytest.mark.parametrize("metric", [(1, 1, 1), (1, 1, -1), (1,) * 5, (-1, -1, 1, 1, -1), (1,) * 7 + (-1,)])
def test_dual_is_geom_with_inverse_pseudoscalar(metric):
    """dual(x) == geom_prod(x, I^{-1}) (reference tests/correctness/test_dual.py:41-65)."""
    n = len(metric)
    dim = 1 << n
    cl = cc.CliffordAlgebra(metric, device="cuda")
    I = torch.zeros(1, dim, device="cuda")
    I[0, dim - 1] = 1.0
    isq = cl.geom_prod(I, I)[0, 0]
    Iinv = (I / isq).expand(16, dim).contiguous()
    x = torch.randn(16, dim, device="cuda")
    torch.testing.assert_close(cl.dual(x), cl.geom_prod(x, Iinv), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("metric", [(1,) * 5, (1, 1, -1, -1, 0), (0, 1, 1, -1, 1, 1)])
def test_norm_sq_is_scalar_part_of_x_xrev(metric):
    """norm_sq(x) == geom_prod(x, reverse(x))[:, 0] (reference test_norm_sq.py:46-63)."""
    n = len(metric)
    cl = cc.CliffordAlgebra(metric, device="cuda")
    x = torch.randn(64, 1 << n, device="cuda")
    torch.testing.assert_close(cl.norm_sq(x), cl.geom_prod(x, cl.reverse(x))[:, 0], rtol=1e-4, atol=1e-3)
