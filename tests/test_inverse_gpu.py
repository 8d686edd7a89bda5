"""GPU checks of the multivector inverse (the reference's inverse,
src/cliffordcuda/extensions/ga/inverse.py, and its tests
tests/correctness/test_inverse.py): the versor path at every n, the
matrix-representation path (single and two copies, degenerate metrics through
the Newton completion) and the dense solve against the fp64 oracle, method
dispatch and errors, leading dimensions, and gradients against autograd
through the oracle."""
import pytest
import torch

import cliffordcuda_amd as cc
from cliffordcuda_amd import _lib
from cliffordcuda_amd._validate import metric_masks
from oracle import clifford_oracle as O

pytestmark = pytest.mark.gpu


def _scalar_res(prod):
    ref = torch.zeros_like(prod)
    ref[..., 0] = 1.0
    return float((prod - ref).abs().max())


def _rand_vector(B, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.zeros(B, 1 << n)
    for i in range(n):
        x[:, 1 << i] = torch.randn(B, generator=g)
    return x.cuda()


def _metrics(n):
    out = [(1,) * n, tuple(-1 if i % 3 == 0 else 1 for i in range(n))]
    if n >= 3:
        out.append((0,) + (1,) * (n - 2) + (-1,))
    return out


def _general(B, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, 1 << n, generator=g)
    x[:, 0] += 3.0
    return x


@pytest.mark.parametrize("n", [5, 8, 11, 13, 15, 17])
def test_versor_exact_all_n(n):
    """Versor inverse at every n, both sides (reference test_inverse.py:62-71)."""
    for metric in _metrics(n):
        print(f"[case] versor n={n} metric={metric}", flush=True)
        R = cc.geom_prod(_rand_vector(2, n, 1), _rand_vector(2, n, 2), metric=metric)
        inv = cc.inverse(R, metric=metric)
        assert _scalar_res(cc.geom_prod(R, inv, metric=metric)) < 1e-4
        assert _scalar_res(cc.geom_prod(inv, R, metric=metric)) < 1e-4


@pytest.mark.parametrize("method", ["auto", "rep", "lu"])
@pytest.mark.parametrize("n", [5, 7, 9, 10])
def test_general_matches_dense_oracle(n, method):
    """A general multivector's inverse against the fp64 dense solve, for
    Euclidean, mixed and degenerate metrics, batches 1 and 3."""
    for metric in _metrics(n):
        for B in (1, 3):
            print(f"[case] general n={n} method={method} metric={metric} B={B}", flush=True)
            x = _general(B, n, 100 + n + B)
            inv = cc.inverse(x.cuda(), metric=metric, method=method)
            ref = O.inverse_dense(x.double(), metric)
            # the fp32 dense solve of a 2^n system is held to the reference's own
            # bar (1e-3, test_inverse.py:82), the representation to 1e-4
            tol = 1e-3 if method == "lu" else 1e-4
            assert float((inv.double().cpu() - ref).abs().max()) < tol * max(1.0, float(ref.abs().max()))
            assert _scalar_res(cc.geom_prod(x.cuda(), inv, metric=metric)) < 1e-3
            assert inv.is_contiguous()


# (n, metric): single copy (even n, odd n with pseudoscalar^2 = -1) and two
# copies (odd n with pseudoscalar^2 = +1), as in the reference's REP_DISPATCH
REP = [(7, (1,) * 7), (8, (1,) * 8), (5, (1, 1, 1, 1, -1)), (9, (-1,) + (1,) * 8), (10, (1,) * 10),
       (5, (1,) * 5), (9, (1,) * 9), (4, (-1,) * 4), (6, (1, -1) * 3)]


@pytest.mark.parametrize("n,metric", REP, ids=str)
def test_rep_matches_dense_oracle(n, metric):
    x = _general(3, n, n)
    inv = cc.inverse(x.cuda(), metric=metric, method="rep")
    ref = O.inverse_dense(x.double(), metric)
    assert float((inv.double().cpu() - ref).abs().max()) < 1e-4 * max(1.0, float(ref.abs().max()))


DEGEN = [(6, (0,) + (1,) * 5), (7, (0,) + (1,) * 6), (6, (1, 1, 1, 1, -1, 0)), (7, (0, 0) + (1,) * 5),
         (10, (1,) * 9 + (0,)), (8, (0, 1, 0, 1, -1, 0, 1, 1))]


@pytest.mark.parametrize("n,metric", DEGEN, ids=str)
def test_degenerate_matches_dense_oracle(n, metric):
    """Degenerate metrics: the representation inverts the non-null part and
    Newton steps add the null part (r = 1, 2, 3 null generators)."""
    x = _general(3, n, 7 * n)
    for method in ("auto", "rep"):
        inv = cc.inverse(x.cuda(), metric=metric, method=method)
        ref = O.inverse_dense(x.double(), metric)
        assert float((inv.double().cpu() - ref).abs().max()) < 1e-4 * max(1.0, float(ref.abs().max()))


@pytest.mark.parametrize("n,metric", [(13, (1,) * 13), (12, (1,) * 11 + (-1,)), (14, (1,) * 14)], ids=str)
def test_rep_large_n_matches_lu(n, metric):
    """n = 12 .. 14 (matrix side 64 and 128, two copies at n = 13): the
    representation against the dense GPU solve, and a valid right inverse."""
    x = _general(1, n, n).cuda()
    inv = cc.inverse(x, metric=metric, method="rep")
    assert _scalar_res(cc.geom_prod(x, inv, metric=metric)) < 1e-3
    if n <= 13:
        lu = cc.inverse(x, metric=metric, method="lu")
        assert float((inv - lu).abs().max()) < 1e-3


def test_rep_supported_matches_reference_dispatch():
    """Every non-degenerate signature up to 14 generators has a representation
    (and every degenerate one whose non-null part does); past that, method='rep'
    raises like the reference (its blade-tensor budget stops at n' = 14)."""
    lib = _lib.load()
    for metric in [(1,) * 7, (1,) * 8, (1, 1, 1, 1, -1), (1,) * 5, (1,) * 9, (1,) * 13, (-1,) + (1,) * 8,
                   (0,) + (1,) * 5, (1,) * 14, (0,) + (1,) * 14]:
        neg, nul = metric_masks(metric)
        assert lib.clf_inverse_rep_supported(len(metric), neg, nul) == 1, metric
    for metric in [(1,) * 15, (-1,) * 16]:
        neg, nul = metric_masks(metric)
        assert lib.clf_inverse_rep_supported(len(metric), neg, nul) == 0, metric
    x = torch.zeros(1, 1 << 15, device="cuda")
    x[0, 0] = 1.0
    x[0, 3] = 0.5
    with pytest.raises(ValueError, match="not representable"):
        cc.inverse(x, metric=(1,) * 15, method="rep")


def test_auto_dispatch_and_method_errors():
    n, metric = 8, (1,) * 8
    R = cc.geom_prod(_rand_vector(1, n, 3), _rand_vector(1, n, 4), metric=metric)
    assert _scalar_res(cc.geom_prod(R, cc.inverse(R, metric=metric), metric=metric)) < 1e-6
    g = _general(1, n, 5).cuda()
    assert _scalar_res(cc.geom_prod(g, cc.inverse(g, metric=metric), metric=metric)) < 1e-3
    with pytest.raises(ValueError, match="not a versor|not scalar"):
        cc.inverse(_general(1, 6, 6).cuda(), metric=(1,) * 6, method="versor")
    with pytest.raises(ValueError, match="method must be"):
        cc.inverse(g, metric=metric, method="cholesky")


def test_non_invertible_raises():
    n = 6
    with pytest.raises(ValueError, match="not invertible"):
        cc.inverse(torch.zeros(1, 1 << n, device="cuda"), metric=(1,) * n)
    x = torch.zeros(1, 1 << n, device="cuda")
    x[0, 1] = 1.0                                   # a null vector
    with pytest.raises(ValueError, match="not invertible"):
        cc.inverse(x, metric=(0,) + (1,) * (n - 1), method="versor")
    # (1 + e_0) w with e_0^2 = +1: (1 - e_0)(1 + e_0) w = 0, a zero divisor
    # (and, for a general w, not a versor)
    p = torch.zeros(1, 1 << n, device="cuda")
    p[0, 0] = 1.0
    p[0, 1] = 1.0
    z = cc.geom_prod(p, _general(1, n, 16).cuda(), metric=(1,) * n)
    for method in ("auto", "rep", "lu"):
        with pytest.raises(ValueError, match="not invertible"):
            cc.inverse(z, metric=(1,) * n, method=method)


def test_leading_dims_and_algebra_method():
    n, metric = 6, (1,) * 6
    x = torch.randn(3, 4, 1 << n, generator=torch.Generator().manual_seed(8))
    x[..., 0] += 3.0
    inv = cc.inverse(x.cuda(), metric=metric)
    assert inv.shape == x.shape
    assert _scalar_res(cc.geom_prod(x.cuda().reshape(-1, 1 << n), inv.reshape(-1, 1 << n), metric=metric)) < 1e-3
    ca = cc.CliffordAlgebra((1, 1, 1, -1, 1), device="cuda")
    R = ca.geom_prod(_rand_vector(4, 5, 9), _rand_vector(4, 5, 10))
    assert _scalar_res(ca.geom_prod(R, ca.inverse(R))) < 1e-5
    gx = _general(2, 5, 11).cuda()
    assert _scalar_res(ca.geom_prod(gx, ca.inverse(gx))) < 1e-3


@pytest.mark.parametrize("method", ["versor", "rep", "lu"])
@pytest.mark.parametrize("metric", [(1,) * 6, (1, -1, 1, 1, -1), (0, 1, 1, 1, -1)], ids=str)
def test_gradients_match_oracle_autograd(method, metric):
    """x.grad against autograd through the oracle: the dense solve (the
    inverse's own derivative -y dx y) for rep and lu, and the formula
    rev(x) / <x rev(x)>_0 for the versor path (what autograd through the
    reference's formula gives)."""
    n = len(metric)
    if method == "versor":
        x = (cc.geom_prod(_rand_vector(2, n, 12), _rand_vector(2, n, 13), metric=metric)).cpu()
    else:
        x = _general(2, n, 14)
    gy = torch.randn(2, 1 << n, generator=torch.Generator().manual_seed(15))
    xd = x.cuda().requires_grad_()
    cc.inverse(xd, metric=metric, method=method).backward(gy.cuda())
    x64 = x.double().requires_grad_()
    if method == "versor":
        r = O.reverse(x64)
        y64 = r / O.einsum_product("geom", x64, r, metric)[:, :1]
    else:
        y64 = O.inverse_dense(x64, metric)
    y64.backward(gy.double())
    ref = x64.grad
    assert float((xd.grad.double().cpu() - ref).abs().max()) <= 1e-4 * float(ref.abs().max())
