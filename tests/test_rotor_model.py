"""The rotor kernels' math (tests/rotor_model.py) equals the oracle's
Euclidean sandwich and its autograd gradients."""
import numpy as np
import scipy.linalg
import torch

from oracle import clifford_oracle as O
from tests import rotor_model as M


def test_rotor_model_matches_oracle():
    n = 5
    g = torch.Generator().manual_seed(1)
    biv = 0.6 * torch.randn(1, 10, generator=g, dtype=torch.float64)
    x = torch.randn(3, 32, generator=g, dtype=torch.float64)
    gy = torch.randn(3, 32, generator=g, dtype=torch.float64)
    bq = biv.clone().requires_grad_()
    xq = x.clone().requires_grad_()
    y = O.apply_bivector(bq, xq, n)
    y.backward(gy)
    Q = scipy.linalg.expm(M.generator(biv[0].numpy(), n))
    cs, E = M.givens(Q)
    np.testing.assert_allclose(E, np.eye(n), atol=1e-12)
    ym = M.apply(cs, x.numpy())
    np.testing.assert_allclose(ym, y.detach().numpy(), atol=1e-12)
    gx = M.apply(cs, gy.numpy(), transpose=True)
    np.testing.assert_allclose(gx, xq.grad.numpy(), atol=1e-12)
    G = M.gamma(x.numpy(), gx, n)
    gb = M.compile_bwd(biv[0].numpy(), n, Q @ G)
    np.testing.assert_allclose(gb, bq.grad[0].numpy(), atol=1e-10)
    # only the antisymmetric part of Gamma reaches the bivector (Q stays in SO(n))
    gb_skew = M.compile_bwd(biv[0].numpy(), n, Q @ (0.5 * (G - G.T)))
    np.testing.assert_allclose(gb_skew, bq.grad[0].numpy(), atol=1e-10)


def test_skew_sums_over_output_conjugate():
    """The kernels accumulate the pair sums over the forward output and its
    gradient: skew Gamma(x, gx) = Q^T skew Gamma(y, gy) Q, hence
    dL/dQ = Q skew Gamma(x, gx) = skew Gamma(y, gy) Q."""
    n = 6
    rng = np.random.default_rng(5)
    biv = 0.5 * rng.standard_normal(15)
    Q = scipy.linalg.expm(M.generator(biv, n))
    cs, _ = M.givens(Q)
    x = rng.standard_normal((4, 64))
    gy = rng.standard_normal((4, 64))
    y = M.apply(cs, x)
    gx = M.apply(cs, gy, transpose=True)
    G, Gy = M.gamma(x, gx, n), M.gamma(y, gy, n)
    K, Ky = 0.5 * (G - G.T), 0.5 * (Gy - Gy.T)
    np.testing.assert_allclose(K, Q.T @ Ky @ Q, atol=1e-12)
    np.testing.assert_allclose(Q @ K, Ky @ Q, atol=1e-12)
    # and the result is the oracle's bivector gradient
    g = torch.Generator().manual_seed(2)
    bq = torch.tensor(biv, dtype=torch.float64).reshape(1, -1).requires_grad_()
    xq = torch.tensor(x).requires_grad_()
    O.apply_bivector(bq, xq, n).backward(torch.tensor(gy))
    np.testing.assert_allclose(M.compile_bwd(biv, n, Ky @ Q), bq.grad[0].numpy(), atol=1e-10)
