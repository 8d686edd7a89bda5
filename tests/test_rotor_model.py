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


def test_rotor16_lane_model_matches_oracle():
    """n = 8 through the Cl(8,0) representation (csrc/rotor_rep.hip): the
    spin matrix built from the chain's half angles, the block transpose by
    permlane swaps between the two products, and the per-plane sums contracted
    from the 16 x 16 accumulator give the oracle's sandwich, x gradient and
    bivector gradient."""
    from tests import rep_model as R
    n = 8
    gens = R.find_generators([1] * 8)
    label, sign = R.blade_tables([1] * 8, gens)
    planes = R.spin_planes(label, sign)
    g = torch.Generator().manual_seed(5)
    # angles past pi/2 exercise the c < 0 half-angle branch
    biv = 0.9 * torch.randn(1, 28, generator=g, dtype=torch.float64)
    x = torch.randn(4, 256, generator=g, dtype=torch.float64)
    gy = torch.randn(4, 256, generator=g, dtype=torch.float64)
    bq = biv.clone().requires_grad_()
    xq = x.clone().requires_grad_()
    y = O.apply_bivector(bq, xq, n)
    y.backward(gy)
    Q = scipy.linalg.expm(M.generator(biv[0].numpy(), n))
    cs, _ = M.givens(Q)
    assert min(c for _, _, c, _ in cs) < 0
    U = R.spin_matrix(cs, planes)
    np.testing.assert_allclose(U @ U.T, np.eye(16), atol=1e-12)
    # the kernel builds U as expm(phi(B)): the same matrix up to sign
    Ue = R.spin_matrix_expm(biv[0].numpy(), label, sign)
    assert min(np.abs(Ue - U).max(), np.abs(Ue + U).max()) < 1e-10
    # lane model of the kernel's fp64-MFMA exponential
    Ul = R.spin_expm_lanes(biv[0].numpy(), R.spin_plane_masks(planes))
    np.testing.assert_allclose(Ul, Ue, atol=1e-12)
    U = Ul
    np.testing.assert_allclose(R.rotor16_fwd(x.numpy(), U, label, sign), y.detach().numpy(), atol=1e-10)
    np.testing.assert_allclose(R.rotor16_fwd(gy.numpy(), U, label, sign, transpose=True), xq.grad.numpy(),
                               atol=1e-10)
    gx, K = R.rotor16_bwd(x.numpy(), gy.numpy(), U, label, sign, planes)
    np.testing.assert_allclose(gx, xq.grad.numpy(), atol=1e-10)
    # K_pq = Gamma_pq - Gamma_qp, and dL/dQ = Q skew(Gamma) carries the bivector gradient
    G = M.gamma(x.numpy(), gx, n)
    iu = np.triu_indices(n, 1)
    np.testing.assert_allclose(K, (G - G.T)[iu], atol=1e-9)
    S = np.zeros((n, n))
    S[iu] = 0.5 * K
    S = S - S.T
    gb = M.compile_bwd(biv[0].numpy(), n, Q @ S)
    np.testing.assert_allclose(gb, bq.grad[0].numpy(), atol=1e-9)
