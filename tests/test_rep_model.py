"""The matrix-representation product (tests/rep_model.py, the algorithm of
cliffordcuda_amd/csrc/rep.hip) equals the oracle's geometric product and its
gradients, for real-matrix-type signatures."""
import numpy as np
import pytest
import torch

from oracle import clifford_oracle as O
from tests import rep_model as R


@pytest.mark.parametrize("metric", [(1,) * 8, (1,) * 4 + (-1,) * 4, (1,) * 5 + (-1,) * 3, (-1,) * 8,
                                    (1,) * 6, (1, 1, 1, -1, -1, -1), (1, 1), (1, -1), (1,) * 4 + (-1,) * 2 + (1,) * 2])
def test_rep_product(metric):
    n = len(metric)
    m = 1 << (n // 2)
    gens = R.find_generators(metric)
    p, q = metric.count(1), metric.count(-1)
    if (p - q) % 8 not in (0, 2):
        assert gens is None
        return
    assert gens is not None
    label, sign = R.blade_tables(metric, gens)
    assert len(set(label)) == 1 << n   # bijection
    g = torch.Generator().manual_seed(n)
    a = torch.randn(3, 1 << n, generator=g, dtype=torch.float64)
    b = torch.randn(3, 1 << n, generator=g, dtype=torch.float64)
    gc = torch.randn(3, 1 << n, generator=g, dtype=torch.float64)
    A = R.to_matrix(a.numpy(), label, sign, m)
    B = R.to_matrix(b.numpy(), label, sign, m)
    # homomorphism on basis blades against the explicit Pauli matrices
    for I in sorted({1, 3 % (1 << n), (1 << n) - 1}):
        x, z = label[I]
        e = np.zeros(1 << n)
        e[I] = 1.0
        np.testing.assert_allclose(R.to_matrix(e, label, sign, m), sign[I] * R.pauli(x, z, m))
    c = R.from_matrix(A @ B, label, sign, m)
    aq, bq = a.clone().requires_grad_(), b.clone().requires_grad_()
    c_ref = O.einsum_product("geom", aq, bq, metric)
    c_ref.backward(gc)
    np.testing.assert_allclose(c, c_ref.detach().numpy(), atol=1e-10)
    np.testing.assert_allclose(R.from_matrix(A, label, sign, m), a.numpy(), atol=1e-12)
    # backward: ga = iconv(conv(gc) B^T), gb = iconv(A^T conv(gc))
    G = R.to_matrix(gc.numpy(), label, sign, m)
    ga = R.from_matrix(G @ np.swapaxes(B, -1, -2), label, sign, m)
    gb = R.from_matrix(np.swapaxes(A, -1, -2) @ G, label, sign, m)
    np.testing.assert_allclose(ga, aq.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(gb, bq.grad.numpy(), atol=1e-10)
