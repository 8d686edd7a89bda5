"""CPU restatement of the inverse kernels' arithmetic (csrc/inverse.hip),
checked against the oracle: the Pauli-label representation of the non-null
generators (labels, phases, the Walsh-Hadamard maps, the two-copy case), the
in-place Gauss-Jordan with partial pivoting and the Newton completion for null
generators. No GPU."""
import math

import numpy as np
import pytest
import torch

from oracle import clifford_oracle as O


def gamma(t, np_, neg):
    m = np_ // 2
    if t < 2 * m:
        k = t >> 1
        a, b, e = 1 << k, ((1 << k) - 1) | ((1 << k) if t & 1 else 0), t & 1
    else:
        a, b, e = 0, (1 << m) - 1, 0
    return a, b, e + (1 if neg else 0)


def blade_label(A, metric):
    n = len(metric)
    nonnull = [g for g in range(n) if metric[g] != 0]
    a = b = e = 0
    for t, g in enumerate(nonnull):
        if (A >> g) & 1:
            ga, gb, ge = gamma(t, len(nonnull), metric[g] == -1)
            e += ge + 2 * (bin(b & ga).count("1") & 1)
            a ^= ga
            b ^= gb
    return a, b, e & 3


def plan(metric):
    n = len(metric)
    nonnull = sum(1 << g for g in range(n) if metric[g] != 0)
    np_ = bin(nonnull).count("1")
    d = 1 << (np_ // 2)
    two = False
    if np_ & 1:
        two = blade_label(nonnull, metric)[2] % 2 == 0
    return nonnull, d, two


def wht_rows(T):
    T = T.copy()
    d = T.shape[1]
    h = 1
    while h < d:
        for b0 in range(d):
            if b0 & h:
                continue
            u, v = T[:, b0].copy(), T[:, b0 | h].copy()
            T[:, b0], T[:, b0 | h] = u + v, u - v
        h <<= 1
    return T


def xor_columns(T):
    d = T.shape[0]
    out = T.copy()
    for c in range(d):
        for i in range(d):
            out[i, c] = T[i ^ c, c]
    return out


def to_matrix(x, metric, involute=False):
    n = len(metric)
    nonnull, d, _ = plan(metric)
    T = np.zeros((d, d), dtype=np.complex128)
    for A in range(1 << n):
        if A & ~nonnull:
            continue
        a, b, e = blade_label(A, metric)
        v = x[A] * (-1.0 if (involute and bin(A).count("1") & 1) else 1.0)
        T[a, b] += (1j ** e) * v
    return xor_columns(wht_rows(T))


def from_matrices(Np, Nm, metric):
    n = len(metric)
    nonnull, d, two = plan(metric)
    Up = wht_rows(xor_columns(Np)) / d
    Um = wht_rows(xor_columns(Nm)) / d if two else None
    y = np.zeros(1 << n)
    for A in range(1 << n):
        if A & ~nonnull:
            continue
        a, b, e = blade_label(A, metric)
        u = Up[a, b]
        if two:
            u = 0.5 * (u + (-1.0 if bin(A).count("1") & 1 else 1.0) * Um[a, b])
        y[A] = ((1j ** (4 - e)) * u).real
    return y


def gauss_jordan(M):
    """In-place Gauss-Jordan with partial pivoting, as the kernel runs it."""
    M = M.copy()
    d = M.shape[0]
    piv = []
    for k in range(d):
        mags = [abs(M[i, k]) ** 2 if i >= k else -1.0 for i in range(d)]
        p = int(np.argmax(mags))
        piv.append(p)
        M[[k, p]] = M[[p, k]]
        inv = 1.0 / M[k, k]
        for j in range(d):
            if j != k:
                M[k, j] *= inv
        for j in range(d):
            if j == k:
                continue
            for i in range(d):
                if i != k:
                    M[i, j] -= M[i, k] * M[k, j]
        for i in range(d):
            if i != k:
                M[i, k] = -M[i, k] * inv
        M[k, k] = inv
    for k in reversed(range(d)):
        p = piv[k]
        M[:, [k, p]] = M[:, [p, k]]
    return M


METRICS = [
    (1, 1, 1, 1),                 # even, single copy
    (1, -1, 1, -1, -1),           # odd, pseudoscalar^2 = -1: single copy
    (1, 1, 1, 1, 1),              # odd, pseudoscalar^2 = +1: two copies
    (-1, 1, 1),                   # odd, small
    (1, 0, 1, -1),                # null generator (non-null part Cl(2,1), two copies)
    (0, 1, 1, 1, 0),              # two null generators
    (1, 1, -1, 1, 1, -1),         # even n' = 6
]


@pytest.mark.parametrize("metric", METRICS, ids=str)
def test_representation_is_a_homomorphism(metric):
    n = len(metric)
    g = torch.Generator().manual_seed(len(metric))
    a = torch.randn(1, 1 << n, generator=g, dtype=torch.float64)
    b = torch.randn(1, 1 << n, generator=g, dtype=torch.float64)
    ab = O.einsum_product("geom", a, b, metric)[0].numpy()
    for inv in (False, True):
        lhs = to_matrix(ab, metric, inv)
        rhs = to_matrix(a[0].numpy(), metric, inv) @ to_matrix(b[0].numpy(), metric, inv)
        np.testing.assert_allclose(lhs, rhs, atol=1e-9)


@pytest.mark.parametrize("metric", METRICS, ids=str)
def test_round_trip_recovers_the_non_null_part(metric):
    n = len(metric)
    nonnull, _, two = plan(metric)
    x = np.random.default_rng(3).standard_normal(1 << n)
    y = from_matrices(to_matrix(x, metric), to_matrix(x, metric, True) if two else None, metric)
    keep = np.array([0.0 if A & ~nonnull else 1.0 for A in range(1 << n)])
    np.testing.assert_allclose(y, x * keep, atol=1e-12)


@pytest.mark.parametrize("metric", METRICS, ids=str)
def test_model_inverse_matches_dense_solve(metric):
    """Invert M(x) by the kernel's Gauss-Jordan, map back, complete null parts
    by Newton steps, and compare with the dense solve of L(x) y = e_0."""
    n = len(metric)
    _, _, two = plan(metric)
    rng = np.random.default_rng(11 + n)
    x = rng.standard_normal(1 << n)
    x[0] += 3.0
    Np = gauss_jordan(to_matrix(x, metric))
    Nm = gauss_jordan(to_matrix(x, metric, True)) if two else None
    y = torch.tensor(from_matrices(Np, Nm, metric)).view(1, -1)
    xt = torch.tensor(x).view(1, -1)
    r = sum(1 for m in metric if m == 0)
    one = torch.zeros_like(xt)
    one[0, 0] = 2.0
    for _ in range(math.ceil(math.log2(r + 1)) if r else 0):
        y = O.einsum_product("geom", y, one - O.einsum_product("geom", xt, y, metric), metric)
    sig = O.sign_value_table(n, metric).double()
    dim = 1 << n
    L = torch.zeros(dim, dim, dtype=torch.float64)
    for k in range(dim):
        for j in range(dim):
            L[k, j] = sig[j ^ k, j] * xt[0, j ^ k]
    e0 = torch.zeros(dim, dtype=torch.float64)
    e0[0] = 1.0
    ref = torch.linalg.solve(L, e0)
    torch.testing.assert_close(y[0], ref, rtol=0, atol=1e-10)


@pytest.mark.parametrize("metric", METRICS, ids=str)
def test_scatter_passes_never_share_a_label(metric):
    """The kernel scatters blades in two passes split by the last non-null
    generator; within a pass no two blades may write the same label."""
    n = len(metric)
    nonnull, d, _ = plan(metric)
    last = max(g for g in range(n) if metric[g] != 0)
    for pass_ in (0, 1):
        seen = set()
        for A in range(1 << n):
            if A & ~nonnull or bool((A >> last) & 1) != bool(pass_):
                continue
            a, b, _ = blade_label(A, metric)
            assert (a, b) not in seen
            seen.add((a, b))


@pytest.mark.parametrize("metric", [(1, 1, 1), (1, -1, 0, 1), (-1, -1, 1, 0, 1), (0, 1, -1, 1, -1)])
def test_dense_lmul_matrix_is_left_multiplication(metric):
    """The dense inverse's L(x) gathered with the blade-product sign table
    (inverse._lmul_tables) is left multiplication by x: L(x) y equals the
    oracle's geometric product x y for random x, y (negative and null
    generators, null ones not only last). A sign or index mistake in the table
    changes a column and fails this."""
    from cliffordcuda_amd.inverse import _lmul_tables
    from cliffordcuda_amd._validate import metric_masks
    n = len(metric)
    neg, nul = metric_masks(metric)
    g = torch.Generator().manual_seed(7 + n)
    x = torch.randn(3, 1 << n, generator=g, dtype=torch.float64)
    y = torch.randn(3, 1 << n, generator=g, dtype=torch.float64)
    idx, sign = _lmul_tables(n, neg, nul, "cpu")
    lmat = x[:, idx] * sign.double()
    got = torch.einsum("bkj,bj->bk", lmat, y)
    want = O.einsum_product("geom", x, y, list(metric))
    assert torch.allclose(got, want, atol=1e-12)
