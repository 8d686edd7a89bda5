"""Pins the CPU oracle (oracle/clifford_oracle.py) with checks that do not
restate its formulas: brute-force generator reordering, real matrix
representations, algebraic identities, grade-selection definitions, closed-form
rotor actions, and autograd vs explicit adjoint formulas.

The reference ships no golden vectors for this path (its tests compute
references on the fly, tests/correctness/*.py), so these checks are the pin.
"""
import itertools
import math

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import clifford_oracle as O

METRICS = {
    3: [(1, 1, 1), (-1, -1, -1), (1, -1, 0), (0, 1, -1), (1, 1, 0)],
    4: [(1, 1, 1, 1), (1, 1, -1, -1), (1, 1, 1, 0), (-1, 0, 1, -1)],
    5: [(1,) * 5, (-1,) * 5, (1, 1, 1, 1, -1), (1, 1, -1, -1, -1), (1, 1, 1, 1, 0), (1, 1, 1, -1, 0)],
}


def blade_product_bruteforce(i, j, metric):
    """Textbook canonical reordering: write e_i e_j as the generator list of i
    followed by that of j (each ascending), bubble-sort with one sign flip per
    swap, then contract equal neighbours with the metric."""
    gens = [k for k in range(len(metric)) if (i >> k) & 1] + [k for k in range(len(metric)) if (j >> k) & 1]
    sign = 1
    arr = list(gens)
    for p in range(len(arr)):
        for q in range(len(arr) - 1 - p):
            if arr[q] > arr[q + 1]:
                arr[q], arr[q + 1] = arr[q + 1], arr[q]
                sign = -sign
    out = []
    for g in arr:
        if out and out[-1] == g:
            out.pop()
            sign *= metric[g]
        else:
            out.append(g)
    blade = sum(1 << g for g in out)
    return sign, blade


@pytest.mark.parametrize("n", [3, 4, 5])
def test_sigma_vs_bruteforce(n):
    for metric in METRICS[n]:
        sig = O.sign_value_table(n, metric)
        for i in range(1 << n):
            for j in range(1 << n):
                s, blade = blade_product_bruteforce(i, j, metric)
                assert blade == i ^ j
                assert int(sig[i, j]) == s, (metric, i, j)


def gamma_matrices(metric):
    """Jordan-Wigner real matrices: gamma_k = Z^{(x)k} (x) G_k (x) I^{(x)(n-k-1)},
    G = X (square +1), J (square -1) or a nilpotent N (square 0). Distinct
    generators anticommute; products of distinct generators are nonzero."""
    X = np.array([[0.0, 1.0], [1.0, 0.0]])
    Z = np.array([[1.0, 0.0], [0.0, -1.0]])
    J = np.array([[0.0, -1.0], [1.0, 0.0]])
    N = np.array([[0.0, 0.0], [1.0, 0.0]])
    I2 = np.eye(2)
    n = len(metric)
    gs = []
    for k, m in enumerate(metric):
        G = {1: X, -1: J, 0: N}[m]
        M = np.array([[1.0]])
        for slot in range(n):
            M = np.kron(M, Z if slot < k else (G if slot == k else I2))
        gs.append(M)
    return gs


@pytest.mark.parametrize("n", [3, 4])
def test_sigma_vs_matrix_representation(n):
    for metric in METRICS[n]:
        gs = gamma_matrices(metric)
        dim = 1 << n
        eye = np.eye(gs[0].shape[0])
        rep = []
        for i in range(dim):
            M = eye.copy()
            for k in range(n):
                if (i >> k) & 1:
                    M = M @ gs[k]
            rep.append(M)
        sig = O.sign_value_table(n, metric)
        for i in range(dim):
            for j in range(dim):
                lhs = rep[i] @ rep[j]
                np.testing.assert_allclose(lhs, float(sig[i, j]) * rep[i ^ j], atol=0)


def test_generator_squares_and_anticommutation():
    metric = (1, -1, 0, 1, -1)
    sig = O.sign_value_table(5, metric)
    for k in range(5):
        assert int(sig[1 << k, 1 << k]) == metric[k]
        for l in range(5):
            if l != k:
                assert int(sig[1 << k, 1 << l]) == -int(sig[1 << l, 1 << k])


def rand_mv(b, n, seed, grade=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(b, 1 << n, generator=g, dtype=torch.float64)
    if grade is not None:
        x = O.grade_projection(x, grade)
    return x


@pytest.mark.parametrize("metric", [(1,) * 5, (1, 1, -1, -1, 0), (-1, 0, 1, 1, -1)])
def test_geom_associative(metric):
    a, b, c = rand_mv(3, 5, 1), rand_mv(3, 5, 2), rand_mv(3, 5, 3)
    ab_c = O.einsum_product("geom", O.einsum_product("geom", a, b, metric), c, metric)
    a_bc = O.einsum_product("geom", a, O.einsum_product("geom", b, c, metric), metric)
    torch.testing.assert_close(ab_c, a_bc, rtol=1e-12, atol=1e-11)


def test_reverse_antiautomorphism():
    metric = (1, 1, -1, 0, 1)
    a, b = rand_mv(3, 5, 4), rand_mv(3, 5, 5)
    lhs = O.reverse(O.einsum_product("geom", a, b, metric))
    rhs = O.einsum_product("geom", O.reverse(b), O.reverse(a), metric)
    torch.testing.assert_close(lhs, rhs, rtol=1e-12, atol=1e-11)


def _unit_vectors(n):
    e = torch.zeros(n + 1, 1 << n, dtype=torch.float64)
    e[0, 0] = 1.0                      # the scalar 1
    for k in range(n):
        e[k + 1, 1 << k] = 1.0         # e_k
    return e


@pytest.mark.parametrize("metric", [(1, 1, -1, 0, 1), (-1, -1, 1, 1, -1), (0, 1, -1, 1, 0)])
def test_grade_involution_is_the_automorphism_negating_vectors(metric):
    """The grade involution is the algebra automorphism with e_k -> -e_k. An
    automorphism is fixed by its action on the generators, so
    inv(1) = 1, inv(e_k) = -e_k and inv(ab) = inv(a) inv(b) (with the
    independently pinned geometric product) determine it; a wrong grade parity
    on any blade breaks the product rule for some pair."""
    n = len(metric)
    e = _unit_vectors(n)
    inv_e = O.grade_involution(e)
    torch.testing.assert_close(inv_e[0], e[0], rtol=0, atol=0)
    torch.testing.assert_close(inv_e[1:], -e[1:], rtol=0, atol=0)
    a, b = rand_mv(4, n, 31), rand_mv(4, n, 32)
    lhs = O.grade_involution(O.einsum_product("geom", a, b, metric))
    rhs = O.einsum_product("geom", O.grade_involution(a), O.grade_involution(b), metric)
    torch.testing.assert_close(lhs, rhs, rtol=1e-12, atol=1e-11)
    # every basis blade, built as an ordered product of generators
    for blade in range(1 << n):
        prod = e[0:1].clone()
        for k in range(n):
            if (blade >> k) & 1:
                prod = O.einsum_product("geom", prod, e[k + 1:k + 2], (1,) * n)
        expect = prod.clone()
        for k in range(n):
            if (blade >> k) & 1:
                expect = -expect
        torch.testing.assert_close(O.grade_involution(prod), expect, rtol=0, atol=0)


@pytest.mark.parametrize("metric", [(1, 1, -1, 0, 1), (-1, 0, 1, 1, -1)])
def test_clifford_conjugation_is_reverse_of_involution(metric):
    """Clifford conjugation is the anti-automorphism with e_k -> -e_k:
    conj(1) = 1, conj(e_k) = -e_k, conj(ab) = conj(b) conj(a), and it equals
    the composition reverse(grade_involution(x)) (both pinned on their own)."""
    n = len(metric)
    e = _unit_vectors(n)
    conj_e = O.clifford_conjugation(e)
    torch.testing.assert_close(conj_e[0], e[0], rtol=0, atol=0)
    torch.testing.assert_close(conj_e[1:], -e[1:], rtol=0, atol=0)
    a, b = rand_mv(4, n, 33), rand_mv(4, n, 34)
    lhs = O.clifford_conjugation(O.einsum_product("geom", a, b, metric))
    rhs = O.einsum_product("geom", O.clifford_conjugation(b), O.clifford_conjugation(a), metric)
    torch.testing.assert_close(lhs, rhs, rtol=1e-12, atol=1e-11)
    x = rand_mv(3, n, 35)
    torch.testing.assert_close(O.clifford_conjugation(x), O.reverse(O.grade_involution(x)), rtol=0, atol=0)
    torch.testing.assert_close(O.clifford_conjugation(x), O.grade_involution(O.reverse(x)), rtol=0, atol=0)


def test_wedge_of_vectors_is_antisymmetric_part():
    metric = (1, -1, 1, 0, 1)
    a, b = rand_mv(4, 5, 6, grade=1), rand_mv(4, 5, 7, grade=1)
    w = O.einsum_product("wedge", a, b, metric)
    half = 0.5 * (O.einsum_product("geom", a, b, metric) - O.einsum_product("geom", b, a, metric))
    torch.testing.assert_close(w, half, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("metric", [(1, 1, 1, 1, 1), (1, -1, 1, -1, 0), (0, 1, 1, -1, 1)])
def test_masks_are_grade_selections(metric):
    """For homogeneous A_r, B_s: wedge = <AB>_{r+s}, lc = <AB>_{s-r} (0 if r>s),
    rc = <AB>_{r-s} (0 if s>r), inner = <AB>_{|r-s|}."""
    n = 5
    for r, s in itertools.product(range(n + 1), repeat=2):
        A, B = rand_mv(2, n, 10 + r, grade=r), rand_mv(2, n, 20 + s, grade=s)
        AB = O.einsum_product("geom", A, B, metric)
        zero = torch.zeros_like(AB)
        exp_w = O.grade_projection(AB, r + s) if r + s <= n else zero
        exp_lc = O.grade_projection(AB, s - r) if s >= r else zero
        exp_rc = O.grade_projection(AB, r - s) if r >= s else zero
        exp_in = O.grade_projection(AB, abs(r - s))
        for op, exp in (("wedge", exp_w), ("lc", exp_lc), ("rc", exp_rc), ("inner", exp_in)):
            torch.testing.assert_close(O.einsum_product(op, A, B, metric), exp, rtol=1e-12, atol=1e-12,
                                       msg=f"{op} r={r} s={s}")


@pytest.mark.parametrize("metric", [(1, 1, 1), (1, -1, 1), (-1, -1, 1, 1, -1)])
def test_dual_is_right_product_with_inverse_pseudoscalar(metric):
    n = len(metric)
    dim = 1 << n
    I = torch.zeros(1, dim, dtype=torch.float64)
    I[0, dim - 1] = 1.0
    isq = O.einsum_product("geom", I, I, metric)[0, 0]
    Iinv = I / isq
    x = rand_mv(3, n, 8)
    torch.testing.assert_close(O.dual(x, metric), O.einsum_product("geom", x, Iinv.expand_as(x), metric),
                               rtol=1e-12, atol=1e-12)


def test_regressive_known_answer_3d():
    # (e1^e2) v (e2^e3) in 3D Euclidean is proportional to e2 (the shared direction)
    metric = (1, 1, 1)
    a = torch.zeros(1, 8, dtype=torch.float64)
    b = torch.zeros(1, 8, dtype=torch.float64)
    a[0, 0b011] = 1.0
    b[0, 0b110] = 1.0
    r = O.einsum_product("regressive", a, b, metric)
    nz = torch.nonzero(r[0].abs() > 1e-12).flatten().tolist()
    assert nz == [0b010]
    # grade of a v b is r + s - n for blades
    for r_, s_ in itertools.product(range(4), repeat=2):
        A, B = rand_mv(1, 3, 30 + r_, grade=r_), rand_mv(1, 3, 40 + s_, grade=s_)
        out = O.einsum_product("regressive", A, B, metric)
        g = r_ + s_ - 3
        exp = O.grade_projection(out, g) if 0 <= g <= 3 else torch.zeros_like(out)
        torch.testing.assert_close(out, exp, rtol=0, atol=1e-12)


def test_norm_sq_identity():
    """norm_sq(x) == <x x~>_0 (reference tests/correctness/test_norm_sq.py:46-63)."""
    for metric in [(1,) * 5, (1, 1, -1, -1, 0), (-1, 0, 0, 1, 1)]:
        x = rand_mv(4, 5, 9)
        lhs = O.norm_sq(x, metric)
        rhs = O.einsum_product("geom", x, O.reverse(x), metric)[:, 0]
        torch.testing.assert_close(lhs, rhs, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("op", O.OPS)
def test_autograd_matches_adjoint_formulas(op):
    """ga[k] = sum_j s(k,j) b[j] gf[k^j], gb[k] = sum_i s(i,k) a[i] gf[i^k]
    (reference extensions/ga/geom_prod.py:155-169), with the op's (D,D) table
    obtained from the oracle by probing basis blades (not from its formula)."""
    n, metric = 4, (1, 1, -1, 1)
    dim = 1 << n
    eye = torch.eye(dim, dtype=torch.float64)
    # T[i, j, :] = op(e_i, e_j)
    T = torch.stack([O.einsum_product(op, eye[i:i + 1].expand(dim, dim), eye, metric) for i in range(dim)])
    a = rand_mv(3, n, 11).requires_grad_()
    b = rand_mv(3, n, 12).requires_grad_()
    gc = rand_mv(3, n, 13)
    c = O.einsum_product(op, a, b, metric)
    ga, gb = torch.autograd.grad(c, (a, b), gc)
    ga_ref = torch.einsum("ijk,bj,bk->bi", T, b.detach(), gc)
    gb_ref = torch.einsum("ijk,bi,bk->bj", T, a.detach(), gc)
    torch.testing.assert_close(ga, ga_ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(gb, gb_ref, rtol=1e-12, atol=1e-12)


def test_rotor_vector_action_is_expm():
    """Grade-1 action of ~R x R equals expm(-B), B = 2(M - M^T), M[i_m, j_m] = b_m
    (the matrix the reference exponentiates, kernels/rotor/eigh_exp.cu:283-288)."""
    n = 5
    g = torch.Generator().manual_seed(3)
    biv = 0.3 * torch.randn(1, n * (n - 1) // 2, generator=g, dtype=torch.float64)
    M = torch.zeros(n, n, dtype=torch.float64)
    for m, (i, j, _) in enumerate(O.bivector_blades(n)):
        M[i, j] = biv[0, m]
    B = 2 * (M - M.T)
    Q = O.vector_rotation_matrix(biv, n)
    np.testing.assert_allclose(Q.numpy(), scipy.linalg.expm(-B.numpy()), atol=1e-12)


def test_rotor_single_plane_closed_form():
    # b_01 = t: e0 -> cos(2t) e0 + sin(2t) e1
    n, t = 4, 0.37
    biv = torch.zeros(1, 6, dtype=torch.float64)
    biv[0, 0] = t
    x = torch.zeros(1, 16, dtype=torch.float64)
    x[0, 1] = 1.0
    y = O.apply_bivector(biv, x, n)
    exp = torch.zeros_like(y)
    exp[0, 1], exp[0, 2] = math.cos(2 * t), math.sin(2 * t)
    torch.testing.assert_close(y, exp, rtol=0, atol=1e-13)


def test_rotor_is_outermorphism_and_preserves_norm():
    n = 5
    g = torch.Generator().manual_seed(4)
    biv = 0.5 * torch.randn(1, 10, generator=g, dtype=torch.float64)
    R = O.rotor_from_bivector(biv, n)
    one = O.einsum_product("geom", O.reverse(R), R)
    exp_one = torch.zeros_like(one)
    exp_one[0, 0] = 1
    torch.testing.assert_close(one, exp_one, rtol=0, atol=1e-12)
    x = rand_mv(3, n, 14)
    y = O.apply_bivector(biv, x, n)
    torch.testing.assert_close(O.norm_sq(y, None), O.norm_sq(x, None), rtol=1e-12, atol=1e-12)
    for k in range(n + 1):
        torch.testing.assert_close(O.apply_bivector(biv, O.grade_projection(x, k), n), O.grade_projection(y, k),
                                   rtol=1e-11, atol=1e-12)
    # (Q a) ^ (Q b) for vectors a, b: the action on a bivector blade
    Q = O.vector_rotation_matrix(biv, n)
    va, vb = rand_mv(1, n, 15, grade=1), rand_mv(1, n, 16, grade=1)
    def rot_vec(v):
        coeffs = torch.stack([v[0, 1 << a] for a in range(n)])
        out = torch.zeros_like(v)
        qv = Q @ coeffs
        for a in range(n):
            out[0, 1 << a] = qv[a]
        return out
    lhs = O.apply_bivector(biv, O.einsum_product("wedge", va, vb), n)
    rhs = O.einsum_product("wedge", rot_vec(va), rot_vec(vb))
    torch.testing.assert_close(lhs, rhs, rtol=1e-11, atol=1e-12)


def test_normalize_metric():
    assert O.normalize_metric(3, None) == (1, 1, 1)
    with pytest.raises(ValueError):
        O.normalize_metric(3, (1, 1))
    with pytest.raises(ValueError):
        O.normalize_metric(2, (1, 2))


# ── the reference's Givens cs chain ─────────────────────────────────────────

def _givens_matrix(n, p, q, c, s):
    """Row rotation the factorisation applies for one plane:
    A[p] <- c A[p] + s A[q], A[q] <- -s A[p] + c A[q] (s = -s_raw)."""
    G = torch.eye(n, dtype=torch.float64)
    G[p, p], G[p, q], G[q, p], G[q, q] = c, s, -s, c
    return G


@pytest.mark.parametrize("n,seed,scale", [(5, 1, 0.3), (7, 2, 1.0), (8, 3, 2.5)])
def test_givens_factor_reconstructs_rotation(n, seed, scale):
    """R = prod over planes (lex order) of G_k^T, i.e. G_C ... G_1 R = I, with
    c^2 + s^2 = 1 per plane: the factorisation the cs pairs describe, checked by
    rebuilding R from cs alone (the storage is reversed: plane k at C-1-k)."""
    g = torch.Generator().manual_seed(seed)
    biv = scale * torch.randn(1, n * (n - 1) // 2, generator=g, dtype=torch.float64)
    R = O.rotation_matrix(biv, n)
    torch.testing.assert_close(R @ R.T, torch.eye(n, dtype=torch.float64), rtol=0, atol=1e-12)
    cs = O.givens_factor(R)
    pairs = O.plane_pairs(n)
    C = len(pairs)
    assert cs.shape == (C, 2)
    torch.testing.assert_close(cs.pow(2).sum(1), torch.ones(C, dtype=torch.float64), rtol=0, atol=1e-13)
    A = R.clone()
    for k, (p, q) in enumerate(pairs):
        A = _givens_matrix(n, p, q, float(cs[C - 1 - k, 0]), float(cs[C - 1 - k, 1])) @ A
        assert abs(float(A[q, p])) < 1e-12        # the plane's entry is eliminated
        assert float(A[p, p]) >= -1e-12           # r >= 0 convention
    torch.testing.assert_close(A, torch.eye(n, dtype=torch.float64), rtol=0, atol=1e-11)
    # R^T is the grade-1 action of the sandwich (pinned to scipy's expm(-B) above)
    torch.testing.assert_close(R.T, O.vector_rotation_matrix(biv, n), rtol=0, atol=1e-11)


@pytest.mark.parametrize("n", [4, 5, 7])
def test_givens_chain_of_factors_is_the_sandwich(n):
    """apply_rotor(compile_bivector(b), x) of the reference equals ~R x R: the
    chain of the factors against the independently pinned sandwich oracle."""
    g = torch.Generator().manual_seed(20 + n)
    biv = 0.5 * torch.randn(1, n * (n - 1) // 2, generator=g, dtype=torch.float64)
    x = torch.randn(3, 1 << n, generator=g, dtype=torch.float64)
    cs = O.compile_bivector_cs(biv, n)
    torch.testing.assert_close(O.givens_chain_apply(cs, x, n), O.apply_bivector(biv, x, n), rtol=0, atol=1e-12)


def test_givens_chain_single_plane_closed_form():
    """One plane (p, q) with (c, s) and every other plane the identity: the
    vector e_p goes to c e_p - s e_q, e_q to s e_p + c e_q, and the bivector
    e_p e_r (r outside the plane) to c e_p e_r - s e_q e_r (a sign from moving
    e_q past generators between p and q does not arise for r > q)."""
    n = 5
    pairs = O.plane_pairs(n)
    C = len(pairs)
    p, q, r = 1, 3, 4
    k = pairs.index((p, q))
    c, s = math.cos(0.7), math.sin(0.7)
    cs = torch.zeros(C, 2, dtype=torch.float64)
    cs[:, 0] = 1.0
    cs[C - 1 - k] = torch.tensor([c, s], dtype=torch.float64)
    x = torch.zeros(3, 1 << n, dtype=torch.float64)
    x[0, 1 << p] = 1.0
    x[1, 1 << q] = 1.0
    x[2, (1 << p) | (1 << r)] = 1.0
    y = O.givens_chain_apply(cs, x, n)
    exp = torch.zeros_like(y)
    exp[0, 1 << p], exp[0, 1 << q] = c, -s
    exp[1, 1 << p], exp[1, 1 << q] = s, c
    exp[2, (1 << p) | (1 << r)], exp[2, (1 << q) | (1 << r)] = c, -s
    torch.testing.assert_close(y, exp, rtol=0, atol=1e-15)


def test_givens_chain_backward_ref_is_autograd_for_unit_pairs():
    """The reference's backward (inputs rebuilt with the transposed pair map)
    equals the exact derivative of the chain when every (c, s) is a unit pair;
    for non-unit pairs it does not (the transposed map is then not the inverse),
    which is the reference's behaviour this restatement keeps."""
    n = 5
    C = n * (n - 1) // 2
    g = torch.Generator().manual_seed(9)
    ang = torch.randn(C, generator=g, dtype=torch.float64)
    x = torch.randn(4, 1 << n, generator=g, dtype=torch.float64)
    gy = torch.randn(4, 1 << n, generator=g, dtype=torch.float64)
    for unit in (True, False):
        cs = torch.stack([ang.cos(), ang.sin()], 1)
        if not unit:
            cs = cs * (1.0 + 0.3 * torch.rand(C, 1, generator=g, dtype=torch.float64))
        cs_l = cs.clone().requires_grad_()
        x_l = x.clone().requires_grad_()
        y = O.givens_chain_apply(cs_l, x_l, n)
        y.backward(gy)
        gcs, gx = O.givens_chain_backward_ref(cs, y.detach(), gy, n)
        torch.testing.assert_close(gx, x_l.grad, rtol=0, atol=1e-12)   # gx: exact for any pairs
        if unit:
            torch.testing.assert_close(gcs, cs_l.grad, rtol=0, atol=1e-11)
        else:
            assert float((gcs - cs_l.grad).abs().max()) > 1e-3


@pytest.mark.parametrize("metric", [(1, 1, 1, 1, 1), (1, -1, 1, 0, -1), (0, 1, 1, -1)])
def test_inverse_dense_is_two_sided_inverse(metric):
    n = len(metric)
    x = rand_mv(3, n, 50)
    x[:, 0] += 3.0
    y = O.inverse_dense(x, metric)
    one = torch.zeros_like(x)
    one[:, 0] = 1.0
    torch.testing.assert_close(O.einsum_product("geom", x, y, metric), one, rtol=0, atol=1e-12)
    torch.testing.assert_close(O.einsum_product("geom", y, x, metric), one, rtol=0, atol=1e-12)


@pytest.mark.parametrize("op", ["geom", "wedge", "inner", "lc", "rc"])
def test_product_coefficients_equal_einsum(op):
    metric = (1, -1, 0, 1, -1)
    a, b = rand_mv(2, 5, 60), rand_mv(2, 5, 61)
    full = O.einsum_product(op, a, b, metric)
    ks = list(range(32))
    torch.testing.assert_close(O.product_coefficients(op, a, b, metric, ks), full, rtol=0, atol=1e-12)
