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


@pytest.mark.parametrize("metric", [(1,) * 8, (1,) * 4 + (-1,) * 4, (1,) * 5 + (-1,) * 3, (-1,) * 8,
                                    (1, -1, 1, 1, -1, -1, 1, -1)])
def test_rep16_lane_model(metric):
    """The lane dataflow of the m = 16 matrix-core kernels (xor-shuffled
    operands, transposed conversion, 4-block MFMA layout, stride-20 relayout)
    gives the oracle's product and gradients."""
    gens = R.find_generators(list(metric))
    label, sign = R.blade_tables(list(metric), gens)
    # the transposed conversion is the matrix transpose
    e = np.random.default_rng(0).standard_normal((2, 256))
    st = R.transpose_signs(label)
    np.testing.assert_allclose(R.to_matrix(e * np.array(st), label, sign, 16),
                               np.swapaxes(R.to_matrix(e, label, sign, 16), -1, -2), atol=1e-12)
    g = torch.Generator().manual_seed(3)
    a, b, gc = (torch.randn(4, 256, generator=g, dtype=torch.float64) for _ in range(3))
    aq, bq = a.clone().requires_grad_(), b.clone().requires_grad_()
    c_ref = O.einsum_product("geom", aq, bq, list(metric))
    c_ref.backward(gc)
    c = R.kernel16_fwd(a.numpy(), b.numpy(), label, sign)
    np.testing.assert_allclose(c, c_ref.detach().numpy(), atol=1e-10)
    ga, gb = R.kernel16_bwd(a.numpy(), b.numpy(), gc.numpy(), label, sign)
    np.testing.assert_allclose(ga, aq.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(gb, bq.grad.numpy(), atol=1e-10)
    # a bank-conflict-free odd-row offset exists for the Euclidean and split
    # tables (others fall back to offset 0: correct, with two-way conflicts)
    h = R.odd_row_xor(label)
    assert h % 4 == 0
    if metric in [(1,) * 8, (1,) * 4 + (-1,) * 4]:
        assert h > 0


@pytest.mark.parametrize("metric9", [(1,) * 9, (1,) * 5 + (-1,) * 4, (1,) + (-1,) * 8, (1, -1) * 4 + (1,)])
def test_split_rep9_product(metric9):
    """Cl(p', q') with p' - q' = 1 (mod 8) as M_16(R) + M_16(R): product, both
    gradients (pair-sum form) and the round trip equal the oracle."""
    label, sign = R.split_tables(metric9)
    assert len(set(label)) == 256 and all(label.count(l) == 2 for l in set(label[:4]))
    g = torch.Generator().manual_seed(9)
    a, b, gc = (torch.randn(2, 512, generator=g, dtype=torch.float64) for _ in range(3))
    aq, bq = a.clone().requires_grad_(), b.clone().requires_grad_()
    c_ref = O.einsum_product("geom", aq, bq, list(metric9))
    c_ref.backward(gc)
    an, bn, gn = a.numpy(), b.numpy(), gc.numpy()
    np.testing.assert_allclose(R.split_from_matrices(R.split_to_matrices(an, label, sign), label, sign), an,
                               atol=1e-12)
    c = R.pair_sum([(an, bn, False, False, False, False)], label, sign)
    np.testing.assert_allclose(c, c_ref.detach().numpy(), atol=1e-10)
    ga = R.pair_sum([(gn, bn, False, True, False, False)], label, sign)
    gb = R.pair_sum([(an, gn, True, False, False, False)], label, sign)
    np.testing.assert_allclose(ga, aq.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(gb, bq.grad.numpy(), atol=1e-10)
    # grade involution folded into the gather signs
    hat = np.array([(-1) ** bin(I).count("1") for I in range(512)])
    np.testing.assert_allclose(R.split_to_matrices(an, label, sign, hat=True),
                               R.split_to_matrices(an * hat, label, sign), atol=1e-12)


@pytest.mark.parametrize("metric9", [(1,) * 9, (1,) * 5 + (-1,) * 4])
def test_split_rep_degenerate10(metric9):
    """Cl(p', q', 1) with the null generator on bit 9 (the C5 signature for
    p' = 9): three pair sums forward, four backward, against the oracle."""
    metric = list(metric9) + [0]
    label, sign = R.split_tables(metric9)
    g = torch.Generator().manual_seed(10)
    a, b, gc = (torch.randn(2, 1024, generator=g, dtype=torch.float64) for _ in range(3))
    aq, bq = a.clone().requires_grad_(), b.clone().requires_grad_()
    c_ref = O.einsum_product("geom", aq, bq, metric)
    c_ref.backward(gc)
    c = R.degenerate10_fwd(a.numpy(), b.numpy(), label, sign)
    np.testing.assert_allclose(c, c_ref.detach().numpy(), atol=1e-9)
    ga, gb = R.degenerate10_bwd(a.numpy(), b.numpy(), gc.numpy(), label, sign)
    np.testing.assert_allclose(ga, aq.grad.numpy(), atol=1e-9)
    np.testing.assert_allclose(gb, bq.grad.numpy(), atol=1e-9)


ODD7 = [(1,) * (7 - q) + (-1,) * q for q in range(8)] + [(-1, 1, -1, 1, 1, -1, 1)]


@pytest.mark.parametrize("metric", ODD7, ids=lambda m: "".join({1: "+", -1: "-"}[x] for x in m))
def test_rep7_lane_model(metric):
    """n = 7 on the 16 x 16 representation (csrc/rep7.hip): pair mode exactly
    when q is odd; each lane holds 8 blades, all 128 once; the lane's small WHT
    times its sign pattern is the x-diagonal of phi(a) = sum_I a_I s(I) P(x_I, z_I)
    (and of phi(a^) in pair mode); the lane dataflow of the kernels (xor-shuffled
    operands, 4-block MFMA, stride-20 relayout, Q sums, pair combination) gives
    the oracle's product and both gradients."""
    metric = list(metric)
    pair, ent, zhi, gens = R.rep7_tables(metric)
    assert pair == (metric.count(-1) % 2 == 1)
    blades = sorted(e[0] for row in ent for e in row)
    assert blades == list(range(128))
    label, sign = R.blade_tables(metric, gens)
    for x in range(16):
        for k, (I, s, ts) in enumerate(ent[x]):
            assert label[I][0] == x and sign[I] == s
            if pair:
                assert R.popc(I) % 2 == k % 2 and label[I][1] == (zhi[x] << 2 | k // 2)
            else:
                assert label[I][1] == (zhi[x] << 3 | k)
    # generators: anticommuting, squares = metric
    for g, (gx, gz) in enumerate(gens):
        P = R.pauli(gx, gz, 16)
        np.testing.assert_allclose(P @ P, metric[g] * np.eye(16))
        for h in range(g):
            Q = R.pauli(*gens[h], 16)
            np.testing.assert_allclose(P @ Q, -Q @ P)
    rng = np.random.default_rng(len(metric) + metric.count(-1))
    a = rng.standard_normal((4, 128))
    T, Th = R.rep7_lane_T(a, ent, pair)
    W = R.rep7_expand(T, zhi, pair)
    hat = np.array([(-1) ** R.popc(I) for I in range(128)])
    for b_, (rowvals, Wrow) in enumerate([(a, W)] + ([(a * hat, R.rep7_expand(Th, zhi, pair))] if pair else [])):
        for r in range(2):
            M = sum(rowvals[r, I] * sign[I] * R.pauli(*label[I], 16) for I in range(128))
            Wd = np.array([[M[x ^ c, c] for c in range(16)] for x in range(16)])
            np.testing.assert_allclose(Wrow[r], Wd, atol=1e-12)
    # operands with the receiving lane's sign: zhi is linear, and each step's
    # operand differs from the xor-shuffled W by one lane-independent sign
    for x in range(16):
        for y in range(16):
            assert zhi[x ^ y] == zhi[x] ^ zhi[y]
    d = 2 if pair else 3
    for TT in [T] + ([Th] if pair else []):
        ratio = R.rep7_dest_operand(TT, zhi, pair) / R.xor_operand(R.rep7_expand(TT, zhi, pair))
        for k in range(16):
            uk = -1 if R.popc(zhi[k] & (k >> d)) & 1 else 1
            np.testing.assert_allclose(ratio[:, :, k], uk)
    b = rng.standard_normal((4, 128))
    gc = rng.standard_normal((4, 128))
    tabs = (pair, ent, zhi, gens)
    aq = torch.tensor(a, requires_grad=True)
    bq = torch.tensor(b, requires_grad=True)
    c_ref = O.einsum_product("geom", aq, bq, metric)
    c_ref.backward(torch.tensor(gc))
    np.testing.assert_allclose(R.kernel7_fwd(a, b, tabs), c_ref.detach().numpy(), atol=1e-10)
    ga, gb = R.kernel7_bwd(a, b, gc, tabs)
    np.testing.assert_allclose(ga, aq.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(gb, bq.grad.numpy(), atol=1e-10)


@pytest.mark.parametrize("pair", [True, False])
def test_rep7_operand_dpp_stages(pair):
    """The DPP stages of rep7.hip's operand builder move register k & low of
    lane x ^ k to lane x for every k."""
    plan = R.rep7_operand_dpp_plan(pair)
    assert sorted(plan) == list(range(16))
    for k, stages in plan.items():
        src = 0
        for st in stages:           # lane x reads lane x ^ s at each stage
            src ^= R.DPP_XOR[st]
        assert src == k, (k, stages)
        assert all(st in R.DPP_XOR for st in stages)


@pytest.mark.parametrize("metric9", [(1,) * 9, (-1,) * 4 + (1,) * 5, (1, -1, 1, -1, 1, -1, 1, -1, 1), (-1,) * 8 + (1,)])
def test_split_pair_blades_are_complements(metric9):
    """The fused n = 9, 10 kernels address the second blade of a label as the
    first xor 511 (csrc/rep_split.hip checks the host table for it): with the
    split labels, the blade I | e_8 sharing a label with I < 256 is (I ^ 255)
    | 256 for every p - q = 1 (mod 8) signature."""
    tabs = R.split_tables(list(metric9))
    assert tabs is not None
    label, _ = tabs
    first = {}
    for I in range(256):
        first[label[I]] = I
    assert len(first) == 256
    for J in range(256, 512):
        assert J == first[label[J]] ^ 511
