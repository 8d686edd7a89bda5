"""Products past the whole-row LDS limit (n = 12 .. 18, the reference's tiled
path, extensions/ga/geom_prod_tiled.py:1-31 and tests/correctness/
test_geom_prod_tiled.py): the tiled kernels against the whole-row kernels at
n = 12 (tiling forced with CLF_PRODUCT_PATH=tiled), against the
per-coefficient generic kernels (an independent algorithm, forced with
CLF_PRODUCT_PATH=generic) at n = 14, 16 and 17, and against the oracle at
n = 13 (every coefficient) and 17 (sampled coefficients).
Bar: normwise relative error <= 1e-5 for values and both gradients."""
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


def run(op, metric, a, b, gc, clf_env, path=None):
    if path:
        clf_env.setenv("CLF_PRODUCT_PATH", path)
    try:
        x = a.clone().requires_grad_()
        y = b.clone().requires_grad_()
        c = cc.products.product(op, x, y, metric)
        c.backward(gc)
        torch.cuda.synchronize()
    finally:
        if path:
            clf_env.delenv("CLF_PRODUCT_PATH")
    return c.detach(), x.grad, y.grad


def inputs(n, batch, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(batch, 1 << n, generator=g).cuda() for _ in range(3)]


def compare(r1, r2):
    return [rel_err(u, v) for u, v in zip(r1, r2)]


@pytest.mark.parametrize("metric", [(1,) * 12, (-1,) * 4 + (1, -1, 0, 1, 1, -1, 0, 1)], ids=["E12", "mixed12"])
@pytest.mark.parametrize("op", O.OPS)
def test_tiled_equals_whole_row_n12(op, metric, clf_env):
    if op == "regressive" and 0 in metric:
        pytest.skip("regressive is undefined for degenerate metrics")
    a, b, gc = inputs(12, 3, 12)
    print(f"[case] n=12 op={op} metric={metric}", flush=True)
    e = compare(run(op, metric, a, b, gc, clf_env, "blocked"), run(op, metric, a, b, gc, clf_env, "tiled"))
    assert max(e) <= TOL, e


@pytest.mark.parametrize("metric", [(1,) * 10 + (-1,), (1, 1, 1, 1, 1, -1, 0, 1, 1, -1, 1),
                                    (1, -1, 1, 0, 1, 1, -1, 1, 1, 1, -1)],
                         ids=["blocked11", "blocked11null", "mixed11"])
@pytest.mark.parametrize("op", O.OPS)
def test_n11_matches_oracle(op, metric):
    """n = 11 takes a launch plan of its own (whole-row blocked kernels with two
    waves per workgroup); every op forward and backward against the fp64
    oracle on an odd batch, for metrics on the blocked path (low generators
    alike, with and without a null generator above them) and on the
    per-coefficient path (mixed low generators)."""
    if op == "regressive" and 0 in metric:
        pytest.skip("regressive is undefined for degenerate metrics")
    g = torch.Generator().manual_seed(11)
    a, b, gc = (torch.randn(3, 1 << 11, generator=g) for _ in range(3))
    print(f"[case] n=11 op={op} metric={metric}", flush=True)
    ad = a.cuda().requires_grad_()
    bd = b.cuda().requires_grad_()
    c = cc.products.product(op, ad, bd, metric)
    c.backward(gc.cuda())
    a64 = a.double().requires_grad_()
    b64 = b.double().requires_grad_()
    c64 = O.einsum_product(op, a64, b64, metric)
    c64.backward(gc.double())
    e = [rel_err(c, c64), rel_err(ad.grad, a64.grad), rel_err(bd.grad, b64.grad)]
    assert max(e) <= TOL, e


@pytest.mark.parametrize("op", O.OPS)
def test_tiled_equals_generic_n14(op, clf_env):
    metric = (1,) * 11 + (-1, -1, 1) if op == "regressive" else (1,) * 11 + (-1, -1, 0)
    a, b, gc = inputs(14, 2, 14)
    print(f"[case] n=14 op={op}", flush=True)
    e = compare(run(op, metric, a, b, gc, clf_env), run(op, metric, a, b, gc, clf_env, "generic"))
    assert max(e) <= TOL, e


@pytest.mark.parametrize("op", ["geom", "lc"])
def test_tiled_equals_generic_n16(op, clf_env):
    """n = 16 (65536 components), Cl(13,2,1) as in the reference's largest
    gradient case."""
    metric = (1,) * 13 + (-1, -1, 0)
    a, b, gc = inputs(16, 1, 16)
    print(f"[case] n=16 op={op}", flush=True)
    e = compare(run(op, metric, a, b, gc, clf_env), run(op, metric, a, b, gc, clf_env, "generic"))
    assert max(e) <= TOL, e


def test_tiled_geom_matches_oracle_n13():
    """n = 13 (past the whole-row limit) against the fp64 oracle, one row."""
    metric = (1,) * 10 + (-1, -1, 1)
    g = torch.Generator().manual_seed(13)
    a = torch.randn(1, 1 << 13, generator=g)
    b = torch.randn(1, 1 << 13, generator=g)
    c = cc.products.product("geom", a.cuda(), b.cuda(), metric)
    ref = O.einsum_product("geom", a.double(), b.double(), metric)
    assert rel_err(c, ref) <= TOL


@pytest.mark.parametrize("op", ["geom", "lc", "wedge"])
@pytest.mark.parametrize("metric", [(1,) * 15 + (-1, 0), (1, -1) * 8 + (1,)], ids=["blocked17", "mixed17"])
def test_n17_matches_oracle_sample_and_generic(op, metric, clf_env):
    """n = 17 (131072 components, the reference's test_inverse.py:64 size):
    the default kernels (tiled for the blocked metric, per-coefficient for the
    mixed one) against the oracle on sampled output coefficients, and the
    tiled forward and backward against the per-coefficient kernels in full."""
    a, b, gc = inputs(17, 2, 17)
    print(f"[case] n=17 op={op} metric={metric}", flush=True)
    res = run(op, metric, a, b, gc, clf_env)
    ks = [0, 1, 5, 777, 65536, 131071]
    ref = O.product_coefficients(op, a.double().cpu(), b.double().cpu(), metric, ks)
    assert rel_err(res[0][:, ks], ref) <= TOL
    if metric[:4] == (1, 1, 1, 1):
        e = compare(res, run(op, metric, a, b, gc, clf_env, "generic"))
        assert max(e) <= TOL, e
    assert all(torch.isfinite(t).all() for t in res)


def test_public_api_past_limit():
    """The algebra object and the free functions accept n = 18 (past 16, where
    the earlier kernels stopped)."""
    metric = (1,) * 18
    cl = cc.CliffordAlgebra(metric, device="cuda")
    x = torch.randn(1, 1 << 18, device="cuda")
    e0 = torch.zeros(1, 1 << 18, device="cuda")
    e0[0, 1] = 1.0                        # the vector e_0
    y = cl.geom_prod(e0, cl.geom_prod(e0, x))   # e_0 e_0 x = x (e_0^2 = +1)
    assert rel_err(y, x) <= TOL
