"""GPU parity of the six binary products (forward + fused backward) against the
fp64 CPU oracle on identical seeded inputs. Bar: normwise relative error
max|y - y_ref| / max|y_ref| <= 1e-5 for values and both gradients (the
tolerance BASELINE.json's north star states)."""
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


def seeded(b, n, seed, count):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(b, 1 << n, generator=g) for _ in range(count)]


def run_case(op, metric, batch, seed=0):
    n = len(metric)
    a, b, gc = seeded(batch, n, seed, 3)
    ad = a.cuda().requires_grad_()
    bd = b.cuda().requires_grad_()
    c = cc.products.product(op, ad, bd, metric)
    c.backward(gc.cuda())
    a64 = a.double().requires_grad_()
    b64 = b.double().requires_grad_()
    c64 = O.einsum_product(op, a64, b64, metric)
    c64.backward(gc.double())
    print(f"[case] op={op} metric={metric} batch={batch}", flush=True)
    return rel_err(c, c64), rel_err(ad.grad, a64.grad), rel_err(bd.grad, b64.grad)


# blocked-path metrics (low 4 generators all +1 / all -1, no null there) and
# generic-path metrics (n < 4, mixed or null low generators)
METRICS = [
    (1, 1, 1, 1, 1),
    (-1, -1, -1, -1, -1),
    (1, 1, 1, 1, -1),
    (1, 1, 1, 1, 0),
    (1, 1, 1, 1, 1, -1, 0),
    (1, 1, 1, 1, 1, 1, 1, 1),
    (1, 1, 1, -1, 0),          # generic: mixed low generators
    (1, 1, 0),                 # generic: n < 4
    (-1, 1, -1, 1, 1, 1),      # generic
    (1,) * 9 + (0,),           # C5 signature
]


@pytest.mark.parametrize("metric", METRICS, ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
@pytest.mark.parametrize("op", O.OPS)
def test_product_parity(op, metric):
    if op == "regressive" and 0 in metric:
        pytest.skip("regressive undefined for degenerate metrics")
    batch = 8 if len(metric) >= 10 else 37   # odd batch: partial workgroups
    e = run_case(op, metric, batch)
    assert max(e) <= TOL, e


def test_c1_cl50_geom_forward():
    """Cl(5,0) GP forward, batch 1024, seed 0."""
    g = torch.Generator().manual_seed(0)
    a = torch.randn(1024, 32, generator=g)
    b = torch.randn(1024, 32, generator=g)
    cl = cc.CliffordAlgebra([1] * 5, device="cuda")
    c = cl.geom_prod(a.cuda(), b.cuda())
    ref = O.einsum_product("geom", a.double(), b.double(), (1,) * 5)
    assert rel_err(c, ref) <= TOL


def test_c2_cl61_six_products_full_batch():
    """Cl(6,1), batch 65536, all six products fwd + bwd,
    upstream gradient all-ones. The oracle checks a 2048-row sample (first,
    last and strided rows); the full batch is checked by bilinearity."""
    metric = (1, 1, 1, 1, 1, 1, -1)
    g = torch.Generator().manual_seed(0)
    a = torch.randn(65536, 128, generator=g)
    b = torch.randn(65536, 128, generator=g)
    rows = torch.cat([torch.arange(0, 1024), torch.arange(65536 - 512, 65536), torch.arange(1024, 65536 - 512, 127)])
    cl = cc.CliffordAlgebra(metric, device="cuda")
    ad = a.cuda()
    bd = b.cuda()
    for op, meth in (("geom", cl.geom_prod), ("wedge", cl.wedge_prod), ("inner", cl.inner_prod),
                     ("lc", cl.left_contraction), ("rc", cl.right_contraction), ("regressive", cl.regressive_prod)):
        x = ad.clone().requires_grad_()
        y = bd.clone().requires_grad_()
        c = meth(x, y)
        c.backward(torch.ones_like(c))
        a64 = a[rows].double().requires_grad_()
        b64 = b[rows].double().requires_grad_()
        c64 = O.einsum_product(op, a64, b64, metric)
        c64.backward(torch.ones_like(c64))
        rs = rows.cuda()
        assert rel_err(c[rs], c64) <= TOL, op
        assert rel_err(x.grad[rs], a64.grad) <= TOL, op
        assert rel_err(y.grad[rs], b64.grad) <= TOL, op
        # bilinearity over the whole batch: op(a, b + 2a) = op(a, b) + 2 op(a, a)
        with torch.no_grad():
            lhs = meth(ad, bd + 2 * ad)
            rhs = c + 2 * meth(ad, ad)
            assert rel_err(lhs, rhs) <= 1e-5, op


def test_c5_degenerate_n10():
    """Cl(9,0,1), batch 16384. The left contraction fwd + bwd
    on its own (seeded upstream gradient, so its gradients are isolated), and the
    geometric product fwd + bwd with norm_sq and grade_projection(2) of it in
    the loss. Checks: the oracle on 8 rows of the batch (values and all
    gradients); the full batch by bilinearity of both forwards; bitwise row
    independence of both forwards and backwards (rows computed inside the full
    batch equal the same rows computed in a batch of their own, large enough to
    run on the same kernels)."""
    metric = (1,) * 9 + (0,)
    g = torch.Generator().manual_seed(0)
    B = 16384
    a = torch.randn(B, 1024, generator=g)
    b = torch.randn(B, 1024, generator=g)
    glc = torch.randn(B, 1024, generator=g)
    cl = cc.CliffordAlgebra(metric, device="cuda")
    ad, bd, glcd = a.cuda(), b.cuda(), glc.cuda()
    rows = torch.tensor([0, 1, 2, 3, 100, 5000, 9999, B - 1])
    rs = rows.cuda()
    a64 = a[rows].double().requires_grad_()
    b64 = b[rows].double().requires_grad_()

    print("[case] C5 lc fwd+bwd", flush=True)
    x = ad.clone().requires_grad_()
    y = bd.clone().requires_grad_()
    lc = cl.left_contraction(x, y)
    lc.backward(glcd)
    lc64 = O.einsum_product("lc", a64, b64, metric)
    lc64.backward(glc[rows].double())
    assert rel_err(lc[rs], lc64) <= TOL
    assert rel_err(x.grad[rs], a64.grad) <= TOL
    assert rel_err(y.grad[rs], b64.grad) <= TOL
    lc_ga, lc_gb = x.grad, y.grad

    print("[case] C5 geom + norm_sq + grade_projection fwd+bwd", flush=True)
    a64.grad = None
    b64.grad = None
    x = ad.clone().requires_grad_()
    y = bd.clone().requires_grad_()
    gp = cl.geom_prod(x, y)
    ns = cl.norm_sq(gp)
    pr = cl.grade_projection(gp, 2)
    (gp.sum() + ns.sum() + pr.sum()).backward()
    gp64 = O.einsum_product("geom", a64, b64, metric)
    ns64 = O.norm_sq(gp64, metric)
    pr64 = O.grade_projection(gp64, 2)
    (gp64.sum() + ns64.sum() + pr64.sum()).backward()
    assert rel_err(gp[rs], gp64) <= TOL
    assert rel_err(ns[rs], ns64) <= TOL
    assert rel_err(pr[rs], pr64) <= TOL
    assert rel_err(x.grad[rs], a64.grad) <= TOL
    assert rel_err(y.grad[rs], b64.grad) <= TOL
    gp_ga, gp_gb = x.grad, y.grad

    print("[case] C5 full-batch bilinearity", flush=True)
    with torch.no_grad():
        for meth, c in ((cl.geom_prod, gp), (cl.left_contraction, lc)):
            lhs = meth(ad, bd + 2 * ad)
            rhs = c + 2 * meth(ad, ad)
            assert rel_err(lhs, rhs) <= TOL

    print("[case] C5 row independence", flush=True)
    idx = torch.tensor([0, 5, 6, 7, 4097, 8191, 12345, B - 3, B - 2, B - 1], device="cuda")
    # the rows again inside a batch of 520 (52 copies): large enough for the kernels of the full batch
    # (fewer than 512 rows of n = 10 take the small-batch kernels)
    rep = idx.repeat(52)
    xs = ad[rep].clone().requires_grad_()
    ys = bd[rep].clone().requires_grad_()
    lcs = cl.left_contraction(xs, ys)
    lcs.backward(glcd[rep])
    k = len(idx)
    assert torch.equal(lcs[:k], lc[idx].detach())
    assert torch.equal(xs.grad[:k], lc_ga[idx]) and torch.equal(ys.grad[:k], lc_gb[idx])
    xs = ad[idx].clone().requires_grad_()
    ys = bd[idx].clone().requires_grad_()
    gps = cl.geom_prod(xs, ys)
    (gps.sum() + cl.norm_sq(gps).sum() + cl.grade_projection(gps, 2).sum()).backward()
    assert torch.equal(gps, gp[idx].detach())
    assert torch.equal(xs.grad, gp_ga[idx]) and torch.equal(ys.grad, gp_gb[idx])


def test_headline_shape_row_independence():
    """Headline shape Cl(8,0), batch 262144: rows computed at full batch equal
    the same rows computed alone (size-independent property), and a sample of
    rows matches the oracle."""
    g = torch.Generator().manual_seed(0)
    B = 262144
    a = torch.randn(B, 256, generator=g).cuda()
    b = torch.randn(B, 256, generator=g).cuda()
    c = cc.geom_prod(a, b)
    idx = torch.tensor([0, 17, 65535, 131072, B - 1], device="cuda")
    c_small = cc.geom_prod(a[idx].contiguous(), b[idx].contiguous())
    assert torch.equal(c[idx], c_small)
    ref = O.einsum_product("geom", a[idx].double().cpu(), b[idx].double().cpu())
    assert rel_err(c[idx], ref) <= TOL


def test_edge_batches_and_layouts():
    cl = cc.CliffordAlgebra([1] * 6, device="cuda")
    empty = torch.empty(0, 64, device="cuda")
    assert cl.geom_prod(empty, empty).shape == (0, 64)
    one = torch.randn(1, 64, device="cuda")
    ref = O.einsum_product("geom", one.double().cpu(), one.double().cpu())
    assert rel_err(cl.geom_prod(one, one), ref) <= TOL
    # free functions accept non-contiguous inputs and leading dims
    x = torch.randn(64, 3, device="cuda").t()   # (3, 64) non-contiguous
    y = torch.randn(3, 64, device="cuda")
    got = cc.geom_prod(x, y)
    assert rel_err(got, O.einsum_product("geom", x.double().cpu(), y.double().cpu())) <= TOL
    z = torch.randn(2, 5, 64, device="cuda")
    got = cc.wedge_prod(z, z)
    assert got.shape == (2, 5, 64)


def test_validation_errors():
    cl = cc.CliffordAlgebra([1] * 5, device="cuda")
    a = torch.randn(4, 32, device="cuda")
    with pytest.raises(ValueError, match="must be 2D"):
        cl.geom_prod(a.view(4, 2, 16), a.view(4, 2, 16))
    with pytest.raises(ValueError, match="last dim"):
        cl.geom_prod(a[:, :16].contiguous(), a[:, :16].contiguous())
    with pytest.raises(ValueError, match="dtype"):
        cl.geom_prod(a.double(), a.double())
    with pytest.raises(ValueError, match="contiguous"):
        cl.geom_prod(a.t().contiguous().t(), a)
    with pytest.raises(ValueError, match="degenerate"):
        cc.CliffordAlgebra([1, 1, 1, 1, 0], device="cuda").regressive_prod(a, a)
    with pytest.raises(ValueError, match="grade must be in"):
        cl.grade_projection(a, 6)


@pytest.mark.parametrize("n", [5, 7])
def test_gradcheck_signatures(n):
    """The reference's gradcheck spread (tests/_gradcheck.py:9-19): six
    signatures per n, fp64 finite differences through the fp32 kernels."""
    sigs = [(1,) * n, (-1,) * n, (1,) * (n - 1) + (-1,), (1,) * (n // 2) + (-1,) * (n - n // 2),
            (1,) * (n - 1) + (0,), (1,) * (n - 2) + (-1, 0)]
    tol = max(1e-3, (1 << n) * 3e-5)
    for metric in sigs:
        for op in O.OPS:
            if op == "regressive" and 0 in metric:
                continue
            torch.manual_seed(0)
            a = torch.randn(2, 1 << n, dtype=torch.float64, device="cuda", requires_grad=True)
            b = torch.randn(2, 1 << n, dtype=torch.float64, device="cuda", requires_grad=True)
            fn = lambda x, y: cc.products.product(op, x.float(), y.float(), metric).double()  # noqa: E731
            assert torch.autograd.gradcheck(fn, (a, b), eps=1e-3, atol=tol, rtol=tol, nondet_tol=tol), (op, metric)


REAL_TYPE = [(1,) * 8, (1,) * 4 + (-1,) * 4, (1,) * 5 + (-1,) * 3, (-1,) * 8, (1, 1, 1, -1, -1, -1), (1, 1, 1, 1),
             (-1, 1, 1, -1)]


@pytest.mark.parametrize("metric", REAL_TYPE, ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
def test_matrix_path_geom_parity(metric):
    """Real-matrix-type signatures take the matrix-representation kernels for
    the geometric product; check them against the oracle, forward and backward."""
    e = run_case("geom", metric, 37)
    assert max(e) <= TOL, e


def test_matrix_path_equals_direct_path_full_batch(clf_env):
    """Headline shape: the matrix-representation kernels and the per-term
    kernels (an independent algorithm, forced with CLF_GEOM_PATH=direct) agree
    at batch 262144, values and both gradients."""
    g = torch.Generator().manual_seed(1)
    B = 262144
    a = torch.randn(B, 256, generator=g).cuda()
    b = torch.randn(B, 256, generator=g).cuda()
    gc = torch.randn(B, 256, generator=g).cuda()

    def run():
        x = a.clone().requires_grad_()
        y = b.clone().requires_grad_()
        c = cc.geom_prod(x, y)
        c.backward(gc)
        return c.detach(), x.grad, y.grad

    c1, ga1, gb1 = run()
    clf_env.setenv("CLF_GEOM_PATH", "direct")
    c2, ga2, gb2 = run()
    clf_env.delenv("CLF_GEOM_PATH")
    for u, v in ((c1, c2), (ga1, ga2), (gb1, gb2)):
        assert rel_err(u, v) <= TOL


SPLIT_TYPE = [(1,) * 9, (1,) * 5 + (-1,) * 4, (1,) + (-1,) * 8, (1, -1) * 4 + (1,), (1,) * 9 + (0,),
              (1,) * 5 + (-1,) * 4 + (0,)]


@pytest.mark.parametrize("metric", SPLIT_TYPE, ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
@pytest.mark.parametrize("batch", [1, 37])
def test_split_path_geom_parity(metric, batch):
    """n = 9 signatures with p - q = 1 (mod 8) and their extension by a null
    e_9 take the split-representation kernels for the geometric product
    (odd batches exercise the clamped last row of a two-row group)."""
    e = run_case("geom", metric, batch)
    assert max(e) <= TOL, e


def test_split_path_equals_direct_path_c5_full_batch(clf_env):
    """C5 shape (Cl(9,0,1), batch 16384): the split-representation kernels and
    the per-term kernels agree on the whole batch, values and both gradients."""
    metric = (1,) * 9 + (0,)
    g = torch.Generator().manual_seed(2)
    B = 16384
    a = torch.randn(B, 1024, generator=g).cuda()
    b = torch.randn(B, 1024, generator=g).cuda()
    gc = torch.randn(B, 1024, generator=g).cuda()

    def run():
        x = a.clone().requires_grad_()
        y = b.clone().requires_grad_()
        c = cc.geom_prod(x, y, metric)
        c.backward(gc)
        return c.detach(), x.grad, y.grad

    r1 = run()
    clf_env.setenv("CLF_GEOM_PATH", "direct")
    r2 = run()
    clf_env.delenv("CLF_GEOM_PATH")
    for u, v in zip(r1, r2):
        assert rel_err(u, v) <= TOL


BAL_METRICS = [
    (1,) * 4,
    (-1,) * 5,
    (1,) * 6 + (-1,),           # C2
    (1,) * 4 + (0, -1, 1, 0),
    (-1,) * 4 + (1, -1, 1, 1, -1),
    (1,) * 9 + (0,),            # C5
]


def _grads(op, a, b, gc, metric, need_a=True, need_b=True):
    ad = a.clone().requires_grad_(need_a)
    bd = b.clone().requires_grad_(need_b)
    c = cc.products.product(op, ad, bd, metric)
    c.backward(gc)
    return c.detach(), (ad.grad if need_a else None), (bd.grad if need_b else None)


@pytest.mark.parametrize("metric", BAL_METRICS, ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
@pytest.mark.parametrize("op", O.OPS)
def test_balanced_kernels_match_blocked_and_oracle(op, metric, clf_env):
    """The balanced kernels (default for the masked products at 4 <= n <= 10,
    forced for geom) give the one-lane-per-output kernels' results on batches
    that end inside a row group, for both gradients and each one alone; small
    batches also against the oracle."""
    if op == "regressive" and 0 in metric:
        pytest.skip("regressive undefined for degenerate metrics")
    n = len(metric)
    R = 1 << (10 - n)
    for batch in (1, R + 3, 4 * 64 * R + 5):
        a, b, gc = (t.cuda() for t in seeded(batch, n, batch + n, 3))
        print(f"[case] balanced op={op} metric={metric} batch={batch}", flush=True)
        clf_env.setenv("CLF_PRODUCT_PATH", "balanced")
        c, ga, gb = _grads(op, a, b, gc, metric)
        _, ga1, _ = _grads(op, a, b, gc, metric, need_b=False)
        _, _, gb1 = _grads(op, a, b, gc, metric, need_a=False)
        clf_env.setenv("CLF_PRODUCT_PATH", "blocked")
        c0, ga0, gb0 = _grads(op, a, b, gc, metric)
        clf_env.delenv("CLF_PRODUCT_PATH")
        assert rel_err(c, c0) <= TOL and rel_err(ga, ga0) <= TOL and rel_err(gb, gb0) <= TOL
        assert torch.equal(ga1, ga) and torch.equal(gb1, gb)
        if batch <= 64:
            a64, b64 = a.double().cpu().requires_grad_(), b.double().cpu().requires_grad_()
            c64 = O.einsum_product(op, a64, b64, metric)
            c64.backward(gc.double().cpu())
            assert max(rel_err(c, c64), rel_err(ga, a64.grad), rel_err(gb, b64.grad)) <= TOL


@pytest.mark.parametrize("metric", [m for m in SPLIT_TYPE if len(m) == 10],
                         ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
def test_split_fused_matches_pair_sums(metric, clf_env):
    """n = 10 with a null e_9: the fused kernels (one launch per direction and
    gradient) equal the separate pair-sum launches, on batches with a partial
    two-row group, for both gradients and each one alone."""
    for batch in (1, 3, 2 * 2048 * 4 + 3):
        a, b, gc = (t.cuda() for t in seeded(batch, 10, batch, 3))
        print(f"[case] split fused metric={metric} batch={batch}", flush=True)
        c, ga, gb = _grads("geom", a, b, gc, metric)
        _, ga1, _ = _grads("geom", a, b, gc, metric, need_b=False)
        _, _, gb1 = _grads("geom", a, b, gc, metric, need_a=False)
        clf_env.setenv("CLF_SPLIT_PATH", "pairs")
        c0, ga0, gb0 = _grads("geom", a, b, gc, metric)
        clf_env.delenv("CLF_SPLIT_PATH")
        assert rel_err(c, c0) <= TOL and rel_err(ga, ga0) <= TOL and rel_err(gb, gb0) <= TOL
        assert torch.equal(ga1, ga) and torch.equal(gb1, gb)


ODD7 = [(1,) * (7 - q) + (-1,) * q for q in range(8)] + [(-1, 1, -1, 1, 1, -1, 1)]


@pytest.mark.parametrize("metric", ODD7, ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
@pytest.mark.parametrize("batch", [1, 6, 37])
def test_n7_matrix_path_geom_parity(metric, batch):
    """Every non-degenerate n = 7 signature takes the 16 x 16 representation
    kernels for the geometric product (two matrices per row when q is odd, one
    when q is even); batches that end inside a four-row group exercise the
    clamped rows."""
    e = run_case("geom", metric, batch)
    assert max(e) <= TOL, e


@pytest.mark.parametrize("metric", [(1,) * 6 + (-1,), (1,) * 7], ids=["C2", "+++++++"])
def test_n7_matrix_path_equals_direct_path(metric, clf_env):
    """C2 shape (batch 65536) and a ragged batch: the n = 7 representation
    kernels give the per-term kernels' values and gradients (an independent
    algorithm, CLF_GEOM_PATH=direct), also with one gradient requested; the
    results are not bit-identical, so the matrix path did run."""
    for B in (65536, 4099):
        a, b, gc = (t.cuda() for t in seeded(B, 7, B, 3))
        print(f"[case] n7 vs direct metric={metric} batch={B}", flush=True)
        c, ga, gb = _grads("geom", a, b, gc, metric)
        _, ga1, _ = _grads("geom", a, b, gc, metric, need_b=False)
        _, _, gb1 = _grads("geom", a, b, gc, metric, need_a=False)
        clf_env.setenv("CLF_GEOM_PATH", "direct")
        c0, ga0, gb0 = _grads("geom", a, b, gc, metric)
        clf_env.delenv("CLF_GEOM_PATH")
        assert rel_err(c, c0) <= TOL and rel_err(ga, ga0) <= TOL and rel_err(gb, gb0) <= TOL
        assert torch.equal(ga1, ga) and torch.equal(gb1, gb)
        assert not torch.equal(c, c0)


FRAME_METRICS = [(1,) * 4, (-1,) * 4, (1,) * 4 + (-1,), (-1,) * 5 + (1,), (1,) * 6 + (-1,), (-1,) * 7,
                 (1, 1, 1, 1, -1, 1, -1), (-1, -1, -1, -1, 1, -1, 1), (1,) * 8, (1,) * 7 + (-1,),
                 (-1, -1, -1, -1, 1, -1, 1, -1)]


@pytest.mark.parametrize("metric", FRAME_METRICS, ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
def test_inner_frame_kernels_match_oracle_and_blocked(metric, clf_env):
    """The inner product's one-lane-per-output kernels (backward for
    4 <= n <= 8 with per-lane frames, forward at n = 7 with helper lanes):
    values and each gradient alone or both against the fp64 oracle, batches
    that end inside a group of rows (and a single row), and equal to the
    blocked kernels (CLF_PRODUCT_PATH=blocked) within rounding."""
    from cliffordcuda_amd import _lib, products
    from cliffordcuda_amd._validate import metric_masks
    n = len(metric)
    neg, nul = metric_masks(metric)
    R = 1024 >> n
    for batch in (1, R - 1, 3 * R + 5, 4 * 64 * R + 7):
        print(f"[case] inner frame metric={metric} batch={batch}", flush=True)
        a, b, gc = seeded(batch, n, batch + n, 3)
        a64 = a.double().requires_grad_()
        b64 = b.double().requires_grad_()
        c64 = O.einsum_product("inner", a64, b64, metric)
        c64.backward(gc.double())
        ad, bd, gd = a.cuda(), b.cuda(), gc.cuda()
        c = products.product("inner", ad, bd, metric)
        assert rel_err(c, c64) <= TOL
        got = {}
        for need in ((True, True), (True, False), (False, True)):
            ga, gb = products._product_bwd(_lib.OP_CODES["inner"], n, neg, nul, ad, bd, gd, *need)
            assert (ga is None) != need[0] and (gb is None) != need[1]
            if ga is not None:
                assert rel_err(ga, a64.grad) <= TOL
            if gb is not None:
                assert rel_err(gb, b64.grad) <= TOL
            got[need] = (ga, gb)
        # each gradient alone equals the one computed together with the other
        assert torch.equal(got[(True, False)][0], got[(True, True)][0])
        assert torch.equal(got[(False, True)][1], got[(True, True)][1])
        clf_env.setenv("CLF_PRODUCT_PATH", "blocked")
        cb = products.product("inner", ad, bd, metric)
        gab, gbb = products._product_bwd(_lib.OP_CODES["inner"], n, neg, nul, ad, bd, gd, True, True)
        clf_env.delenv("CLF_PRODUCT_PATH")
        assert rel_err(c, cb) <= 1e-6
        assert rel_err(got[(True, True)][0], gab) <= 1e-6 and rel_err(got[(True, True)][1], gbb) <= 1e-6


@pytest.mark.parametrize("metric", [m for m in FRAME_METRICS if len(m) == 7],
                         ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
@pytest.mark.parametrize("op", ["inner", "lc", "rc", "wedge", "regressive"])
def test_out7_forward_matches_oracle_and_blocked(op, metric, clf_env):
    """The n = 7 one-lane-per-output forward (inner: both halves, lc and rc:
    one half each, wedge: the lc half's schedule on complemented outputs)
    against the fp64 oracle on batches that end inside a group of eight rows,
    and equal to the blocked kernel within rounding."""
    from cliffordcuda_amd import products
    n = 7
    for batch in (1, 7, 29, 4 * 64 * 8 + 7):
        print(f"[case] out7 forward op={op} metric={metric} batch={batch}", flush=True)
        a, b = seeded(batch, n, batch + 3 * n, 2)
        c64 = O.einsum_product(op, a.double(), b.double(), metric)
        c = products.product(op, a.cuda(), b.cuda(), metric)
        assert rel_err(c, c64) <= TOL
        clf_env.setenv("CLF_PRODUCT_PATH", "blocked")
        cb = products.product(op, a.cuda(), b.cuda(), metric)
        clf_env.delenv("CLF_PRODUCT_PATH")
        assert rel_err(c, cb) <= 1e-6


@pytest.mark.parametrize("metric", FRAME_METRICS, ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
@pytest.mark.parametrize("op", ["lc", "rc", "wedge"])
def test_contraction_frame_backward_matches_oracle_and_blocked(op, metric, clf_env):
    """The contractions' and the wedge product's backward on the frame schedule
    (4 <= n <= 8, one accumulator per lane, a store at each mode's end): each
    gradient alone and
    both against the fp64 oracle, batches that end inside a group of rows (and
    a single row), each alone bitwise equal to both, and equal to the blocked
    kernels (CLF_PRODUCT_PATH=blocked) within rounding."""
    from cliffordcuda_amd import _lib, products
    from cliffordcuda_amd._validate import metric_masks
    n = len(metric)
    neg, nul = metric_masks(metric)
    R = 1024 >> n
    for batch in (1, R - 1, 3 * R + 5, 4 * 64 * R + 7):
        print(f"[case] contraction frame op={op} metric={metric} batch={batch}", flush=True)
        a, b, gc = seeded(batch, n, batch + 2 * n, 3)
        a64 = a.double().requires_grad_()
        b64 = b.double().requires_grad_()
        O.einsum_product(op, a64, b64, metric).backward(gc.double())
        ad, bd, gd = a.cuda(), b.cuda(), gc.cuda()
        got = {}
        for need in ((True, True), (True, False), (False, True)):
            ga, gb = products._product_bwd(_lib.OP_CODES[op], n, neg, nul, ad, bd, gd, *need)
            assert (ga is None) != need[0] and (gb is None) != need[1]
            if ga is not None:
                assert rel_err(ga, a64.grad) <= TOL
            if gb is not None:
                assert rel_err(gb, b64.grad) <= TOL
            got[need] = (ga, gb)
        assert torch.equal(got[(True, False)][0], got[(True, True)][0])
        assert torch.equal(got[(False, True)][1], got[(True, True)][1])
        clf_env.setenv("CLF_PRODUCT_PATH", "blocked")
        gab, gbb = products._product_bwd(_lib.OP_CODES[op], n, neg, nul, ad, bd, gd, True, True)
        clf_env.delenv("CLF_PRODUCT_PATH")
        assert rel_err(got[(True, True)][0], gab) <= 1e-6 and rel_err(got[(True, True)][1], gbb) <= 1e-6
