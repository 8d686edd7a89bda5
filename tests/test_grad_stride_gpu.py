"""Upstream gradients with a batch stride of 0 (autograd's expansion of the
gradient of a sum) go to the kernels as one row read for every batch row
(row stride 0 through the ``*_ld`` entries) instead of a materialised copy.
Bar: bitwise equal to the same backward on the materialised gradient, on every
kernel route (generic, blocked, balanced, tiled, matrix representations,
split representation, layer GEMMs, rotor register / LDS chains and the n = 8
spin-matrix kernels), with batches that end inside a row group."""
import pytest
import torch

import cliffordcuda_amd as cc
from cliffordcuda_amd import _lib, bcast, products, rotor
from cliffordcuda_amd._validate import metric_masks

pytestmark = pytest.mark.gpu


def _rows(batch, n, seed, count):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(batch, 1 << n, generator=g).cuda() for _ in range(count)]


def _expanded(batch, n, seed):
    g = torch.Generator().manual_seed(seed + 1000)
    row = torch.randn(1 << n, generator=g).cuda()
    exp = row.expand(batch, 1 << n)
    assert batch == 1 or exp.stride(0) == 0
    return exp, exp.contiguous()


# (op, metric, CLF_* switches): each line lands on a different backward route
PRODUCT_CASES = [
    ("geom", (1, 1, 0), {}),                                      # generic, n < 4
    ("inner", (1, 1, 1, -1, 0), {}),                              # generic, mixed low metric
    ("lc", (1,) * 5, {"CLF_PRODUCT_PATH": "generic"}),
    ("geom", (1,) * 5, {"CLF_PRODUCT_PATH": "balanced"}),
    ("geom", (1,) * 5, {}),                                       # blocked
    ("wedge", (-1,) * 6, {}),                                     # balanced
    ("inner", (1,) * 6 + (-1,), {}),                              # blocked inner backward
    ("regressive", (1,) * 6 + (-1,), {"CLF_PRODUCT_PATH": "blocked"}),
    ("geom", (1,) * 6 + (-1,), {}),                               # n = 7 matrix representation
    ("geom", (1,) * 6 + (-1,), {"CLF_GEOM_PATH": "direct"}),
    ("geom", (1,) * 7 + (-1,), {}),                               # n = 8 matrix representation
    ("inner", (1,) * 8, {}),                                      # balanced inner (two deals)
    ("rc", (1,) * 8, {}),
    ("geom", (1,) * 9, {}),                                       # n = 9 split representation
    ("geom", (1,) * 9 + (0,), {}),                                # n = 10 fused split kernels
    ("geom", (1,) * 9 + (0,), {"CLF_SPLIT_PATH": "pairs"}),
    ("lc", (1,) * 9 + (0,), {}),
    ("inner", (1,) * 9 + (0,), {}),
    ("geom", (1,) * 12, {"CLF_PRODUCT_PATH": "blocked"}),         # blocked at n = 12
    ("geom", (1,) * 12, {}),                                      # small-batch split kernels
    ("regressive", (1,) * 11, {}),
    ("inner", (1,) * 9 + (0,), {"CLF_PRODUCT_PATH": "split"}),
    ("wedge", (1,) * 12, {"CLF_PRODUCT_PATH": "tiled"}),
]


def _ids(case):
    op, metric, env = case
    m = "".join({1: "+", -1: "-", 0: "0"}[x] for x in metric)
    return f"{op}-{m}" + ("-" + "-".join(env.values()) if env else "")


@pytest.mark.parametrize("case", PRODUCT_CASES, ids=_ids)
def test_product_bwd_stride0_equals_materialised(case, clf_env):
    op, metric, env = case
    n = len(metric)
    neg, nul = metric_masks(metric)
    for k, v in env.items():
        clf_env.setenv(k, v)
    batches = (1, 3, 5) if n >= 12 else (1, 3, 4 * 64 * max(1, 1 << max(0, 10 - n)) + 5)
    for batch in batches:
        print(f"[case] product stride0 op={op} metric={metric} env={env} batch={batch}", flush=True)
        a, b = _rows(batch, n, batch + n, 2)
        g0, gm = _expanded(batch, n, batch + n)
        for need in ((True, True), (True, False), (False, True)):
            ga0, gb0 = products._product_bwd(_lib.OP_CODES[op], n, neg, nul, a, b, g0, *need)
            gam, gbm = products._product_bwd(_lib.OP_CODES[op], n, neg, nul, a, b, gm, *need)
            for x0, xm in ((ga0, gam), (gb0, gbm)):
                assert (x0 is None) == (xm is None)
                if x0 is not None:
                    assert torch.equal(x0, xm)


def test_autograd_hands_over_stride0_rows(monkeypatch):
    """sum() and sum(0) backward reach the kernels with row stride 0 (the
    expansion is not materialised), with the gradients of the materialised
    upstream gradient. Spied on the Python autograd.Function's path (the C++
    node, csrc/torch_autograd.cpp, applies the same rule and is compared with
    this path bit for bit in test_autograd_ext_gpu.py)."""
    seen = []
    real = _lib.grad_rows

    def spy(g, dim):
        out = real(g, dim)
        seen.append(out[1])
        return out

    from cliffordcuda_amd import products
    monkeypatch.setattr(products, "_ext", None)
    monkeypatch.setattr(products, "_ext_tried", True)
    monkeypatch.setattr(_lib, "grad_rows", spy)
    metric = (1,) * 7 + (-1,)
    cl = cc.CliffordAlgebra(metric, device="cuda")
    a, b, t = _rows(1001, 8, 7, 3)
    for loss_kind in ("sum", "sum0"):
        seen.clear()
        ad, bd = a.clone().requires_grad_(), b.clone().requires_grad_()
        c = cl.geom_prod(ad, bd)
        loss = c.sum() if loss_kind == "sum" else (c.sum(0) * t[0]).sum()
        loss.backward()
        assert seen == [0], (loss_kind, seen)
        gm = torch.ones_like(c) if loss_kind == "sum" else t[0].expand_as(c).contiguous()
        ae, be = a.clone().requires_grad_(), b.clone().requires_grad_()
        cl.geom_prod(ae, be).backward(gm)
        assert torch.equal(ad.grad, ae.grad) and torch.equal(bd.grad, be.grad)


@pytest.mark.parametrize("metric", [(1,) * 7, (1,) * 7 + (-1,), (-1, 1) * 4 + (1,), (1,) * 9 + (0,)],
                         ids=lambda m: "".join({1: "+", -1: "-", 0: "0"}[x] for x in m))
@pytest.mark.parametrize("op", ["geom", "inner", "lc", "regressive"])
@pytest.mark.parametrize("side", [0, 1])
def test_layer_bwd_stride0_equals_materialised(op, metric, side):
    if op == "regressive" and 0 in metric:
        pytest.skip("regressive undefined for degenerate metrics")
    n = len(metric)
    neg, nul = metric_masks(metric)
    for batch in (1, 5, 3001):
        print(f"[case] layer stride0 op={op} metric={metric} side={side} batch={batch}", flush=True)
        (x,) = _rows(batch, n, batch, 1)
        (w,) = _rows(1, n, batch + 1, 1)
        g0, gm = _expanded(batch, n, batch)
        args = (_lib.OP_CODES[op], side, n, neg, nul)
        gx0, gw0 = bcast._bcast_bwd(x, w, g0, *args, True, True)
        gxm, gwm = bcast._bcast_bwd(x, w, gm, *args, True, True)
        assert torch.equal(gx0, gxm) and torch.equal(gw0, gwm)


@pytest.mark.parametrize("n,env", [(7, {}), (8, {}), (8, {"CLF_ROTOR_PATH": "chain"}), (10, {}), (12, {})],
                         ids=["n7", "n8-matrix", "n8-chain", "n10", "n12"])
def test_rotor_apply_bwd_stride0_equals_materialised(n, env, clf_env):
    for k, v in env.items():
        clf_env.setenv(k, v)
    g = torch.Generator().manual_seed(n)
    biv = (0.6 * torch.randn(1, n * (n - 1) // 2, generator=g)).cuda()
    state = rotor._compile_fwd(biv, n)
    for batch in (1, 27, 4097):
        print(f"[case] rotor stride0 n={n} env={env} batch={batch}", flush=True)
        (x,) = _rows(batch, n, batch, 1)
        g0, gm = _expanded(batch, n, batch)
        for need in ((True, True), (True, False), (False, True)):
            gs0, gx0 = rotor._apply_bwd(state, x, g0, n, *need)
            gsm, gxm = rotor._apply_bwd(state, x, gm, n, *need)
            for r0, rm in ((gs0, gsm), (gx0, gxm)):
                assert (r0 is None) == (rm is None)
                if r0 is not None:
                    assert torch.equal(r0, rm)


@pytest.mark.parametrize("n,env", [(7, {}), (8, {}), (8, {"CLF_ROTOR_PATH": "chain"}), (10, {}), (12, {})],
                         ids=["n7", "n8-matrix", "n8-chain", "n10", "n12"])
def test_bivector_apply_bwd_stride0_equals_materialised(n, env, clf_env):
    """The one-call bivector backward (apply backward, partial sum and compile
    backward) on an expanded gradient: bitwise the materialised gradient's
    results; an empty batch gives a zero bivector gradient."""
    for k, v in env.items():
        clf_env.setenv(k, v)
    g = torch.Generator().manual_seed(n + 20)
    biv = (0.6 * torch.randn(1, n * (n - 1) // 2, generator=g)).cuda()
    state = rotor._compile_fwd(biv, n)
    for batch in (1, 27, 4097):
        print(f"[case] bivector apply stride0 n={n} env={env} batch={batch}", flush=True)
        (x,) = _rows(batch, n, batch, 1)
        g0, gm = _expanded(batch, n, batch)
        for need in ((True, True), (True, False), (False, True)):
            gb0, gx0 = rotor._biv_apply_bwd(biv, state, x, g0, n, *need)
            gbm, gxm = rotor._biv_apply_bwd(biv, state, x, gm, n, *need)
            for r0, rm in ((gb0, gbm), (gx0, gxm)):
                assert (r0 is None) == (rm is None)
                if r0 is not None:
                    assert torch.equal(r0, rm)
    x = torch.empty(0, 1 << n, device="cuda")
    gb, _ = rotor._biv_apply_bwd(biv, state, x, torch.empty_like(x), n, True, False)
    torch.cuda.synchronize()
    assert torch.equal(gb, torch.zeros_like(biv))


@pytest.mark.parametrize("n", [7, 8, 12])
def test_rotor_cs_apply_bwd_stride0_equals_materialised(n):
    g = torch.Generator().manual_seed(n + 50)
    biv = (0.6 * torch.randn(1, n * (n - 1) // 2, generator=g)).cuda()
    _, cs = rotor._compile_fwd(biv, n, want_cs=True)
    for batch in (1, 27, 4097):
        print(f"[case] cs stride0 n={n} batch={batch}", flush=True)
        (x,) = _rows(batch, n, batch, 1)
        y = rotor._cs_apply_fwd(cs, x, n)
        g0, gm = _expanded(batch, n, batch)
        gc0, gx0 = rotor._cs_apply_bwd(cs, y, g0, n, True, True)
        gcm, gxm = rotor._cs_apply_bwd(cs, y, gm, n, True, True)
        assert torch.equal(gc0, gcm) and torch.equal(gx0, gxm)


def test_ld_entries_reject_other_strides():
    """Row strides other than 0 and 2^n are argument errors, returned before
    any launch."""
    lib = _lib.load()
    n = 7
    a = torch.zeros(4, 1 << n, device="cuda")
    out = torch.empty_like(a)
    s = _lib.stream_of(a)
    p, q = a.data_ptr(), out.data_ptr()
    for ldg in (1, 64, 256, -128):
        calls = (
            lambda: lib.clf_product_bwd_ld(0, n, 0, 0, p, p, p, ldg, q, None, 4, s),
            lambda: lib.clf_product_bcast_bwd_ld(0, 0, n, 0, 0, p, p, p, ldg, q, None, 4, None, 0, s),
            lambda: lib.clf_rotor_apply_bwd_ld(n, p, p, p, ldg, q, None, 4, None, 0, s),
            lambda: lib.clf_rotor_cs_apply_bwd_ld(n, p, p, p, ldg, q, None, 4, None, 0, s),
        )
        for call in calls:
            assert call() == _lib.CLF_ERR_ARG
            assert "row stride" in _lib.last_error()
    torch.cuda.synchronize()


@pytest.mark.parametrize("kind", ["reverse", "grade_involution", "clifford_conjugation", "grade_projection", "dual"])
def test_graded_bwd_stride0_equals_materialised(kind):
    """The graded ops' backward computes a batch-stride-0 upstream gradient's
    one row and hands it back expanded (no full-size write): bitwise equal to
    the backward of the materialised gradient, and still stride 0."""
    n = 10
    cl = cc.CliffordAlgebra((1,) * 9 + (0,) if kind != "dual" else (1,) * 8 + (-1, 1), device="cuda")
    (x,) = _rows(37, n, 71, 1)
    exp, mat = _expanded(37, n, 71)
    fn = {"grade_projection": lambda t: cl.grade_projection(t, 2)}.get(kind, getattr(cl, kind))
    outs = []
    for g in (exp, mat):
        xd = x.clone().requires_grad_()
        y = fn(xd)
        (gx,) = torch.autograd.grad(y, (xd,), g)
        outs.append(gx)
    assert torch.equal(outs[0], outs[1])


def test_graded_after_sum_keeps_stride0_into_the_product_backward():
    """C5's chain grade_projection(geom_prod(a, b), 2).sum().backward(): the
    projection's backward hands the product backward an expanded row, and the
    gradients equal those of the materialised upstream gradient."""
    n = 10
    cl = cc.CliffordAlgebra((1,) * 9 + (0,), device="cuda")
    a, b = _rows(29, n, 72, 2)
    res = []
    for mode in ("sum", "ones"):
        ad = a.clone().requires_grad_()
        bd = b.clone().requires_grad_()
        pr = cl.grade_projection(cl.geom_prod(ad, bd), 2)
        if mode == "sum":
            pr.sum().backward()
        else:
            pr.backward(torch.ones_like(pr))
        res.append((ad.grad, bd.grad))
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])


def test_inverse_bwd_accepts_stride0():
    """The inverse's backward (versor formula and the dense path's product
    backwards) takes the expanded gradient of a sum as it is."""
    n = 5
    cl = cc.CliffordAlgebra((1,) * 5, device="cuda")
    g = torch.Generator().manual_seed(73)
    v = torch.randn(19, n, generator=g)
    x = torch.zeros(19, 1 << n)
    for i in range(n):
        x[:, 1 << i] = v[:, i]                    # vectors: versors
    y = torch.randn(19, 1 << n, generator=g) + 3.0 * torch.nn.functional.one_hot(torch.zeros(19, dtype=torch.long), 1 << n)
    for xin, method in ((x, "versor"), (y, "lu")):
        grads = []
        for mode in ("sum", "ones"):
            xd = xin.cuda().requires_grad_()
            inv = cl.inverse(xd, method=method)
            if mode == "sum":
                inv.sum().backward()
            else:
                inv.backward(torch.ones_like(inv))
            grads.append(xd.grad)
        torch.testing.assert_close(grads[0], grads[1], rtol=1e-6, atol=1e-6)
