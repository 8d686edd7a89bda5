"""prod_fwd_contr5 / prod_bwd_contr5 (the contractions on 5 high bits: lc and
rc at n = 9, lc at n = 10 whose only null generator is e9, C5's Cl(9,0,1)) and
prod_bwd_inner5 (the inner product's backward on the same schedules, n = 9
and the null-top n = 10): parity with the fp64 oracle, with the balanced
kernels they replace (CLF_PRODUCT_PATH=balanced), on ragged batches (two rows
per wave at n = 9), with a batch-stride-0 upstream gradient, and bitwise row
independence. Bar: normwise relative error <= 1e-5 for the product and both
gradients."""
import pytest
import torch

import cliffordcuda_amd as cc
from cliffordcuda_amd import _lib, products
from cliffordcuda_amd._validate import metric_masks
from oracle import clifford_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-5


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = float(ref.abs().max())
    return float((got - ref).abs().max()) / (den if den > 0 else 1.0)


def inputs(n, batch, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(batch, 1 << n, generator=g) for _ in range(3)]


CASES = [("lc", (1,) * 9), ("rc", (1,) * 9), ("lc", (-1,) * 4 + (1, -1, 1, 1, -1)), ("rc", (1,) * 4 + (-1,) * 5),
         ("lc", (1,) * 9 + (0,)), ("lc", (-1,) * 4 + (1, -1, 1, 1, -1, 0)),
         ("inner", (1,) * 9), ("inner", (-1,) * 4 + (1, -1, 1, 1, -1)), ("inner", (1,) * 9 + (0,)),
         ("inner", (-1,) * 4 + (1, 1, -1, 1, -1, 0))]


def _ids(c):
    return c[0] + "-" + "".join({1: "+", -1: "-", 0: "0"}[x] for x in c[1])


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_contr5_matches_oracle(case):
    op, metric = case
    n = len(metric)
    # large enough to leave the small-batch kernels (batch * 2^(n-4) >= 2^15 at n = 10)
    batch = 1029 if n == 9 else 517
    a, b, gc = inputs(n, batch, 50 + n)
    rows = torch.tensor([0, 1, 2, 511, batch - 2, batch - 1])
    print(f"[case] contr5 {op} {metric} batch={batch}", flush=True)
    x = a.cuda().requires_grad_()
    y = b.cuda().requires_grad_()
    c = products.product(op, x, y, metric)
    c.backward(gc.cuda())
    a64 = a[rows].double().requires_grad_()
    b64 = b[rows].double().requires_grad_()
    O.einsum_product(op, a64, b64, metric).backward(gc[rows].double())
    rs = rows.cuda()
    with torch.no_grad():
        c64 = O.einsum_product(op, a[rows].double(), b[rows].double(), metric)
    assert rel_err(c[rs], c64) <= TOL
    assert rel_err(x.grad[rs], a64.grad) <= TOL
    assert rel_err(y.grad[rs], b64.grad) <= TOL


@pytest.mark.parametrize("case", CASES, ids=_ids)
def test_contr5_equals_balanced_kernels(case, clf_env):
    """The whole batch against the balanced kernels (which the oracle tests pin
    on their own), odd batch sizes included."""
    op, metric = case
    n = len(metric)
    for batch in ((1029, 4001) if n == 9 else (517, 2049)):
        a, b, gc = [t.cuda() for t in inputs(n, batch, 60 + batch)]
        print(f"[case] contr5 vs balanced {op} {metric} batch={batch}", flush=True)
        res = []
        for path in (None, "balanced"):
            if path:
                clf_env.setenv("CLF_PRODUCT_PATH", path)
            x = a.clone().requires_grad_()
            y = b.clone().requires_grad_()
            c = products.product(op, x, y, metric)
            c.backward(gc)
            res.append((x.grad, y.grad, c.detach()))
            if path:
                clf_env.delenv("CLF_PRODUCT_PATH")
        assert rel_err(res[0][0], res[1][0]) <= TOL
        assert rel_err(res[0][1], res[1][1]) <= TOL
        assert rel_err(res[0][2], res[1][2]) <= TOL


@pytest.mark.parametrize("case", CASES[::3], ids=_ids)
def test_contr5_stride0_and_one_gradient(case):
    """A batch-stride-0 upstream gradient gives, bit for bit, the gradients of
    its materialised copy; asking for one gradient gives the same values."""
    op, metric = case
    n = len(metric)
    neg, nul = metric_masks(metric)
    batch = 1029 if n == 9 else 517
    a, b, _ = [t.cuda() for t in inputs(n, batch, 70)]
    row = torch.randn(1 << n, generator=torch.Generator().manual_seed(71)).cuda()
    g0 = row.expand(batch, 1 << n)
    gm = g0.contiguous()
    code = _lib.OP_CODES[op]
    ga0, gb0 = products._product_bwd(code, n, neg, nul, a, b, g0, True, True)
    gam, gbm = products._product_bwd(code, n, neg, nul, a, b, gm, True, True)
    assert torch.equal(ga0, gam) and torch.equal(gb0, gbm)
    ga1, _ = products._product_bwd(code, n, neg, nul, a, b, gm, True, False)
    _, gb1 = products._product_bwd(code, n, neg, nul, a, b, gm, False, True)
    assert torch.equal(ga1, gam) and torch.equal(gb1, gbm)


@pytest.mark.parametrize("op", ["lc", "inner"])
def test_contr5_rows_are_independent(op):
    """C5's shape: rows computed in the full batch of 16384 equal, bit for bit,
    the same rows inside a batch of 1025 (both on prod_bwd_contr5 or
    prod_bwd_inner5)."""
    metric = (1,) * 9 + (0,)
    B = 16384
    a, b, gc = [t.cuda() for t in inputs(10, B, 80)]
    code = _lib.OP_CODES[op]
    neg, nul = metric_masks(metric)
    ga, gb = products._product_bwd(code, 10, neg, nul, a, b, gc, True, True)
    idx = torch.cat([torch.arange(0, 512), torch.arange(B - 513, B)]).cuda()
    ga_s, gb_s = products._product_bwd(code, 10, neg, nul, a[idx].contiguous(), b[idx].contiguous(),
                                       gc[idx].contiguous(), True, True)
    assert torch.equal(ga[idx], ga_s) and torch.equal(gb[idx], gb_s)
    c = products._product_fwd(code, 10, neg, nul, a, b)
    c_s = products._product_fwd(code, 10, neg, nul, a[idx].contiguous(), b[idx].contiguous())
    assert torch.equal(c[idx], c_s)
