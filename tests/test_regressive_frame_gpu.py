"""The regressive product's backward on the wedge frame schedule
(prod_bwd_contr_frame<OP_REGR, n>, 4 <= n <= 8): the wedge backward on the
duals (D a, D b, D^T gc) with (D x)[k] = t(~k) x[~k], followed by D^T on
both gradients, folded into the kernel's row fetch and row-order stores.
Parity with the fp64 oracle (the reference's definition dual(dual(a) ^
dual(b))) on mixed signatures and ragged batches, with the balanced kernels
(CLF_PRODUCT_PATH=balanced) at a larger batch, and for a batch-stride-0
upstream gradient. Bar: normwise relative error <= 1e-5."""
import pytest
import torch

from cliffordcuda_amd import _lib, products
from cliffordcuda_amd._validate import metric_masks
from oracle import clifford_oracle as O

pytestmark = pytest.mark.gpu
TOL = 1e-5

METRICS = [(1,) * 4, (-1, 1, -1, 1, 1), (1,) * 5 + (-1,), (1,) * 6 + (-1,), (1, -1, 1, -1, -1, 1, 1),
           (-1,) * 7, (1,) * 8, (1, 1, -1, 1, -1, 1, 1, -1)]


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = float(ref.abs().max())
    return float((got - ref).abs().max()) / (den if den > 0 else 1.0)


def _ids(m):
    return "".join({1: "+", -1: "-"}[x] for x in m)


@pytest.mark.parametrize("metric", METRICS, ids=_ids)
def test_regressive_backward_matches_oracle(metric):
    n = len(metric)
    batch = 333
    g = torch.Generator().manual_seed(90 + n)
    a, b, gc = (torch.randn(batch, 1 << n, generator=g) for _ in range(3))
    print(f"[case] regressive frame backward {metric} batch={batch}", flush=True)
    x = a.cuda().requires_grad_()
    y = b.cuda().requires_grad_()
    products.product("regressive", x, y, metric).backward(gc.cuda())
    a64 = a.double().requires_grad_()
    b64 = b.double().requires_grad_()
    O.einsum_product("regressive", a64, b64, metric).backward(gc.double())
    assert rel_err(x.grad, a64.grad) <= TOL
    assert rel_err(y.grad, b64.grad) <= TOL


@pytest.mark.parametrize("metric", METRICS[2::2], ids=_ids)
def test_regressive_backward_equals_balanced(metric, clf_env):
    n = len(metric)
    batch = 65537 if n == 7 else 20001
    g = torch.Generator().manual_seed(95 + n)
    a, b, gc = (torch.randn(batch, 1 << n, generator=g).cuda() for _ in range(3))
    print(f"[case] regressive frame vs balanced {metric} batch={batch}", flush=True)
    neg, nul = metric_masks(metric)
    code = _lib.OP_CODES["regressive"]
    res = []
    for path in (None, "balanced"):
        if path:
            clf_env.setenv("CLF_PRODUCT_PATH", path)
        res.append(products._product_bwd(code, n, neg, nul, a, b, gc, True, True))
        if path:
            clf_env.delenv("CLF_PRODUCT_PATH")
    assert rel_err(res[0][0], res[1][0]) <= TOL
    assert rel_err(res[0][1], res[1][1]) <= TOL


def test_regressive_backward_stride0():
    metric = (1,) * 6 + (-1,)
    n, batch = 7, 1001
    neg, nul = metric_masks(metric)
    g = torch.Generator().manual_seed(99)
    a, b = (torch.randn(batch, 1 << n, generator=g).cuda() for _ in range(2))
    row = torch.randn(1 << n, generator=g).cuda()
    code = _lib.OP_CODES["regressive"]
    ga0, gb0 = products._product_bwd(code, n, neg, nul, a, b, row.expand(batch, 1 << n), True, True)
    gam, gbm = products._product_bwd(code, n, neg, nul, a, b, row.expand(batch, 1 << n).contiguous(), True, True)
    assert torch.equal(ga0, gam) and torch.equal(gb0, gbm)
