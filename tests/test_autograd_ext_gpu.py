"""The products' C++ autograd node (cliffordcuda_amd/_clf_autograd.so, from
csrc/torch_autograd.cpp) against the Python autograd.Function it stands in for:
both call the same library entries, so values and gradients agree bit for
bit, with both gradients, with one, with a batch-stride-0 upstream gradient,
under no_grad (the forward without a node), and errors keep their types."""
import pytest
import torch

from cliffordcuda_amd import _lib, products
from cliffordcuda_amd._validate import metric_masks

pytestmark = pytest.mark.gpu


def _ext():
    ext = products._autograd_ext()
    if ext is None:
        pytest.fail("the C++ autograd node is not built (run __graft_entry__.build())")
    return ext


@pytest.mark.parametrize("op", ["geom", "wedge", "inner", "lc", "rc", "regressive"])
@pytest.mark.parametrize("metric", [(1,) * 7, (1,) * 6 + (-1,), (1,) * 9 + (0,)], ids=["7+", "7-", "10null"])
def test_cpp_node_equals_python_function(op, metric):
    if op == "regressive" and 0 in metric:
        pytest.skip("regressive undefined for degenerate metrics")
    ext = _ext()
    n = len(metric)
    neg, nul = metric_masks(metric)
    code = _lib.OP_CODES[op]
    g = torch.Generator().manual_seed(7)
    a, b, gc = (torch.randn(37, 1 << n, generator=g).cuda() for _ in range(3))
    print(f"[case] cpp node op={op} metric={metric}", flush=True)
    for need in ((True, True), (True, False), (False, True)):
        x1, y1 = a.clone().requires_grad_(need[0]), b.clone().requires_grad_(need[1])
        x2, y2 = a.clone().requires_grad_(need[0]), b.clone().requires_grad_(need[1])
        c1 = ext.product(x1, y1, code, n, neg, nul)
        c2 = products._ProductFunc.apply(x2, y2, code, n, neg, nul)
        assert torch.equal(c1, c2)
        c1.backward(gc)
        c2.backward(gc)
        for u, v in ((x1.grad, x2.grad), (y1.grad, y2.grad)):
            assert (u is None) == (v is None)
            if u is not None:
                assert torch.equal(u, v)
    with torch.no_grad():
        assert torch.equal(ext.product_fwd(a, b, code, n, neg, nul), products._product_fwd(code, n, neg, nul, a, b))


def test_cpp_node_stride0_gradient():
    ext = _ext()
    metric = (1,) * 7
    neg, nul = metric_masks(metric)
    g = torch.Generator().manual_seed(8)
    a, b = (torch.randn(53, 128, generator=g).cuda().requires_grad_() for _ in range(2))
    c = ext.product(a, b, 0, 7, neg, nul)
    c.sum().backward()  # autograd hands the gradient over as a stride-0 expansion
    a2, b2 = a.detach().clone().requires_grad_(), b.detach().clone().requires_grad_()
    products._ProductFunc.apply(a2, b2, 0, 7, neg, nul).backward(torch.ones(53, 128, device="cuda"))
    assert torch.equal(a.grad, a2.grad) and torch.equal(b.grad, b2.grad)


def test_cpp_node_error_types():
    ext = _ext()
    a = torch.randn(4, 128, device="cuda")
    with pytest.raises(ValueError):  # an unknown op code: CLF_ERR_ARG
        ext.product_fwd(a, a, 17, 7, 0, 0)


def test_product_uses_the_cpp_node():
    _ext()
    a, b = (torch.randn(8, 128, device="cuda").requires_grad_() for _ in range(2))
    c = products.product("geom", a, b)
    assert type(c.grad_fn).__name__ != "_ProductFuncBackward"  # not the Python Function's node
