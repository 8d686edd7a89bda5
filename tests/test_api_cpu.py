"""Host-side API behaviour that needs no GPU: argument checks with the
reference's exception types and messages (src/cliffordcuda/_validate.py)."""
import pytest
import torch

import cliffordcuda_amd as cc
from cliffordcuda_amd import _validate


def test_public_names_match_reference():
    ref_all = {
        "CliffordAlgebra", "geom_prod", "geom_prod_multik", "wedge_prod", "wedge_prod_multik", "wedge_prod_skip",
        "wedge_prod_multik_skip", "wedge_prod_subset_grade", "inner_prod", "inner_prod_kskip", "inner_prod_multik",
        "inner_prod_multik_skip", "inner_prod_skip", "inner_prod_subset_grade", "left_contract",
        "left_contract_skip", "left_contract_subset_grade", "right_contract", "right_contract_skip",
        "right_contract_subset_grade", "regressive_prod", "regressive_prod_skip", "regressive_prod_subset_grade",
        "inverse", "reverse", "GeometricProductLayer", "WedgeProductLayer", "InnerProductLayer",
        "LeftContractionLayer", "RightContractionLayer", "RegressiveProductLayer", "RotorLayer",
    }
    assert ref_all <= set(cc.__all__)
    for name in ref_all:
        assert hasattr(cc, name)


def test_metric_validation():
    with pytest.raises(ValueError, match="iterable"):
        _validate.check_metric(3)
    with pytest.raises(ValueError, match="each be in"):
        _validate.check_metric([1, 2])
    with pytest.raises(ValueError, match="at least one"):
        _validate.check_metric([])
    assert _validate.check_metric([1, -1, 0]) == (1, -1, 0)


def test_device_validation_cpu():
    with pytest.raises(ValueError, match="CUDA-only"):
        cc.CliffordAlgebra([1, 1, 1], device="cpu")
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="is_available"):
            cc.CliffordAlgebra([1, 1, 1], device="cuda")


def test_mv_and_bivector_checks():
    dev = torch.device("cpu")
    x = torch.zeros(2, 8)
    _validate.check_mv(x, "x", 8, dev, torch.float32)
    with pytest.raises(ValueError, match="must be a torch.Tensor"):
        _validate.check_mv([1], "x", 8, dev, torch.float32)
    with pytest.raises(ValueError, match="last dim 8 != 2\\^n = 16"):
        _validate.check_mv(x, "x", 16, dev, torch.float32)
    with pytest.raises(ValueError, match="C\\(n, 2\\) = 28"):
        _validate.check_bivector(torch.zeros(1, 27), 8, 28, dev, torch.float32)
    with pytest.raises(ValueError, match="first dim must be 1"):
        _validate.check_bivector(torch.zeros(2, 28), 8, 28, dev, torch.float32)


def test_masks():
    assert _validate.metric_masks((1, -1, 0, -1)) == (0b1010, 0b0100)
    assert _validate.dim_to_n(256) == 8
    with pytest.raises(ValueError):
        _validate.dim_to_n(48)


def test_free_functions_reject_cpu_tensors():
    with pytest.raises(RuntimeError, match="GPU"):
        cc.geom_prod(torch.zeros(2, 32), torch.zeros(2, 32))


def test_bench_refuses_several_gpus():
    """bench.py measures one GPU; --gpus above 1 exits with a message before
    touching any device."""
    import json
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    msg = json.loads(res.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_grad_rows_hands_over_stride0_gradients_as_one_row():
    """The backward entries take the upstream gradient's row stride: a batch
    stride of 0 (autograd's expansion of the gradient of a sum) goes over as
    its one row with stride 0, anything else as a contiguous tensor with
    stride 2^n."""
    from cliffordcuda_amd import _lib
    D = 32
    row = torch.arange(D, dtype=torch.float32)
    g, ld = _lib.grad_rows(row.expand(7, D), D)          # expanded row: (0, 1) strides
    assert ld == 0 and g.shape == (D,) and g.is_contiguous() and torch.equal(g, row)
    g, ld = _lib.grad_rows(torch.ones(()).expand(5, D), D)  # expanded scalar: (0, 0) strides
    assert ld == 0 and g.shape == (D,) and g.is_contiguous() and torch.equal(g, torch.ones(D))
    full = torch.randn(6, D)
    g, ld = _lib.grad_rows(full, D)                        # packed rows go as they are
    assert ld == D and g.data_ptr() == full.data_ptr()
    t = torch.randn(D, 6).t()                              # other layouts are made contiguous
    g, ld = _lib.grad_rows(t, D)
    assert ld == D and g.is_contiguous() and torch.equal(g, t)
    g, ld = _lib.grad_rows(row.expand(1, D), D)            # one row: nothing to save
    assert ld == D and g.shape == (1, D)
    odd = torch.randn(2 * D + 1)[1:D + 1]                  # a row 4 bytes off 16-byte alignment
    g, ld = _lib.grad_rows(odd.expand(3, D), D)
    assert ld == 0 and g.data_ptr() % 16 == 0 and torch.equal(g, odd)
