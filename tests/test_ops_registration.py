"""The native entry points are registered as torch.library operators with
shape-only fake implementations (what torch.compile traces), checked on the
CPU with fake tensors: no kernel runs."""
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import cliffordcuda_amd  # noqa: F401  (registers the operators)

OPS = ["product", "product_bwd", "graded", "norm_sq", "norm_sq_bwd", "bcast_product", "bcast_product_bwd",
       "rotor_compile", "rotor_compile_bwd", "rotor_apply", "rotor_apply_bwd"]


def test_operators_registered():
    for name in OPS:
        assert hasattr(torch.ops.cliffordcuda_amd, name), name


def test_fake_shapes():
    ops = torch.ops.cliffordcuda_amd
    with FakeTensorMode():
        a = torch.empty(5, 256)
        w = torch.empty(1, 256)
        biv = torch.empty(28)
        assert ops.product(a, a, 0, 8, 0, 0).shape == (5, 256)
        ga, gb = ops.product_bwd(a, a, a, 0, 8, 0, 0, True, False)
        assert ga.shape == (5, 256) and gb.numel() == 0
        assert ops.graded(a, 0, 8, 0, 0, 0).shape == (5, 256)
        assert ops.norm_sq(a, 8, 0, 0).shape == (5,)
        assert ops.bcast_product(a, w, 0, 0, 8, 0, 0).shape == (5, 256)
        gx, gw = ops.bcast_product_bwd(a, w, a, 0, 0, 8, 0, 0, True, True)
        assert gx.shape == (5, 256) and gw.shape == (1, 256)
        state = ops.rotor_compile(biv, 8)
        assert state.shape == (8 * 8 + 8 * 7 + 256,)
        assert ops.rotor_apply(state, a, 8).shape == (5, 256)
