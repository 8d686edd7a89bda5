"""``nn.Module`` layers of the reference (``src/cliffordcuda/layers.py:30-108``).

Product layers hold a learnable ``weight`` of shape (1, 2^n) and compute
``product(x, weight)`` (x on the left). The weight is broadcast over the batch
without being materialised: the broadcast path treats ``x -> op(x, w)`` as one
linear map, so the weight is read once per launch and its gradient is
reduced on the device (``cliffordcuda_amd.bcast``).

``RotorLayer`` holds a learnable ``bivector`` of shape (1, C(n,2)) and applies
the sandwich ~R x R, recompiling the rotor on every forward in train mode and
caching it in eval mode. The eval cache is also keyed on the parameter's
version counter, so in-place edits and ``load_state_dict`` invalidate it.
"""
import torch
import torch.nn as nn

from . import bcast as _bcast


class _ProductLayer(nn.Module):
    _op: str = None
    _method: str = None

    def __init__(self, cl):
        super().__init__()
        self.cl = cl
        self.weight = nn.Parameter(torch.randn(1, cl.dim, device=cl.device, dtype=cl.dtype))

    def forward(self, x):
        return _bcast.product_bcast(self._op, x, self.weight, self.cl)

    def extra_repr(self):
        return f"n={self.cl.n}, dim={self.cl.dim}, op={self._method}"


class GeometricProductLayer(_ProductLayer):
    _op, _method = "geom", "geom_prod"


class WedgeProductLayer(_ProductLayer):
    _op, _method = "wedge", "wedge_prod"


class InnerProductLayer(_ProductLayer):
    _op, _method = "inner", "inner_prod"


class LeftContractionLayer(_ProductLayer):
    _op, _method = "lc", "left_contraction"


class RightContractionLayer(_ProductLayer):
    _op, _method = "rc", "right_contraction"


class RegressiveProductLayer(_ProductLayer):
    # non-degenerate signatures only; raises on r > 0 like CliffordAlgebra.regressive_prod
    _op, _method = "regressive", "regressive_prod"


class RotorLayer(nn.Module):
    """Learnable rotor ~R x R from a (1, C(n,2)) bivector; requires n >= 7."""

    def __init__(self, cl):
        super().__init__()
        if cl.n < 7:
            raise ValueError(f"RotorLayer requires n>=7 (rotor support); got n={cl.n}")
        self.cl = cl
        num_basis_biv = cl.n * (cl.n - 1) // 2
        self.bivector = nn.Parameter(torch.randn(1, num_basis_biv, device=cl.device, dtype=cl.dtype))
        self._cs = None
        self._cs_key = None

    def train(self, mode=True):
        self._cs = None
        return super().train(mode)

    def forward(self, x):
        if self.training:
            return self.cl.apply_bivector(self.bivector, x)
        key = (self.bivector.data_ptr(), self.bivector._version)
        if self._cs is None or self._cs_key != key:
            with torch.no_grad():
                self._cs = self.cl.compile_bivector(self.bivector)
            self._cs_key = key
        return self.cl.apply_rotor(self._cs, x)

    def extra_repr(self):
        return f"n={self.cl.n}, dim={self.cl.dim}, num_basis_biv={self.bivector.shape[-1]}"
