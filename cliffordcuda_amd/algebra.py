"""``CliffordAlgebra``: the reference's public class (``src/cliffordcuda/algebra.py:88-385``)
with the same constructor, attributes, methods, argument checks and error
messages, running on the gfx950 kernels of ``libclifford_hip.so``.

Differences from the reference, all supersets:
  * products accept any n >= 1 (the reference requires n >= 5);
  * ``apply_rotor`` / ``apply_bivector`` also return a gradient to ``x``
    (the reference's rotor backward returns ``None`` for x), and rotors are
    served for 7 <= n <= 12 (the reference's tables go to n = 12);
  * ``compile=`` on ``dual`` / ``norm_sq`` selects the same single-pass HIP
    kernel as the default (the reference uses torch.compile for it).
"""
from __future__ import annotations

import torch

from . import _validate, graded as _graded, products as _products, rotor as _rotor


class CliffordAlgebra:
    def __init__(self, metric, device="cuda"):
        metric = _validate.check_metric(metric)
        self.metric = metric
        self.n = len(metric)
        self.dim = 1 << self.n
        self.device = _validate.check_device(device)
        # fp32 only, as in the reference (``algebra.py:100-104``)
        self.dtype = torch.float32
        self._num_basis_biv = self.n * (self.n - 1) // 2
        self._neg, self._nul = _validate.metric_masks(metric)
        self._rotor_supported = self.n >= 7
        self._dev_index = self.device.index
        self._plans = {}

    # ── products (reference algebra.py:143-175) ─────────────────────────
    def _binary(self, op, a, b):
        # The usual call, tested in one expression: plain 2-D contiguous fp32
        # tensors of this algebra's row length and device, of one shape. It
        # then goes straight to the launch with the plan cached per op. Any
        # other call, and every call traced by torch.compile, takes the
        # argument checks in the reference's order (same exceptions and
        # messages) and the generic entry.
        plan = self._plans.get(op)
        if (plan is not None and not torch.compiler.is_compiling() and type(a) is torch.Tensor
                and type(b) is torch.Tensor and a.dim() == 2 and a.shape == b.shape and a.shape[1] == self.dim
                and a.dtype is torch.float32 and b.dtype is torch.float32 and a.is_cuda and b.is_cuda
                and a.get_device() == self._dev_index and b.get_device() == self._dev_index
                and a.is_contiguous() and b.is_contiguous()):
            return _products.run_rows(a, b, *plan)
        _validate.check_mv(a, "a", self.dim, self.device, self.dtype)
        _validate.check_mv(b, "b", self.dim, self.device, self.dtype)
        out = _products.product(op, a, b, self.metric)
        self._plans[op] = _products._plan(op, self.dim, self.metric)
        return out

    def geom_prod(self, a, b):
        return self._binary("geom", a, b)

    def wedge_prod(self, a, b):
        return self._binary("wedge", a, b)

    def inner_prod(self, a, b):
        return self._binary("inner", a, b)

    def left_contraction(self, a, b):
        return self._binary("lc", a, b)

    def right_contraction(self, a, b):
        return self._binary("rc", a, b)

    def regressive_prod(self, a, b):
        if 0 in self.metric:
            raise ValueError(
                "regressive_prod is undefined for degenerate metrics "
                "(any 0 in the metric makes the pseudoscalar non-invertible).")
        return self._binary("regressive", a, b)

    # ── inverse (reference algebra.py:178-192) ──────────────────────────
    def inverse(self, x, method="auto"):
        """Multivector inverse x^{-1}; see ``cliffordcuda_amd.inverse.inverse``."""
        _validate.check_mv(x, "x", self.dim, self.device, self.dtype)
        from .inverse import inverse as _inverse
        return _inverse(x, metric=self.metric, method=method)

    # ── graded ops (reference algebra.py:195-334) ───────────────────────
    def reverse(self, x):
        _validate.check_mv(x, "x", self.dim, self.device, self.dtype)
        return _graded.graded("reverse", x)

    def dual(self, x, compile=False):
        """x * I^{-1}: a signed reversal of the coefficients, one HIP pass.
        ``compile`` is accepted for compatibility; the kernel is already fused."""
        if 0 in self.metric:
            raise ValueError(
                "dual is undefined for degenerate metrics (any 0 in the "
                "metric makes the pseudoscalar I non-invertible).")
        _validate.check_mv(x, "x", self.dim, self.device, self.dtype)
        return _graded.graded("dual", x, self._neg, self._nul)

    def grade_involution(self, x):
        _validate.check_mv(x, "x", self.dim, self.device, self.dtype)
        return _graded.graded("involution", x)

    def clifford_conjugation(self, x):
        _validate.check_mv(x, "x", self.dim, self.device, self.dtype)
        return _graded.graded("conjugation", x)

    def grade_projection(self, x, grade):
        if not 0 <= grade <= self.n:
            raise ValueError(f"grade must be in [0, {self.n}] for n={self.n}; got {grade}")
        _validate.check_mv(x, "x", self.dim, self.device, self.dtype)
        return _graded.graded("projection", x, grade=int(grade))

    def norm_sq(self, x, compile=False):
        """<x x~>_0 = sum_b x_b^2 prod_{i in b} metric[i], shape (batch,), one HIP pass."""
        _validate.check_mv(x, "x", self.dim, self.device, self.dtype)
        return _graded.norm_sq(x, self._neg, self._nul)

    # ── rotor (reference algebra.py:337-373) ────────────────────────────
    def _check_rotor_supported(self):
        if not self._rotor_supported:
            raise ValueError(
                f"rotor application requires n >= 7 (ppr = 2^(n-2) must be "
                f"at least 32 = warp size); got n={self.n}")

    def compile_bivector(self, bivector):
        """Givens cs chain (C(n,2), 2) of the rotor of ``bivector`` (1, C(n,2))
        in lex-pair order; differentiable to the bivector. Returns a tensor
        that ``apply_rotor`` consumes."""
        self._check_rotor_supported()
        _validate.check_bivector(bivector, self.n, self._num_basis_biv, self.device, self.dtype)
        return _rotor.compile_bivector(bivector, self.n)

    def apply_rotor(self, cs, x):
        """Apply a cs chain (from ``compile_bivector``, or any (C(n,2), 2)
        tensor of (c, s) pairs) to a batch of multivectors; differentiable to
        cs and to x. The gradient to cs follows the reference's rule
        (``givens_apply_mb_perm_packed.cu:111-160``: each plane's input rebuilt
        from the output with the transposed pair map), which is the true
        derivative for unit (c, s) pairs only; the gradient to x is exact."""
        self._check_rotor_supported()
        _validate.check_mv(x, "x", self.dim, self.device, self.dtype)
        return _rotor.apply_rotor(cs, x, self.n)

    def apply_bivector(self, bivector, x):
        """``apply_rotor(compile_bivector(bivector), x)`` in one pass, without
        materialising cs; differentiable to the bivector and to x."""
        self._check_rotor_supported()
        _validate.check_bivector(bivector, self.n, self._num_basis_biv, self.device, self.dtype)
        _validate.check_mv(x, "x", self.dim, self.device, self.dtype)
        return _rotor.apply_bivector(bivector, x, self.n)

    # ── misc ───────────────────────────────────────────────────────────
    def to(self, device):
        return CliffordAlgebra(self.metric, device=device)

    def __repr__(self):
        p = sum(1 for m in self.metric if m == 1)
        q = sum(1 for m in self.metric if m == -1)
        r = sum(1 for m in self.metric if m == 0)
        return (f"CliffordAlgebra(metric={list(self.metric)}, "
                f"Cl({p}, {q}, {r}), n={self.n}, dim={self.dim}, "
                f"device={self.device})")
