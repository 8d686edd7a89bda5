"""Single-pass graded ops (reverse, grade involution, Clifford conjugation,
grade projection, dual) and norm_sq, differentiable, on the gfx950 kernels.

Semantics follow ``src/cliffordcuda/algebra.py:195-334``. Each op is one
streaming kernel launch (``clf_graded`` / ``clf_norm_sq_fwd``); the reference
runs them as 1-3 eager torch passes.
"""
from __future__ import annotations

import torch

from . import _lib, _ops
from ._validate import dim_to_n


def _graded_launch(kind: int, n: int, neg: int, nul: int, grade: int, x: torch.Tensor) -> torch.Tensor:
    y = torch.empty_like(x)
    lib = _lib.load()
    with _lib.on_device(x):
        rc = lib.clf_graded(kind, n, neg, nul, grade, x.data_ptr(), y.data_ptr(), x.shape[0],
                            _lib.stream_of(x))
    _lib.check(rc, "clf_graded")
    return y


def graded_adjoint(kind: int, n: int, neg: int, nul: int, grade: int, gy: torch.Tensor, launch) -> torch.Tensor:
    """The backward of a graded op: its adjoint (the op itself for the sign and
    mask ops, DUAL_ADJ for the dual) applied to the upstream gradient. The op is
    row by row, so an upstream gradient whose batch stride is 0 (autograd's
    expansion of the gradient of a sum) gives a result with the same one row:
    it is computed on that row and handed back expanded, with no full-size
    read or write."""
    adj = _lib.GRADED_CODES["dual_adj"] if kind == _lib.GRADED_CODES["dual"] else kind
    if gy.dim() == 2 and gy.shape[0] > 1 and gy.stride(0) == 0:
        return launch(adj, n, neg, nul, grade, gy[:1].contiguous()).expand(gy.shape)
    return launch(adj, n, neg, nul, grade, gy.contiguous())


class _GradedFunc(torch.autograd.Function):
    """y = kind(x); sign / mask ops are self-adjoint, the dual's adjoint is
    the DUAL_ADJ kernel."""

    @staticmethod
    def forward(ctx, x, kind, n, neg, nul, grade):
        ctx.meta = (kind, n, neg, nul, grade)
        return _graded_launch(kind, n, neg, nul, grade, x)

    @staticmethod
    def backward(ctx, gy):
        kind, n, neg, nul, grade = ctx.meta
        return graded_adjoint(kind, n, neg, nul, grade, gy, _graded_launch), None, None, None, None, None


def graded(kind: str, x: torch.Tensor, neg: int = 0, nul: int = 0, grade: int = 0) -> torch.Tensor:
    if not x.is_cuda or x.dtype != torch.float32:
        raise RuntimeError(f"{kind}: x must be a float32 GPU tensor")
    dim = x.shape[-1]
    n = dim_to_n(dim)
    shape = x.shape
    x2 = x.contiguous().reshape(-1, dim)
    code = _lib.GRADED_CODES[kind]
    if torch.compiler.is_compiling():
        return _ops.graded(x2, code, n, neg, nul, grade).reshape(shape)
    return _GradedFunc.apply(x2, code, n, neg, nul, grade).reshape(shape)


def _norm_sq_fwd(x: torch.Tensor, n: int, neg: int, nul: int) -> torch.Tensor:
    out = torch.empty(x.shape[0], dtype=x.dtype, device=x.device)
    lib = _lib.load()
    with _lib.on_device(x):
        rc = lib.clf_norm_sq_fwd(n, neg, nul, x.data_ptr(), out.data_ptr(), x.shape[0], _lib.stream_of(x))
    _lib.check(rc, "clf_norm_sq_fwd")
    return out


def _norm_sq_bwd(x: torch.Tensor, gout: torch.Tensor, n: int, neg: int, nul: int) -> torch.Tensor:
    gx = torch.empty_like(x)
    gout = gout.contiguous()
    lib = _lib.load()
    with _lib.on_device(x):
        rc = lib.clf_norm_sq_bwd(n, neg, nul, x.data_ptr(), gout.data_ptr(), gx.data_ptr(), x.shape[0],
                                 _lib.stream_of(x))
    _lib.check(rc, "clf_norm_sq_bwd")
    return gx


class _NormSqFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, n, neg, nul):
        ctx.save_for_backward(x)
        ctx.meta = (n, neg, nul)
        return _norm_sq_fwd(x, n, neg, nul)

    @staticmethod
    def backward(ctx, gout):
        (x,) = ctx.saved_tensors
        n, neg, nul = ctx.meta
        return _norm_sq_bwd(x, gout, n, neg, nul), None, None, None


def norm_sq(x: torch.Tensor, neg: int = 0, nul: int = 0) -> torch.Tensor:
    if not x.is_cuda or x.dtype != torch.float32:
        raise RuntimeError("norm_sq: x must be a float32 GPU tensor")
    dim = x.shape[-1]
    n = dim_to_n(dim)
    lead = x.shape[:-1]
    x2 = x.contiguous().reshape(-1, dim)
    if torch.compiler.is_compiling():
        out = _ops.norm_sq(x2, n, neg, nul)
    else:
        out = _NormSqFunc.apply(x2, n, neg, nul)
    return out.reshape(lead)


def reverse(x: torch.Tensor) -> torch.Tensor:
    """Reversion x~ (reference free function ``extensions/ga/inverse.py:64-67``)."""
    return graded("reverse", x)
