"""Broadcast-weight products ``op(x, w)`` with one weight multivector w of shape
(1, 2^n) shared by the batch: the computation of the product layers
(reference ``src/cliffordcuda/layers.py:30-50``).

For n in [7, 10] this runs as fp32 MFMA GEMMs against the signed 2^n x 2^n
matrix of w (``clf_product_bcast_fwd`` / ``_bwd``): the weight is never
expanded to (batch, 2^n) and its gradient is reduced on the device. Smaller
algebras use the per-row product kernels on the expanded weight, as the
reference does.
"""
from __future__ import annotations

import torch

from . import _lib, _ops
from . import products as _products
from ._validate import check_mv


def _ws(lib, n, batch, device):
    nbytes = lib.clf_product_bcast_ws_bytes(n, batch)
    return torch.empty(max(4, nbytes) // 4, dtype=torch.float32, device=device), nbytes


def _bcast_fwd(x, w, op_code, side, n, neg, nul):
    lib = _lib.load()
    y = torch.empty_like(x)
    ws, nbytes = _ws(lib, n, x.shape[0], x.device)
    with _lib.on_device(x):
        rc = lib.clf_product_bcast_fwd(op_code, side, n, neg, nul, x.data_ptr(), w.data_ptr(), y.data_ptr(),
                                       x.shape[0], ws.data_ptr(), nbytes, _lib.stream_of(x))
    _lib.check(rc, "clf_product_bcast_fwd")
    return y


def _bcast_bwd(x, w, gy, op_code, side, n, neg, nul, need_x, need_w):
    if not (need_x or need_w):
        return None, None
    lib = _lib.load()
    gy, ldg = _lib.grad_rows(gy, x.shape[1])
    gx = torch.empty_like(x) if need_x else None
    gw = torch.empty_like(w) if need_w else None
    ws, nbytes = _ws(lib, n, x.shape[0], x.device)
    with _lib.on_device(x):
        rc = lib.clf_product_bcast_bwd_ld(op_code, side, n, neg, nul, x.data_ptr(), w.data_ptr(), gy.data_ptr(),
                                          ldg, _lib.ptr(gx), _lib.ptr(gw), x.shape[0], ws.data_ptr(), nbytes,
                                          _lib.stream_of(x))
    _lib.check(rc, "clf_product_bcast_bwd_ld")
    return gx, gw


class _BcastFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, op_code, side, n, neg, nul):
        ctx.save_for_backward(x, w)
        ctx.meta = (op_code, side, n, neg, nul)
        return _bcast_fwd(x, w, op_code, side, n, neg, nul)

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        gx, gw = _bcast_bwd(x, w, gy, *ctx.meta, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return gx, gw, None, None, None, None, None


def bcast_product(op: str, x: torch.Tensor, w: torch.Tensor, metric: tuple, side: int = 0) -> torch.Tensor:
    """op(x, w) (side 0) or op(w, x) (side 1) for x (batch, 2^n), w (1, 2^n)."""
    from ._validate import metric_masks
    n = len(metric)
    if op == "regressive" and 0 in metric:
        raise ValueError(
            "regressive_prod is undefined for degenerate metrics "
            "(any 0 in the metric makes the pseudoscalar non-invertible).")
    if not (7 <= n <= 10):
        wb = w.expand_as(x).contiguous()
        return _products.product(op, x, wb, metric) if side == 0 else _products.product(op, wb, x, metric)
    neg, nul = metric_masks(metric)
    args = (x.contiguous(), w.contiguous().reshape(1, -1), _lib.OP_CODES[op], side, n, neg, nul)
    if torch.compiler.is_compiling():
        return _ops.bcast_product(*args)
    return _BcastFunc.apply(*args)


def product_bcast(op: str, x: torch.Tensor, w: torch.Tensor, cl) -> torch.Tensor:
    """The layer computation: op(x, weight) with x validated like the algebra's methods."""
    check_mv(x, "x", cl.dim, cl.device, cl.dtype)
    return bcast_product(op, x, w, cl.metric, side=0)
