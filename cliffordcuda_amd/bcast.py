"""Broadcast-weight products ``op(x, w)`` with w of shape (1, 2^n) (the product layers)."""
from __future__ import annotations

import torch

from . import products as _products


def product_bcast(op: str, x: torch.Tensor, w: torch.Tensor, cl) -> torch.Tensor:
    from ._validate import check_mv
    check_mv(x, "x", cl.dim, cl.device, cl.dtype)
    if op == "regressive" and 0 in cl.metric:
        raise ValueError(
            "regressive_prod is undefined for degenerate metrics "
            "(any 0 in the metric makes the pseudoscalar non-invertible).")
    return _products.product(op, x, w.expand_as(x).contiguous(), cl.metric)
