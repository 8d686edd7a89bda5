"""Multivector inverse (reference ``src/cliffordcuda/extensions/ga/inverse.py:139-194``).

Two paths, selected like the reference's ``method`` argument:
  * versor / blade fast path ``x~ / (x x~)`` when ``x x~`` is a scalar;
  * general path: the dense solve ``L(x) y = e_0`` with ``L(x)[k, j] =
    sigma(j^k, j) x[j^k]`` (left-multiplication matrix), verified by the
    residual ``|x y - 1|``. ``method="rep"`` is served by the same dense solve
    (the reference's matrix-representation inverse computes the same
    mathematical inverse).
Both are torch code over this package's geometric-product kernel.
"""
from __future__ import annotations

from functools import lru_cache

import torch

from ._validate import dim_to_n, normalize_metric
from .graded import reverse
from .products import geom_prod


@lru_cache(maxsize=None)
def _left_mult_tables(n: int, metric: tuple, device: str):
    """S[k, j] = sigma(j^k, j) and gather index a[k, j] = j^k, built from the
    closed-form sign on the device."""
    dim = 1 << n
    k = torch.arange(dim, device=device, dtype=torch.int64).view(dim, 1)
    j = torch.arange(dim, device=device, dtype=torch.int64).view(1, dim)
    i = j ^ k
    par = torch.zeros(dim, dim, dtype=torch.int64, device=device)
    for a in range(n):
        ia = (i >> a) & 1
        for b in range(a):
            par += ia * ((j >> b) & 1)
    sign = (1 - 2 * (par & 1)).to(torch.float32)
    common = i & j
    for g, m in enumerate(metric):
        if m != 1:
            hit = ((common >> g) & 1).bool()
            sign = torch.where(hit, sign * float(m), sign)
    return sign, i


def _versor_inverse(x, metric, rtol):
    r = reverse(x)
    xr = geom_prod(x, r, metric=metric)
    s = xr[..., :1]
    nonscalar = xr[..., 1:].abs().amax(dim=-1, keepdim=True) if xr.shape[-1] > 1 else torch.zeros_like(s)
    scale = xr.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
    ok = bool((nonscalar <= rtol * scale).all())
    return r / s, s, ok


def _dense_inverse(xf, metric, atol=1e-2):
    B, dim = xf.shape
    n = dim_to_n(dim)
    S, a = _left_mult_tables(n, tuple(metric), str(xf.device))
    L = S * xf[:, a]
    rhs = torch.zeros(B, dim, 1, device=xf.device, dtype=xf.dtype)
    rhs[:, 0, 0] = 1.0
    try:
        y = torch.linalg.solve(L, rhs).squeeze(-1)
    except torch.linalg.LinAlgError as e:
        raise ValueError(f"multivector is not invertible ({e}).")
    with torch.no_grad():
        resid = (geom_prod(xf, y.contiguous(), metric=metric) - rhs.squeeze(-1)).abs().amax(dim=-1)
    if not bool(torch.isfinite(resid).all()) or bool((resid > atol).any()):
        bad = int((~(resid <= atol)).sum())
        raise ValueError(
            f"{bad}/{B} multivector(s) are not invertible or are too ill-conditioned for a stable "
            f"fp32 inverse (max residual {float(resid.max()):.2e}).")
    return y


def inverse(x: torch.Tensor, metric=None, method: str = "auto", rtol: float = 1e-4) -> torch.Tensor:
    """Inverse x^{-1} in Cl(p,q,r); ``method`` in {"auto", "versor", "rep", "lu"}."""
    dim = x.size(-1)
    n = dim_to_n(dim)
    metric = normalize_metric(n, metric)
    lead = x.shape[:-1]
    xf = x.reshape(-1, dim).contiguous()
    if method in ("auto", "versor"):
        inv_v, s, ok = _versor_inverse(xf, metric, rtol)
        if method == "versor" and not ok:
            raise ValueError(
                "method='versor' but x x~ is not scalar (x is not a versor/blade); use "
                "method='auto', 'rep', or 'lu' for a general inverse.")
        if ok:
            if bool((s.abs() < 1e-20).any()):
                raise ValueError("multivector is not invertible (x x~ = 0).")
            return inv_v.reshape(*lead, dim)
    elif method not in ("lu", "rep"):
        raise ValueError(f"method must be 'auto', 'versor', 'rep', or 'lu'; got {method!r}")
    return _dense_inverse(xf, metric).reshape(*lead, dim)
