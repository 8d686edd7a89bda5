"""Multivector inverse in Cl(p, q, r): the reference's ``inverse(x, metric,
method, rtol)`` (``src/cliffordcuda/extensions/ga/inverse.py:139-194``), with
the same methods, results and error messages, computed by this package's
kernels (``clf_inverse_versor``, ``clf_inverse_rep``, the product kernels).

* versor: x^-1 = rev(x) / <x rev(x)>_0 when x rev(x) is a scalar (every blade
  and versor). One product launch for x rev(x), then one fused pass that
  divides and flags non-scalar or zero rows.
* rep: the inverse of x's non-null part through a complex matrix
  representation of the non-null generators (side 2^floor(n'/2) <= 128, two
  copies when the non-null pseudoscalar squares to +1), inverted per row in
  LDS; for a degenerate metric the null part is added by Newton steps
  y <- y (2 - x y): the error 1 - x y is nilpotent (it lies in the ideal of the
  null generators), so ceil(log2(r + 1)) steps make it exactly zero.
* lu: the dense solve L(x) y = e_0 with L(x) the left-multiplication matrix
  (L e_j = x e_j), gathered from x with a table of blade-product signs, so the
  memory guard's 2 B 4^n floats (L and the solver's factorised copy) is the
  real peak.

"auto" tries the versor test first, then the representation, then the dense
solve. Every result is checked by the residual |x y - 1| (one product launch).
Gradients: for the rep and dense paths dy = -y dx y (two product backward
launches); for the versor path the derivative of rev(x) / <x rev(x)>_0 as a
function of x, which is what the reference's autograd through that formula
gives.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from ._validate import dim_to_n, metric_masks, normalize_metric

_GEOM = 0
_METHODS = ("auto", "versor", "rep", "lu")


def _geom(x, y, n, neg, nul):
    from .products import _product_fwd
    return _product_fwd(_GEOM, n, neg, nul, x, y)


def _reverse_signs(n, device):
    idx = torch.arange(1 << n, device=device)
    g = torch.zeros_like(idx)
    for b in range(n):
        g += (idx >> b) & 1
    return torch.where((g * (g - 1) // 2) % 2 == 1, -1.0, 1.0).to(torch.float32)


def _norm_weights(n, metric, device):
    """<e_A rev(e_A)>_0 = prod_{k in A} metric[k]: the weight of x_A^2 in <x rev(x)>_0."""
    idx = torch.arange(1 << n, device=device)
    w = torch.ones(1 << n, device=device)
    for k, m in enumerate(metric):
        if m != 1:
            w = torch.where(((idx >> k) & 1).bool(), w * float(m), w)
    return w


def _versor_try(xf, n, neg, nul, rtol):
    """(y, scalar_ok, invertible) for rev(x) / <x rev(x)>_0."""
    from .graded import _graded_launch
    xr = _geom(xf, _graded_launch(0, n, 0, 0, 0, xf), n, neg, nul)
    y = torch.empty_like(xf)
    flags = torch.empty(xf.shape[0], dtype=torch.int32, device=xf.device)
    lib = _lib.load()
    with _lib.on_device(xf):
        rc = lib.clf_inverse_versor(n, xf.data_ptr(), xr.data_ptr(), y.data_ptr(), flags.data_ptr(), float(rtol),
                                    xf.shape[0], _lib.stream_of(xf))
    _lib.check(rc, "clf_inverse_versor")
    f = int(flags.max()) if flags.numel() else 0
    return y, not (f & 1), not (f & 2)


def _rep_supported(n, neg, nul) -> bool:
    return bool(_lib.load().clf_inverse_rep_supported(n, neg, nul))


def _rep_inverse(xf, n, neg, nul):
    y = torch.empty_like(xf)
    singular = torch.empty(xf.shape[0], dtype=torch.int32, device=xf.device)
    lib = _lib.load()
    with _lib.on_device(xf):
        rc = lib.clf_inverse_rep(n, neg, nul, xf.data_ptr(), y.data_ptr(), singular.data_ptr(), xf.shape[0],
                                 _lib.stream_of(xf))
    _lib.check(rc, "clf_inverse_rep")
    r = bin(nul).count("1")
    if r:
        two = torch.zeros_like(xf)
        two[:, 0] = 2.0
        for _ in range(math.ceil(math.log2(r + 1))):
            y = _geom(y, two - _geom(xf, y, n, neg, nul), n, neg, nul)
    if singular.numel() and bool(singular.any()):
        raise ValueError("multivector is not invertible (a zero pivot in its matrix representation).")
    return y


def _lmul_tables(n, neg, nul, device):
    """The left-multiplication matrix L(x) (L e_j = x e_j) as a gather: its
    entry (K, j) is s(K ^ j, j) x[K ^ j], with s(I, J) the sign of the blade
    product e_I e_J (0 when I and J share a null generator): (-1) to the number
    of pairs (i in I, j in J) with i > j, times the squares of the shared
    generators. Returns the index table K ^ j and the sign table."""
    dim = 1 << n
    k = torch.arange(dim, device=device)
    pc = torch.zeros(dim, dtype=torch.int64, device=device)
    for b in range(n):
        pc += (k >> b) & 1
    K, J = k.view(dim, 1), k.view(1, dim)
    I = K ^ J
    swaps = torch.zeros(dim, dim, dtype=torch.int64, device=device)
    for b in range(n):
        swaps += ((J >> b) & 1) * pc[I >> (b + 1)]
    common = I & J
    sign = (1 - 2 * ((swaps + pc[common & neg]) & 1)).to(torch.float32)
    return I, torch.where((common & nul) != 0, torch.zeros_like(sign), sign)


def _dense_inverse(xf, n, neg, nul):
    B, dim = xf.shape
    # L(x) and the solver's factorised copy of it
    need = 2 * B * dim * dim * xf.element_size()
    free, _ = torch.cuda.mem_get_info(xf.device)
    if need > 0.8 * free:
        raise ValueError(
            f"general (non-versor) inverse needs a dense ({B}, 2**{n}, 2**{n}) "
            f"system (~{need/1e9:.1f} GB) but only {free/1e9:.1f} GB is free. "
            f"If x is a versor/blade use method='versor' (no matrix); otherwise "
            f"reduce batch or n.")
    # L(x) gathered from x with the blade-product signs (exact: each entry is
    # +-x_I or 0), built in place
    idx, sign = _lmul_tables(n, neg, nul, xf.device)
    lmat = xf[:, idx]
    lmat.mul_(sign)
    del idx, sign
    rhs = torch.zeros(B, dim, 1, device=xf.device)
    rhs[:, 0, 0] = 1.0
    try:
        y = torch.linalg.solve(lmat, rhs).squeeze(-1).contiguous()
    except torch.linalg.LinAlgError as e:
        raise ValueError(f"multivector is not invertible ({e}).")
    return y


def _residual_guard(xf, y, n, neg, nul, atol, dense):
    prod = _geom(xf, y, n, neg, nul)
    prod[:, 0] -= 1.0
    resid = prod.abs().amax(dim=-1)
    if not bool(torch.isfinite(resid).all()) or bool((resid > atol).any()):
        bad = int((~(resid <= atol)).sum())
        how = "are too ill-conditioned for a stable fp32 inverse" if dense else "too ill-conditioned"
        raise ValueError(
            f"{bad}/{xf.shape[0]} multivector(s) are not invertible or {how} "
            f"(max residual {float(resid.max()):.2e}).")


class _InverseFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, xf, n, metric, method, rtol):
        neg, nul = metric_masks(metric)
        y = None
        versor = False
        if method in ("auto", "versor"):
            yv, scalar, invertible = _versor_try(xf, n, neg, nul, rtol)
            if method == "versor" and not scalar:
                raise ValueError(
                    "method='versor' but x x~ is not scalar (x is not a versor/"
                    "blade); use method='auto', 'rep', or 'lu' for a general inverse.")
            if scalar:
                if not invertible:
                    raise ValueError("multivector is not invertible (x x~ = 0).")
                y, versor = yv, True
        if y is None and method in ("auto", "rep"):
            if _rep_supported(n, neg, nul):
                y = _rep_inverse(xf, n, neg, nul)
                _residual_guard(xf, y, n, neg, nul, 1e-2, dense=False)
            elif method == "rep":
                raise ValueError(
                    "method='rep' but this signature is not representable "
                    "(non-null part too large, or n too large); use 'auto' or 'lu'.")
        if y is None:
            y = _dense_inverse(xf, n, neg, nul)
            _residual_guard(xf, y, n, neg, nul, 1e-2, dense=True)
        ctx.save_for_backward(xf, y)
        ctx.meta = (n, neg, nul, versor, metric)
        return y

    @staticmethod
    def backward(ctx, gy):
        xf, y = ctx.saved_tensors
        n, neg, nul, versor, metric = ctx.meta
        # gy is used as autograd hands it over: the elementwise versor formula
        # broadcasts a batch-stride-0 gradient, and the product backwards read
        # such a gradient as its one row
        if versor:
            # y = rev(x) / s(x), s(x) = sum_A w_A x_A^2
            rs = _reverse_signs(n, xf.device)
            w = _norm_weights(n, metric, xf.device)
            s = (w * xf * xf).sum(-1, keepdim=True)
            dot = (gy * rs * xf).sum(-1, keepdim=True)
            gx = gy * rs / s - (2.0 * dot / (s * s)) * w * xf
            return gx, None, None, None, None
        from .products import _product_bwd
        # dy = -y dx y: gx = -R_y^T L_y^T gy (L_y, R_y: multiplication by y on the left / right)
        (_, h) = _product_bwd(_GEOM, n, neg, nul, y, y, gy, False, True)
        (g, _) = _product_bwd(_GEOM, n, neg, nul, y, y, h, True, False)
        return -g, None, None, None, None


def inverse(x: torch.Tensor, metric=None, method: str = "auto", rtol: float = 1e-4) -> torch.Tensor:
    """Inverse x^-1 of multivectors x (..., 2^n) in Cl(p, q, r); ``method`` in
    {"auto", "versor", "rep", "lu"}. Raises ValueError if x is not invertible
    or the requested method does not apply. Differentiable w.r.t. x."""
    dim = x.size(-1)
    n = dim_to_n(dim)
    metric = normalize_metric(n, metric)
    if method not in _METHODS:
        raise ValueError(f"method must be 'auto', 'versor', 'rep', or 'lu'; got {method!r}")
    lead = x.shape[:-1]
    xf = x.reshape(-1, dim).contiguous()
    if xf.shape[0] == 0:
        return x.clone()
    return _InverseFunc.apply(xf, n, metric, method, rtol).reshape(*lead, dim)
