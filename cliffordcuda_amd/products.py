"""Differentiable binary products backed by the gfx950 kernels.

Free-function surface of the reference (``src/cliffordcuda/__init__.py:2-26``):
``geom_prod``, ``wedge_prod``, ``inner_prod``, ``left_contract``,
``right_contract``, ``regressive_prod`` with ``metric=None`` meaning Cl(n, 0),
plus the reference's variant names (``*_multik``, ``*_skip``, ``*_kskip``,
``*_subset_grade``), which compute the same products and are aliases here.

Forward and backward each make one kernel launch through the C ABI
(``clf_product_fwd`` / ``clf_product_bwd``); the backward produces both input
gradients in one pass over the upstream gradient, where the reference launches
its forward kernel twice (``extensions/ga/geom_prod.py:242-250``).
"""
from __future__ import annotations

import importlib.util
import os

import torch

from . import _lib, _ops
from ._validate import dim_to_n, metric_masks, normalize_metric

_EXT_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_clf_autograd.so")
_ext = None
_ext_tried = False


def _autograd_ext():
    """The products' C++ autograd node (csrc/torch_autograd.cpp, built in-tree
    by __graft_entry__.build()), or None when it is not built: then the Python
    autograd.Function below runs the same library calls."""
    global _ext, _ext_tried
    if not _ext_tried:
        _ext_tried = True
        if os.path.exists(_EXT_PATH):
            _lib.load()  # the library first: its ABI check, and the extension links to it
            spec = importlib.util.spec_from_file_location("_clf_autograd", _EXT_PATH)
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            _ext = mod
    return _ext


def _check_operands(a: torch.Tensor, b: torch.Tensor, name: str):
    if not (isinstance(a, torch.Tensor) and isinstance(b, torch.Tensor)):
        raise TypeError(f"{name}: operands must be torch.Tensors")
    if not (a.is_cuda and b.is_cuda):
        raise RuntimeError(f"{name}: operands must be GPU tensors")
    if a.dtype != torch.float32 or b.dtype != torch.float32:
        raise RuntimeError(f"{name}: operands must be float32")
    if a.shape != b.shape:
        raise RuntimeError(f"{name}: operand shapes differ: {tuple(a.shape)} vs {tuple(b.shape)}")
    if a.device != b.device:
        raise RuntimeError(f"{name}: operands on different devices")


def _product_fwd(op_code, n, neg, nul, a, b):
    c = torch.empty_like(a)
    lib = _lib.load()
    with _lib.on_device(a):
        rc = lib.clf_product_fwd(op_code, n, neg, nul, a.data_ptr(), b.data_ptr(), c.data_ptr(),
                                 a.shape[0], _lib.stream_of(a))
    _lib.check(rc, "clf_product_fwd")
    return c


def _product_bwd(op_code, n, neg, nul, a, b, gc, need_a, need_b):
    ga = torch.empty_like(a) if need_a else None
    gb = torch.empty_like(b) if need_b else None
    if ga is None and gb is None:
        return None, None
    gc, ldg = _lib.grad_rows(gc, a.shape[1])
    lib = _lib.load()
    with _lib.on_device(a):
        rc = lib.clf_product_bwd_ld(op_code, n, neg, nul, a.data_ptr(), b.data_ptr(), gc.data_ptr(), ldg,
                                    _lib.ptr(ga), _lib.ptr(gb), a.shape[0], _lib.stream_of(a))
    _lib.check(rc, "clf_product_bwd_ld")
    return ga, gb


class _ProductFunc(torch.autograd.Function):
    """c = op(a, b) on (batch, 2^n) rows; backward to both operands.
    Same chain-rule formulas as the reference's per-product autograd wrappers
    (``geom_prod.py:216-250``, ``wedge_prod/chunk.py:70-102``,
    ``inner_prod/chunk.py:66-98``, ``left_contract.py:87-118``,
    ``right_contract.py:76-107``, ``regressive_prod.py:143-183``)."""

    @staticmethod
    def forward(ctx, a, b, op_code, n, neg, nul):
        ctx.save_for_backward(a, b)
        ctx.meta = (op_code, n, neg, nul)
        return _product_fwd(op_code, n, neg, nul, a, b)

    @staticmethod
    def backward(ctx, gc):
        a, b = ctx.saved_tensors
        op_code, n, neg, nul = ctx.meta
        ga, gb = _product_bwd(op_code, n, neg, nul, a, b, gc,
                              ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return ga, gb, None, None, None, None


_PLANS: dict = {}


def _plan(op: str, dim: int, metric) -> tuple:
    """(op code, n, negative mask, null mask) of a call, validated once per
    (op, row length, metric) and then looked up: the published benchmarks call
    the products on a few rows, where host time is the latency."""
    if metric is not None and type(metric) is not tuple:
        metric = tuple(metric)
    key = (op, dim, metric)
    plan = _PLANS.get(key)
    if plan is None:
        code = _lib.OP_CODES[op]
        n = dim_to_n(dim)
        full = normalize_metric(n, metric)
        if op == "regressive" and 0 in full:
            raise ValueError(f"regressive product undefined for degenerate metric {full}")
        neg, nul = metric_masks(full)
        plan = (code, n, neg, nul)
        if len(_PLANS) < 4096:
            _PLANS[key] = plan
    return plan


def product(op: str, a: torch.Tensor, b: torch.Tensor, metric=None) -> torch.Tensor:
    """Generic entry: ``op`` in {geom, wedge, inner, lc, rc, regressive};
    inputs (..., 2^n) fp32 on the GPU, same shape."""
    _check_operands(a, b, op)
    shape = a.shape
    dim = shape[-1]
    code, n, neg, nul = _plan(op, dim, metric)
    flat = len(shape) != 2  # (batch, dim) inputs go in as they are: no view nodes in the autograd graph
    a2 = a.contiguous().reshape(-1, dim) if flat else a.contiguous()
    b2 = b.contiguous().reshape(-1, dim) if flat else b.contiguous()
    out = run_rows(a2, b2, code, n, neg, nul)
    return out.reshape(shape) if flat else out


def run_rows(a2, b2, code, n, neg, nul):
    """The product of checked (batch, 2^n) contiguous fp32 GPU operands of one
    shape: the custom op under torch.compile, the autograd node when a
    gradient may be needed, else the launch alone."""
    ext = _ext if _ext_tried else _autograd_ext()
    if torch.compiler.is_compiling():
        return _ops.product(a2, b2, code, n, neg, nul)
    if torch.is_grad_enabled() and (a2.requires_grad or b2.requires_grad):
        return ext.product(a2, b2, code, n, neg, nul) if ext is not None else _ProductFunc.apply(a2, b2, code, n, neg,
                                                                                                 nul)
    if ext is not None:  # nothing to differentiate: the launch without the autograd node
        return ext.product_fwd(a2, b2, code, n, neg, nul)
    return _product_fwd(code, n, neg, nul, a2, b2)


def geom_prod(a, b, metric=None):
    """Geometric product in Cl(p,q,r) (reference ``extensions/ga/geom_prod.py:253-276``)."""
    return product("geom", a, b, metric)


def wedge_prod(a, b, metric=None):
    """Outer product (reference ``extensions/ga/wedge_prod/chunk.py:105-121``)."""
    return product("wedge", a, b, metric)


def inner_prod(a, b, metric=None):
    """Hestenes inner product incl. scalar terms (reference ``inner_prod/chunk.py:101-115``)."""
    return product("inner", a, b, metric)


def left_contract(a, b, metric=None):
    """Left contraction (reference ``extensions/ga/left_contract.py:121-138``)."""
    return product("lc", a, b, metric)


def right_contract(a, b, metric=None):
    """Right contraction (reference ``extensions/ga/right_contract.py:110-127``)."""
    return product("rc", a, b, metric)


def regressive_prod(a, b, metric=None):
    """Regressive product dual(dual a ^ dual b), non-degenerate metrics only
    (reference ``extensions/ga/regressive_prod.py:186-201``)."""
    return product("regressive", a, b, metric)


# spelling used by CliffordAlgebra and the north-star API
left_contraction = left_contract
right_contraction = right_contract

# The reference's kernel variants (multik / skip / kskip / subset-grade,
# ``src/cliffordcuda/__init__.py:3-20``) compute the same products with other
# CUDA launch shapes; on gfx950 one kernel serves all of them.
geom_prod_multik = geom_prod
wedge_prod_multik = wedge_prod
wedge_prod_skip = wedge_prod
wedge_prod_multik_skip = wedge_prod
wedge_prod_subset_grade = wedge_prod
inner_prod_kskip = inner_prod
inner_prod_multik = inner_prod
inner_prod_multik_skip = inner_prod
inner_prod_skip = inner_prod
inner_prod_subset_grade = inner_prod
left_contract_skip = left_contract
left_contract_subset_grade = left_contract
right_contract_skip = right_contract
right_contract_subset_grade = right_contract
regressive_prod_skip = regressive_prod
regressive_prod_subset_grade = regressive_prod
