"""torch.library registrations of the native entry points.

Under ``torch.compile`` the public functions call these operators instead of
their ``autograd.Function`` wrappers: each one is opaque to the tracer, has a
fake (shape-only) implementation and a registered backward, so compiled
models keep the Clifford ops in one graph instead of breaking it at the
ctypes calls (the reference exposes ``compile=True`` knobs for the same
purpose, ``src/cliffordcuda/algebra.py:63-85``). Eager calls keep the direct
``autograd.Function`` path, which has no dispatcher overhead.

Outputs that a backward does not need come back as empty tensors (operator
schemas return plain Tensors) and are turned into ``None`` gradients.
"""
from __future__ import annotations

from typing import Tuple

import torch
from torch import Tensor

_NS = "cliffordcuda_amd"


def _none_if_unneeded(t: Tensor, needed: bool):
    return t if needed else None


def _placeholder(like: Tensor) -> Tensor:
    return like.new_empty(0)


# ---- binary products ---------------------------------------------------------

@torch.library.custom_op(f"{_NS}::product", mutates_args=())
def product(a: Tensor, b: Tensor, op: int, n: int, neg: int, nul: int) -> Tensor:
    from .products import _product_fwd
    return _product_fwd(op, n, neg, nul, a, b)


@product.register_fake
def _(a, b, op, n, neg, nul):
    return torch.empty_like(a)


@torch.library.custom_op(f"{_NS}::product_bwd", mutates_args=())
def product_bwd(a: Tensor, b: Tensor, gc: Tensor, op: int, n: int, neg: int, nul: int, need_a: bool,
                need_b: bool) -> Tuple[Tensor, Tensor]:
    from .products import _product_bwd
    ga, gb = _product_bwd(op, n, neg, nul, a, b, gc, need_a, need_b)
    return (ga if ga is not None else _placeholder(a)), (gb if gb is not None else _placeholder(b))


@product_bwd.register_fake
def _(a, b, gc, op, n, neg, nul, need_a, need_b):
    return (torch.empty_like(a) if need_a else _placeholder(a)), (torch.empty_like(b) if need_b else _placeholder(b))


def _product_setup(ctx, inputs, output):
    a, b, op, n, neg, nul = inputs
    ctx.save_for_backward(a, b)
    ctx.meta = (op, n, neg, nul)


def _product_backward(ctx, gc):
    a, b = ctx.saved_tensors
    need_a, need_b = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    ga, gb = product_bwd(a, b, gc, *ctx.meta, need_a, need_b)
    return _none_if_unneeded(ga, need_a), _none_if_unneeded(gb, need_b), None, None, None, None


product.register_autograd(_product_backward, setup_context=_product_setup)


# ---- graded ops and norm_sq ----------------------------------------------------

@torch.library.custom_op(f"{_NS}::graded", mutates_args=())
def graded(x: Tensor, kind: int, n: int, neg: int, nul: int, grade: int) -> Tensor:
    from .graded import _graded_launch
    return _graded_launch(kind, n, neg, nul, grade, x)


@graded.register_fake
def _(x, kind, n, neg, nul, grade):
    return torch.empty_like(x)


def _graded_setup(ctx, inputs, output):
    _, kind, n, neg, nul, grade = inputs
    ctx.meta = (kind, n, neg, nul, grade)


def _graded_backward(ctx, gy):
    from .graded import graded_adjoint
    kind, n, neg, nul, grade = ctx.meta
    g = graded_adjoint(kind, n, neg, nul, grade, gy, lambda k, n_, ng, nl, gr, t: graded(t, k, n_, ng, nl, gr))
    return g, None, None, None, None, None


graded.register_autograd(_graded_backward, setup_context=_graded_setup)


@torch.library.custom_op(f"{_NS}::norm_sq", mutates_args=())
def norm_sq(x: Tensor, n: int, neg: int, nul: int) -> Tensor:
    from .graded import _norm_sq_fwd
    return _norm_sq_fwd(x, n, neg, nul)


@norm_sq.register_fake
def _(x, n, neg, nul):
    return x.new_empty(x.shape[0])


@torch.library.custom_op(f"{_NS}::norm_sq_bwd", mutates_args=())
def norm_sq_bwd(x: Tensor, gout: Tensor, n: int, neg: int, nul: int) -> Tensor:
    from .graded import _norm_sq_bwd
    return _norm_sq_bwd(x, gout, n, neg, nul)


@norm_sq_bwd.register_fake
def _(x, gout, n, neg, nul):
    return torch.empty_like(x)


def _norm_sq_setup(ctx, inputs, output):
    x, n, neg, nul = inputs
    ctx.save_for_backward(x)
    ctx.meta = (n, neg, nul)


def _norm_sq_backward(ctx, gout):
    (x,) = ctx.saved_tensors
    return norm_sq_bwd(x, gout.contiguous(), *ctx.meta), None, None, None


norm_sq.register_autograd(_norm_sq_backward, setup_context=_norm_sq_setup)


# ---- broadcast-weight products (the layers) ------------------------------------

@torch.library.custom_op(f"{_NS}::bcast_product", mutates_args=())
def bcast_product(x: Tensor, w: Tensor, op: int, side: int, n: int, neg: int, nul: int) -> Tensor:
    from .bcast import _bcast_fwd
    return _bcast_fwd(x, w, op, side, n, neg, nul)


@bcast_product.register_fake
def _(x, w, op, side, n, neg, nul):
    return torch.empty_like(x)


@torch.library.custom_op(f"{_NS}::bcast_product_bwd", mutates_args=())
def bcast_product_bwd(x: Tensor, w: Tensor, gy: Tensor, op: int, side: int, n: int, neg: int, nul: int,
                      need_x: bool, need_w: bool) -> Tuple[Tensor, Tensor]:
    from .bcast import _bcast_bwd
    gx, gw = _bcast_bwd(x, w, gy, op, side, n, neg, nul, need_x, need_w)
    return (gx if gx is not None else _placeholder(x)), (gw if gw is not None else _placeholder(w))


@bcast_product_bwd.register_fake
def _(x, w, gy, op, side, n, neg, nul, need_x, need_w):
    return (torch.empty_like(x) if need_x else _placeholder(x)), (torch.empty_like(w) if need_w else _placeholder(w))


def _bcast_setup(ctx, inputs, output):
    x, w, op, side, n, neg, nul = inputs
    ctx.save_for_backward(x, w)
    ctx.meta = (op, side, n, neg, nul)


def _bcast_backward(ctx, gy):
    x, w = ctx.saved_tensors
    need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    gx, gw = bcast_product_bwd(x, w, gy, *ctx.meta, need_x, need_w)
    return _none_if_unneeded(gx, need_x), _none_if_unneeded(gw, need_w), None, None, None, None, None


bcast_product.register_autograd(_bcast_backward, setup_context=_bcast_setup)


# ---- rotor ---------------------------------------------------------------------

@torch.library.custom_op(f"{_NS}::rotor_compile", mutates_args=())
def rotor_compile(biv: Tensor, n: int) -> Tensor:
    from .rotor import _compile_fwd
    return _compile_fwd(biv, n)


@rotor_compile.register_fake
def _(biv, n):
    from .rotor import _state_len
    return biv.new_empty(_state_len(n))


@torch.library.custom_op(f"{_NS}::rotor_compile_bwd", mutates_args=())
def rotor_compile_bwd(biv: Tensor, g_state: Tensor, n: int) -> Tensor:
    from .rotor import _compile_bwd
    return _compile_bwd(biv, g_state, n)


@rotor_compile_bwd.register_fake
def _(biv, g_state, n):
    return torch.empty_like(biv)


def _rotor_compile_setup(ctx, inputs, output):
    biv, n = inputs
    ctx.save_for_backward(biv)
    ctx.n = n


def _rotor_compile_backward(ctx, g_state):
    (biv,) = ctx.saved_tensors
    return rotor_compile_bwd(biv, g_state.contiguous(), ctx.n), None


rotor_compile.register_autograd(_rotor_compile_backward, setup_context=_rotor_compile_setup)


# The state operators serve apply_bivector: the state's gradient is the
# component of dL/dQ that rotor_compile's backward reads (its cs and spin
# blocks are caches of Q and get zero), not a derivative with respect to every
# state entry, so the state is never handed to callers as a free tensor.
@torch.library.custom_op(f"{_NS}::rotor_apply", mutates_args=())
def rotor_apply(state: Tensor, x: Tensor, n: int) -> Tensor:
    from .rotor import _apply_fwd
    return _apply_fwd(state, x, n)


@rotor_apply.register_fake
def _(state, x, n):
    return torch.empty_like(x)


@torch.library.custom_op(f"{_NS}::rotor_apply_bwd", mutates_args=())
def rotor_apply_bwd(state: Tensor, x: Tensor, gy: Tensor, n: int, need_state: bool,
                    need_x: bool) -> Tuple[Tensor, Tensor]:
    from .rotor import _apply_bwd
    g_state, gx = _apply_bwd(state, x, gy, n, need_state, need_x)
    return (g_state if g_state is not None else _placeholder(state)), (gx if gx is not None else _placeholder(x))


@rotor_apply_bwd.register_fake
def _(state, x, gy, n, need_state, need_x):
    return ((torch.empty_like(state) if need_state else _placeholder(state)),
            (torch.empty_like(x) if need_x else _placeholder(x)))


def _rotor_apply_setup(ctx, inputs, output):
    state, x, n = inputs
    ctx.save_for_backward(state, x)
    ctx.n = n


def _rotor_apply_backward(ctx, gy):
    state, x = ctx.saved_tensors
    need_state, need_x = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    g_state, gx = rotor_apply_bwd(state, x, gy, ctx.n, need_state, need_x)
    return _none_if_unneeded(g_state, need_state), _none_if_unneeded(gx, need_x), None


rotor_apply.register_autograd(_rotor_apply_backward, setup_context=_rotor_apply_setup)


@torch.library.custom_op(f"{_NS}::rotor_compile_cs", mutates_args=())
def rotor_compile_cs(biv: Tensor, n: int) -> Tensor:
    from .rotor import _compile_fwd
    return _compile_fwd(biv, n, want_cs=True)[1]


@rotor_compile_cs.register_fake
def _(biv, n):
    from .rotor import n_planes
    return biv.new_empty(n_planes(n), 2)


@torch.library.custom_op(f"{_NS}::rotor_compile_cs_bwd", mutates_args=())
def rotor_compile_cs_bwd(biv: Tensor, g_cs: Tensor, n: int) -> Tensor:
    from .rotor import _cs_compile_bwd
    return _cs_compile_bwd(biv, g_cs, n)


@rotor_compile_cs_bwd.register_fake
def _(biv, g_cs, n):
    return torch.empty_like(biv)


def _rotor_compile_cs_backward(ctx, g_cs):
    (biv,) = ctx.saved_tensors
    return rotor_compile_cs_bwd(biv, g_cs.contiguous(), ctx.n), None


rotor_compile_cs.register_autograd(_rotor_compile_cs_backward, setup_context=_rotor_compile_setup)


@torch.library.custom_op(f"{_NS}::rotor_cs_apply", mutates_args=())
def rotor_cs_apply(cs: Tensor, x: Tensor, n: int) -> Tensor:
    from .rotor import _cs_apply_fwd
    return _cs_apply_fwd(cs, x, n)


@rotor_cs_apply.register_fake
def _(cs, x, n):
    return torch.empty_like(x)


@torch.library.custom_op(f"{_NS}::rotor_cs_apply_bwd", mutates_args=())
def rotor_cs_apply_bwd(cs: Tensor, y: Tensor, gy: Tensor, n: int, need_cs: bool,
                       need_x: bool) -> Tuple[Tensor, Tensor]:
    from .rotor import _cs_apply_bwd
    g_cs, gx = _cs_apply_bwd(cs, y, gy, n, need_cs, need_x)
    return (g_cs if g_cs is not None else _placeholder(cs)), (gx if gx is not None else _placeholder(y))


@rotor_cs_apply_bwd.register_fake
def _(cs, y, gy, n, need_cs, need_x):
    return ((torch.empty_like(cs) if need_cs else _placeholder(cs)),
            (torch.empty_like(y) if need_x else _placeholder(y)))


def _rotor_cs_apply_setup(ctx, inputs, output):
    cs, x, n = inputs
    ctx.save_for_backward(cs, output)
    ctx.n = n


def _rotor_cs_apply_backward(ctx, gy):
    cs, y = ctx.saved_tensors
    need_cs, need_x = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
    g_cs, gx = rotor_cs_apply_bwd(cs, y, gy, ctx.n, need_cs, need_x)
    return _none_if_unneeded(g_cs, need_cs), _none_if_unneeded(gx, need_x), None


rotor_cs_apply.register_autograd(_rotor_cs_apply_backward, setup_context=_rotor_cs_apply_setup)
