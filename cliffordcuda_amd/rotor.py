"""Rotor compile (bivector -> Givens cs) and the sandwich ~R x R, differentiable
to the bivector, to cs and to x, on the gfx950 kernels (``clf_rotor_*``).

Semantics are the reference's (``src/cliffordcuda/algebra.py:343-373``):

* ``compile_bivector(b)`` returns the (C(n,2), 2) tensor ``cs`` of Givens
  factors of R = expm(2 (M - M^T)) (lex planes, plane k at row C - 1 - k, the
  layout of ``kernels/rotor/givens_factor.cu:23-38``), differentiable to the
  bivector;
* ``apply_rotor(cs, x)`` runs the plane chain of any such cs (built by
  ``compile_bivector``, by hand, or learned) and is differentiable to cs (the
  reference's rule, ``givens_apply_mb_perm_packed.cu:111-160``) and to x (the
  reference has no gradient to x);
* ``apply_bivector(b, x)`` is their composition: the Euclidean sandwich
  ~R x R with R = exp(sum_m b_m e_{i_m} e_{j_m}), whatever the algebra's
  metric (the reference ignores it on this path too).

Besides cs, a compile produces the library's own rotor state: the rotation Q
and, for n = 8, the rotor's 16 x 16 matrix in the real representation of
Cl(8,0), which the n = 8 sandwich kernels run on the matrix cores. The state is
internal: ``apply_bivector`` (and ``RotorLayer``) differentiate through it to
the bivector directly, and ``apply_rotor`` runs its forward on it when it is
handed a cs that ``compile_bivector`` produced and that has not changed since
(cs stays in y's autograd graph; its gradient comes from the plane chain's
backward); any other cs runs the plane chain itself.

The gradient to cs follows the reference's rule (each plane's input rebuilt
from the chain's output with the transposed pair map), which is the true
derivative for unit (c, s) pairs, the pairs ``compile_bivector`` makes; for
other pairs it is the reference's value, not the derivative.
"""
from __future__ import annotations

import torch

from . import _lib, _ops


def _check_n(n: int):
    if not 2 <= n <= 12:
        raise ValueError(f"rotor kernels support 2 <= n <= 12; got n={n}")


def _state_len(n: int) -> int:
    """Floats of the rotor state: the n x n rotation, the cs pairs and, for
    n = 8, the 16 x 16 spin matrix (``clf_rotor_state_floats``, computed here
    without a library call so that traced graphs stay free of host calls)."""
    _check_n(n)
    return n * n + n * (n - 1) + (256 if n == 8 else 0)


def n_planes(n: int) -> int:
    return n * (n - 1) // 2


# ---- native calls ---------------------------------------------------------------

def _compile_fwd(biv: torch.Tensor, n: int, want_cs: bool = False):
    biv = biv.contiguous()
    state = torch.empty(_state_len(n), dtype=torch.float32, device=biv.device)
    cs = torch.empty(n_planes(n), 2, dtype=torch.float32, device=biv.device) if want_cs else None
    lib = _lib.load()
    with _lib.on_device(biv):
        rc = lib.clf_rotor_compile_fwd(n, biv.data_ptr(), state.data_ptr(), _lib.ptr(cs), _lib.stream_of(biv))
    _lib.check(rc, "clf_rotor_compile_fwd")
    return (state, cs) if want_cs else state


def _compile_bwd(biv: torch.Tensor, g_state: torch.Tensor, n: int) -> torch.Tensor:
    biv = biv.contiguous()
    g_state = g_state.contiguous()
    g_biv = torch.empty_like(biv)
    lib = _lib.load()
    with _lib.on_device(biv):
        rc = lib.clf_rotor_compile_bwd(n, biv.data_ptr(), g_state.data_ptr(), g_biv.data_ptr(), _lib.stream_of(biv))
    _lib.check(rc, "clf_rotor_compile_bwd")
    return g_biv


def _cs_compile_bwd(biv: torch.Tensor, g_cs: torch.Tensor, n: int) -> torch.Tensor:
    biv = biv.contiguous()
    g_cs = g_cs.contiguous()
    g_biv = torch.empty_like(biv)
    lib = _lib.load()
    with _lib.on_device(biv):
        rc = lib.clf_rotor_cs_compile_bwd(n, biv.data_ptr(), g_cs.data_ptr(), g_biv.data_ptr(), _lib.stream_of(biv))
    _lib.check(rc, "clf_rotor_cs_compile_bwd")
    return g_biv


def _apply_fwd(state: torch.Tensor, x: torch.Tensor, n: int) -> torch.Tensor:
    y = torch.empty_like(x)
    lib = _lib.load()
    with _lib.on_device(x):
        rc = lib.clf_rotor_apply_fwd(n, state.data_ptr(), x.data_ptr(), y.data_ptr(), x.shape[0], _lib.stream_of(x))
    _lib.check(rc, "clf_rotor_apply_fwd")
    return y


def _apply_bwd(state: torch.Tensor, x: torch.Tensor, gy: torch.Tensor, n: int, need_state: bool, need_x: bool):
    if not (need_state or need_x):
        return None, None
    gy, ldg = _lib.grad_rows(gy, x.shape[1])
    gx = torch.empty_like(x) if need_x else None
    g_state = torch.empty_like(state) if need_state else None
    lib = _lib.load()
    ws = None
    ws_bytes = 0
    if need_state:
        ws_bytes = lib.clf_rotor_apply_ws_bytes(n, x.shape[0])
        ws = torch.empty(max(1, ws_bytes // 4), dtype=torch.float32, device=x.device)
    with _lib.on_device(x):
        rc = lib.clf_rotor_apply_bwd_ld(n, state.data_ptr(), x.data_ptr(), gy.data_ptr(), ldg, _lib.ptr(gx),
                                        _lib.ptr(g_state), x.shape[0], _lib.ptr(ws), ws_bytes, _lib.stream_of(x))
    _lib.check(rc, "clf_rotor_apply_bwd_ld")
    return g_state, gx


def _biv_apply_bwd(biv: torch.Tensor, state: torch.Tensor, x: torch.Tensor, gy: torch.Tensor, n: int,
                   need_biv: bool, need_x: bool):
    """Gradients of apply(compile(biv), x) to biv and x in one library call."""
    if not (need_biv or need_x):
        return None, None
    gy, ldg = _lib.grad_rows(gy, x.shape[1])
    gx = torch.empty_like(x) if need_x else None
    g_biv = torch.empty_like(biv) if need_biv else None
    lib = _lib.load()
    ws = None
    ws_bytes = 0
    if need_biv:
        ws_bytes = lib.clf_rotor_bivector_apply_ws_bytes(n, x.shape[0])
        ws = torch.empty(max(1, ws_bytes // 4), dtype=torch.float32, device=x.device)
    with _lib.on_device(x):
        rc = lib.clf_rotor_bivector_apply_bwd(n, biv.data_ptr(), state.data_ptr(), x.data_ptr(), gy.data_ptr(), ldg,
                                              _lib.ptr(gx), _lib.ptr(g_biv), x.shape[0], _lib.ptr(ws), ws_bytes,
                                              _lib.stream_of(x))
    _lib.check(rc, "clf_rotor_bivector_apply_bwd")
    return g_biv, gx


def _cs_apply_fwd(cs: torch.Tensor, x: torch.Tensor, n: int) -> torch.Tensor:
    y = torch.empty_like(x)
    lib = _lib.load()
    with _lib.on_device(x):
        rc = lib.clf_rotor_cs_apply_fwd(n, cs.data_ptr(), x.data_ptr(), y.data_ptr(), x.shape[0], _lib.stream_of(x))
    _lib.check(rc, "clf_rotor_cs_apply_fwd")
    return y


def _cs_apply_bwd(cs: torch.Tensor, y: torch.Tensor, gy: torch.Tensor, n: int, need_cs: bool, need_x: bool):
    if not (need_cs or need_x):
        return None, None
    gy, ldg = _lib.grad_rows(gy, y.shape[1])
    gx = torch.empty_like(y) if need_x else None
    g_cs = torch.empty_like(cs) if need_cs else None
    lib = _lib.load()
    ws = None
    ws_bytes = 0
    if need_cs:
        ws_bytes = lib.clf_rotor_cs_apply_ws_bytes(n, y.shape[0])
        ws = torch.empty(max(1, ws_bytes // 4), dtype=torch.float32, device=y.device)
    with _lib.on_device(y):
        rc = lib.clf_rotor_cs_apply_bwd_ld(n, cs.data_ptr(), y.data_ptr(), gy.data_ptr(), ldg, _lib.ptr(gx),
                                           _lib.ptr(g_cs), y.shape[0], _lib.ptr(ws), ws_bytes, _lib.stream_of(y))
    _lib.check(rc, "clf_rotor_cs_apply_bwd_ld")
    return g_cs, gx


# ---- autograd ---------------------------------------------------------------------

class _StateApplyFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, state, x, n):
        ctx.save_for_backward(state, x)
        ctx.n = n
        return _apply_fwd(state, x, n)

    @staticmethod
    def backward(ctx, gy):
        state, x = ctx.saved_tensors
        g_state, gx = _apply_bwd(state, x, gy, ctx.n, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return g_state, gx, None


class _BivectorApplyFunc(torch.autograd.Function):
    """y = ~R x R with R compiled from the bivector in the same call: one
    autograd node for compile and apply, whose backward is one library call
    (apply backward, batch sum and compile backward)."""

    @staticmethod
    def forward(ctx, biv, x, n):
        state = _compile_fwd(biv, n)
        ctx.save_for_backward(biv, state, x)
        ctx.n = n
        return _apply_fwd(state, x, n)

    @staticmethod
    def backward(ctx, gy):
        biv, state, x = ctx.saved_tensors
        g_biv, gx = _biv_apply_bwd(biv, state, x, gy, ctx.n, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return g_biv, gx, None


class _CompiledCsApplyFunc(torch.autograd.Function):
    """y = chain(cs) x for a cs that ``compile_bivector`` made and nobody has
    changed since: the forward runs on that compile's state (the n = 8 kernels
    on the matrix cores), cs stays an input of the node, so gradients and hooks
    reach cs and, through cs's own node, the bivector."""

    @staticmethod
    def forward(ctx, cs, x, state, n):
        y = _apply_fwd(state, x, n)
        ctx.save_for_backward(cs, state, x, y)
        ctx.n = n
        return y

    @staticmethod
    def backward(ctx, gy):
        cs, state, x, y = ctx.saved_tensors
        if ctx.needs_input_grad[0]:
            g_cs, gx = _cs_apply_bwd(cs, y, gy, ctx.n, True, ctx.needs_input_grad[1])
        else:
            _, gx = _apply_bwd(state, x, gy, ctx.n, False, ctx.needs_input_grad[1])
            g_cs = None
        return g_cs, gx, None, None


class _CompileCsFunc(torch.autograd.Function):
    """bivector -> cs (the reference's compile_bivector output). The internal
    state made by the same launch is handed out through ``holder``."""

    @staticmethod
    def forward(ctx, biv, n, holder):
        state, cs = _compile_fwd(biv, n, want_cs=True)
        holder.append(state)
        ctx.save_for_backward(biv)
        ctx.n = n
        return cs

    @staticmethod
    def backward(ctx, g_cs):
        (biv,) = ctx.saved_tensors
        return _cs_compile_bwd(biv, g_cs, ctx.n), None, None


class _CsApplyFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, cs, x, n):
        y = _cs_apply_fwd(cs, x, n)
        ctx.save_for_backward(cs, y)
        ctx.n = n
        return y

    @staticmethod
    def backward(ctx, gy):
        cs, y = ctx.saved_tensors
        g_cs, gx = _cs_apply_bwd(cs, y, gy, ctx.n, ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        return g_cs, gx, None


class _Compiled:
    """What ``compile_bivector`` knows about the cs it returned: the internal
    state of the same compile, and the version and address that say whether cs
    has changed since."""

    __slots__ = ("state", "cs_version", "cs_ptr")

    def __init__(self, state, cs):
        self.state = state
        self.cs_version = cs._version
        self.cs_ptr = cs.data_ptr()

    def unchanged(self, cs) -> bool:
        return cs._version == self.cs_version and cs.data_ptr() == self.cs_ptr


# ---- public functions ---------------------------------------------------------------

def compile_bivector(bivector: torch.Tensor, n: int) -> torch.Tensor:
    """(1, C(n,2)) bivector -> cs (C(n,2), 2), the reference's Givens factors.
    Differentiable to the bivector."""
    _check_n(n)
    biv = bivector.reshape(-1)
    if torch.compiler.is_compiling():
        return _ops.rotor_compile_cs(biv.contiguous(), n)
    holder = []
    cs = _CompileCsFunc.apply(biv, n, holder)
    cs._clf_rotor = _Compiled(holder[0], cs)
    return cs


def check_cs(cs, n: int, device) -> None:
    C = n_planes(n)
    if not isinstance(cs, torch.Tensor):
        raise ValueError(f"cs must be a torch.Tensor, got {type(cs).__name__}")
    if tuple(cs.shape) != (C, 2):
        raise ValueError(
            f"cs must have shape ({C}, 2) (the output of compile_bivector for n={n}); got {tuple(cs.shape)}")
    if cs.dtype != torch.float32:
        raise ValueError(f"cs must be float32, got {cs.dtype}")
    if cs.device != device:
        raise ValueError(f"cs on device {cs.device}, x on {device}")


def apply_rotor(cs: torch.Tensor, x: torch.Tensor, n: int) -> torch.Tensor:
    """y = chain(cs) x for x (batch, 2^n): ~R x R when cs = compile_bivector(b).
    Differentiable to cs and to x."""
    check_cs(cs, n, x.device)
    if torch.compiler.is_compiling():
        return _ops.rotor_cs_apply(cs.contiguous(), x.contiguous(), n)
    info = getattr(cs, "_clf_rotor", None)
    grad = torch.is_grad_enabled() and (x.requires_grad or cs.requires_grad)
    if info is not None and info.unchanged(cs):
        if grad and cs.requires_grad:
            return _CompiledCsApplyFunc.apply(cs, x, info.state, n)
        # nothing to differentiate: the launch without an autograd node
        return _StateApplyFunc.apply(info.state, x, n) if grad else _apply_fwd(info.state, x, n)
    return _CsApplyFunc.apply(cs.contiguous(), x, n) if grad else _cs_apply_fwd(cs.contiguous(), x, n)


def apply_bivector(bivector: torch.Tensor, x: torch.Tensor, n: int) -> torch.Tensor:
    """y = ~R x R, R = exp(sum_m b_m e_{i_m} e_{j_m}); differentiable to the
    bivector and to x (one compile launch, the state never leaves this call)."""
    _check_n(n)
    if torch.compiler.is_compiling():
        return _ops.rotor_apply(_ops.rotor_compile(bivector.reshape(-1).contiguous(), n), x.contiguous(), n)
    # the kernels read the C(n,2) floats of a contiguous bivector whatever its shape
    return _BivectorApplyFunc.apply(bivector.contiguous(), x, n)
