"""Rotor compile (bivector -> rotor state) and the sandwich ~R x R, differentiable
to the bivector and to x, on the gfx950 kernels (``clf_rotor_*``).

Semantics are the reference's composite ``compile_bivector`` + ``apply_rotor``
(``src/cliffordcuda/algebra.py:343-373``): Euclidean rotor
R = exp(sum_m b_m e_{i_m} e_{j_m}), bivector slots in ``triu_indices(n, n, 1)``
order, y = ~R x R, whatever the algebra's metric (the reference ignores it on
this path too). The rotor state is a 1-D float tensor (rotation matrix + its
plane-rotation chain) that ``apply_rotor`` consumes; it is produced in one
kernel launch with no host synchronisation.
"""
from __future__ import annotations

import torch

from . import _lib, _ops


def _state_len(n: int) -> int:
    """Floats of the rotor state: the n x n rotation, the (c, s) pairs of its
    C(n, 2) plane rotations and, for n = 8, the 16 x 16 spin matrix of the
    Cl(8,0) representation (``clf_rotor_state_floats``, computed here without
    a library call so that traced graphs stay free of host calls)."""
    if not 2 <= n <= 10:
        raise ValueError(f"rotor kernels support 2 <= n <= 10; got n={n}")
    return n * n + n * (n - 1) + (256 if n == 8 else 0)


def _compile_fwd(biv: torch.Tensor, n: int) -> torch.Tensor:
    biv = biv.contiguous()
    state = torch.empty(_state_len(n), dtype=torch.float32, device=biv.device)
    lib = _lib.load()
    with torch.cuda.device(biv.device):
        rc = lib.clf_rotor_compile_fwd(n, biv.data_ptr(), state.data_ptr(), _lib.stream_of(biv))
    _lib.check(rc, "clf_rotor_compile_fwd")
    return state


def _compile_bwd(biv: torch.Tensor, g_state: torch.Tensor, n: int) -> torch.Tensor:
    biv = biv.contiguous()
    g_state = g_state.contiguous()
    g_biv = torch.empty_like(biv)
    lib = _lib.load()
    with torch.cuda.device(biv.device):
        rc = lib.clf_rotor_compile_bwd(n, biv.data_ptr(), g_state.data_ptr(), g_biv.data_ptr(), _lib.stream_of(biv))
    _lib.check(rc, "clf_rotor_compile_bwd")
    return g_biv


def _apply_fwd(state: torch.Tensor, x: torch.Tensor, n: int) -> torch.Tensor:
    y = torch.empty_like(x)
    lib = _lib.load()
    with torch.cuda.device(x.device):
        rc = lib.clf_rotor_apply_fwd(n, state.data_ptr(), x.data_ptr(), y.data_ptr(), x.shape[0], _lib.stream_of(x))
    _lib.check(rc, "clf_rotor_apply_fwd")
    return y


def _apply_bwd(state: torch.Tensor, x: torch.Tensor, gy: torch.Tensor, n: int, need_state: bool, need_x: bool):
    if not (need_state or need_x):
        return None, None
    gy = gy.contiguous()
    gx = torch.empty_like(x) if need_x else None
    g_state = torch.empty_like(state) if need_state else None
    lib = _lib.load()
    ws = None
    ws_bytes = 0
    if need_state:
        ws_bytes = lib.clf_rotor_apply_ws_bytes(n, x.shape[0])
        ws = torch.empty(max(1, ws_bytes // 4), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        rc = lib.clf_rotor_apply_bwd(n, state.data_ptr(), x.data_ptr(), gy.data_ptr(), _lib.ptr(gx),
                                     _lib.ptr(g_state), x.shape[0], _lib.ptr(ws), ws_bytes, _lib.stream_of(x))
    _lib.check(rc, "clf_rotor_apply_bwd")
    return g_state, gx


class _CompileFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, biv, n):
        ctx.save_for_backward(biv)
        ctx.n = n
        return _compile_fwd(biv, n)

    @staticmethod
    def backward(ctx, g_state):
        (biv,) = ctx.saved_tensors
        return _compile_bwd(biv, g_state, ctx.n), None


class _ApplyFunc(torch.autograd.Function):
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


def compile_bivector(bivector: torch.Tensor, n: int) -> torch.Tensor:
    """(1, C(n,2)) bivector -> rotor state (1-D). Differentiable."""
    if torch.compiler.is_compiling():
        return _ops.rotor_compile(bivector.reshape(-1).contiguous(), n)
    return _CompileFunc.apply(bivector.reshape(-1), n)


def apply_rotor(state: torch.Tensor, x: torch.Tensor, n: int) -> torch.Tensor:
    """y = ~R x R for x (batch, 2^n). Differentiable to the state and to x."""
    if state.dim() != 1 or state.numel() != _state_len(n):
        raise ValueError(
            f"rotor state must be the 1-D tensor compile_bivector returns ({_state_len(n)} floats for "
            f"n={n}); got shape {tuple(state.shape)}")
    if state.device != x.device:
        raise ValueError(f"rotor state on device {state.device}, x on {x.device}")
    if torch.compiler.is_compiling():
        return _ops.rotor_apply(state.contiguous(), x.contiguous(), n)
    return _ApplyFunc.apply(state.contiguous(), x, n)
