"""Boundary checks with the same exception types and messages as the reference
(``src/cliffordcuda/_validate.py:10-82``), so callers that match on them keep
working. All checks run before any device work."""
from __future__ import annotations

import torch


def check_device(device) -> torch.device:
    """A GPU device (torch's ``cuda`` type, which is HIP on ROCm), with a
    concrete index (reference ``_validate.py:10-27``)."""
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError(f"cliffordcuda is CUDA-only; device must be a CUDA device, got {dev}")
    if not torch.cuda.is_available():
        raise RuntimeError("cliffordcuda requires CUDA, but torch.cuda.is_available() is False")
    if dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def check_metric(metric) -> tuple:
    """Reference ``_validate.py:30-39``."""
    if not hasattr(metric, "__iter__"):
        raise ValueError("metric must be an iterable of {-1, 0, +1}")
    metric = tuple(int(m) for m in metric)
    if any(m not in (-1, 0, 1) for m in metric):
        raise ValueError(f"metric entries must each be in {{-1, 0, +1}}, got {metric}")
    if len(metric) < 1:
        raise ValueError("metric must have at least one entry")
    return metric


def _same_device(t: torch.Tensor, device: torch.device) -> bool:
    return t.device.type == device.type and (device.index is None or t.device.index == device.index)


def check_mv(tensor, name, dim, device, dtype):
    """Reference ``_validate.py:42-59``."""
    if not isinstance(tensor, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor, got {type(tensor).__name__}")
    if tensor.dim() != 2:
        raise ValueError(f"{name} must be 2D (batch, 2^n); got shape {tuple(tensor.shape)}")
    if tensor.shape[-1] != dim:
        raise ValueError(f"{name} last dim {tensor.shape[-1]} != 2^n = {dim}")
    if not _same_device(tensor, device):
        raise ValueError(f"{name} on device {tensor.device}, algebra pinned to {device}")
    if tensor.dtype != dtype:
        raise ValueError(f"{name} dtype {tensor.dtype}, algebra dtype {dtype}")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def check_bivector(b, n, num_basis_biv, device, dtype):
    """Reference ``_validate.py:62-82``."""
    if not isinstance(b, torch.Tensor):
        raise ValueError(f"bivector must be a torch.Tensor, got {type(b).__name__}")
    if b.dim() != 2:
        raise ValueError(f"bivector must be 2D (1, C(n, 2)); got shape {tuple(b.shape)}")
    if b.shape[-1] != num_basis_biv:
        raise ValueError(
            f"bivector last dim {b.shape[-1]} != C(n, 2) = {num_basis_biv} "
            f"(lex-pair order: e_01, e_02, ..., e_(n-2)(n-1))")
    if b.shape[0] != 1:
        raise ValueError(
            f"bivector first dim must be 1 (single rotor per call); got shape {tuple(b.shape)}")
    if not _same_device(b, device):
        raise ValueError(f"bivector on device {b.device}, algebra pinned to {device}")
    if b.dtype != dtype:
        raise ValueError(f"bivector dtype {b.dtype}, algebra dtype {dtype}")


def normalize_metric(n: int, metric) -> tuple:
    """metric=None -> Cl(n, 0) (reference ``extensions/ga/geom_prod.py:32-41``)."""
    if metric is None:
        return (1,) * n
    metric = tuple(int(m) for m in metric)
    if len(metric) != n:
        raise ValueError(f"metric must have {n} entries, got {len(metric)}")
    if any(m not in (-1, 0, 1) for m in metric):
        raise ValueError(f"metric entries must be in {{-1, 0, 1}}, got {metric}")
    return metric


def metric_masks(metric: tuple) -> tuple:
    """(neg_mask, null_mask) bit masks of the C ABI."""
    neg = sum(1 << k for k, m in enumerate(metric) if m == -1)
    nul = sum(1 << k for k, m in enumerate(metric) if m == 0)
    return neg, nul


def dim_to_n(dim: int) -> int:
    n = dim.bit_length() - 1
    if dim < 2 or (1 << n) != dim:
        raise ValueError(f"dim must be a power of two, got {dim}")
    return n
