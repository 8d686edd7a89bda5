"""ctypes binding of ``libclifford_hip.so`` (the C ABI in ``include/clifford_hip.h``).

The shared library is built in-tree by ``__graft_entry__.build()`` (hipcc,
``--offload-arch=gfx950``). There is deliberately no fallback: if the library
is missing, every op raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_NAME = "libclifford_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

ABI_VERSION = 3  # CLF_ABI_VERSION of include/clifford_hip.h

# status codes (include/clifford_hip.h)
CLF_OK = 0
CLF_ERR_ARG = 1
CLF_ERR_UNSUPPORTED = 2
CLF_ERR_HIP = 3
CLF_ERR_WORKSPACE = 4

OP_CODES = {"geom": 0, "wedge": 1, "inner": 2, "lc": 3, "rc": 4, "regressive": 5}
GRADED_CODES = {"reverse": 0, "involution": 1, "conjugation": 2, "projection": 3,
                "dual": 4, "dual_adj": 5}

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_u32 = ctypes.c_uint32
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t


class DeviceInfo(ctypes.Structure):
    _fields_ = [("device", ctypes.c_int), ("compute_units", ctypes.c_int),
                ("lds_bytes_per_block", ctypes.c_int), ("clock_khz", ctypes.c_int),
                ("memory_clock_khz", ctypes.c_int), ("memory_bus_width_bits", ctypes.c_int),
                ("arch_name", ctypes.c_char * 64), ("wall_clock_khz", ctypes.c_int)]


# name -> (restype, argtypes); the exact export list of include/clifford_hip.h
SIGNATURES = {
    "clf_abi_version": (_i32, []),
    "clf_options_reload": (None, []),
    "clf_last_error": (ctypes.c_char_p, []),
    "clf_device_info_get": (_i32, [_i32, ctypes.POINTER(DeviceInfo)]),
    "clf_clock_sample": (_i32, [_vp, _i32, _vp]),
    "clf_stream_probe": (_i32, [_i32, _i32, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _vp]),
    "clf_product_max_n": (_i32, []),
    "clf_product_fwd": (_i32, [_i32, _i32, _u32, _u32, _vp, _vp, _vp, _i64, _vp]),
    "clf_product_bwd": (_i32, [_i32, _i32, _u32, _u32, _vp, _vp, _vp, _vp, _vp, _i64, _vp]),
    "clf_product_bwd_ld": (_i32, [_i32, _i32, _u32, _u32, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp]),
    "clf_graded": (_i32, [_i32, _i32, _u32, _u32, _i32, _vp, _vp, _i64, _vp]),
    "clf_norm_sq_fwd": (_i32, [_i32, _u32, _u32, _vp, _vp, _i64, _vp]),
    "clf_norm_sq_bwd": (_i32, [_i32, _u32, _u32, _vp, _vp, _vp, _i64, _vp]),
    "clf_rotor_state_floats": (_i32, [_i32]),
    "clf_rotor_compile_fwd": (_i32, [_i32, _vp, _vp, _vp, _vp]),
    "clf_rotor_compile_bwd": (_i32, [_i32, _vp, _vp, _vp, _vp]),
    "clf_rotor_apply_fwd": (_i32, [_i32, _vp, _vp, _vp, _i64, _vp]),
    "clf_rotor_apply_ws_bytes": (_sz, [_i32, _i64]),
    "clf_rotor_apply_bwd": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _sz, _vp]),
    "clf_rotor_apply_bwd_ld": (_i32, [_i32, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _sz, _vp]),
    "clf_rotor_bivector_apply_ws_bytes": (_sz, [_i32, _i64]),
    "clf_rotor_bivector_apply_bwd": (_i32, [_i32, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _sz, _vp]),
    "clf_rotor_cs_apply_fwd": (_i32, [_i32, _vp, _vp, _vp, _i64, _vp]),
    "clf_rotor_cs_apply_ws_bytes": (_sz, [_i32, _i64]),
    "clf_rotor_cs_apply_bwd": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _sz, _vp]),
    "clf_rotor_cs_apply_bwd_ld": (_i32, [_i32, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _sz, _vp]),
    "clf_rotor_cs_compile_bwd": (_i32, [_i32, _vp, _vp, _vp, _vp]),
    "clf_inverse_rep_supported": (_i32, [_i32, _u32, _u32]),
    "clf_inverse_rep": (_i32, [_i32, _u32, _u32, _vp, _vp, _vp, _i64, _vp]),
    "clf_inverse_versor": (_i32, [_i32, _vp, _vp, _vp, _vp, ctypes.c_float, _i64, _vp]),
    "clf_product_bcast_ws_bytes": (_sz, [_i32, _i64]),
    "clf_product_bcast_fwd": (_i32, [_i32, _i32, _i32, _u32, _u32, _vp, _vp, _vp, _i64, _vp, _sz, _vp]),
    "clf_product_bcast_bwd": (_i32, [_i32, _i32, _i32, _u32, _u32, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _sz, _vp]),
    "clf_product_bcast_bwd_ld": (
        _i32, [_i32, _i32, _i32, _u32, _u32, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _sz, _vp]),
    "clf_product_bcast_bwd_noalloc_scratch_bytes": (_sz, []),
    "clf_product_bcast_bwd_noalloc": (_i32, [_i32, _i32, _i32, _u32, _u32, _vp, _vp, _vp, _vp, _vp, _i64, _vp]),
}

_lock = threading.Lock()
_lib = None


def load():
    """Load (once) and return the native library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"cliffordcuda_amd: native library {LIB_PATH} is not built; run "
                    "`python -c 'import __graft_entry__ as g; g.build()'` from the repo root")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.clf_abi_version() != ABI_VERSION:
                raise RuntimeError(
                    f"cliffordcuda_amd: {LIB_PATH} has ABI version {lib.clf_abi_version()}, this package needs "
                    f"{ABI_VERSION}; rebuild it")
            _lib = lib
    return _lib


def last_error() -> str:
    return load().clf_last_error().decode("utf-8", "replace")


def check(rc: int, what: str):
    """Map a CLF status to the reference's exception types (ValueError for
    argument / unsupported errors, RuntimeError for HIP failures)."""
    if rc == CLF_OK:
        return
    msg = last_error() or f"{what} failed with status {rc}"
    if rc in (CLF_ERR_ARG, CLF_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(f"{what}: {msg}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def grad_rows(g: torch.Tensor, dim: int):
    """(tensor, row stride in floats) for an upstream gradient of shape
    (batch, dim). A gradient whose batch stride is 0 (autograd's expansion of
    the gradient of a sum) is handed over as its one row with stride 0, so the
    kernels read that row for every batch row instead of a materialised copy;
    any other layout is made contiguous (stride dim)."""
    if g.dim() == 2 and g.shape[0] > 1 and g.stride(0) == 0:
        row = g[0]
        if row.stride(0) != 1 or row.data_ptr() % 16:
            row = row.clone(memory_format=torch.contiguous_format)
        return row, 0
    return g.contiguous(), dim


def reload_options() -> None:
    """Re-read the CLF_* path switches (the library reads them once per
    process otherwise)."""
    load().clf_options_reload()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
# torch.cuda.current_device() less its lazy-init check (a tensor on the GPU exists, so
# the runtime is up)
_current_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def stream_of(t: torch.Tensor) -> int:
    """The current HIP stream of ``t``'s device (torch's ``cuda`` namespace is
    HIP on ROCm), as the raw handle the C ABI takes; the direct query skips
    building a Stream object per call (about 1.7 us of host time each)."""
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


class _CurrentDevice:
    __slots__ = ()

    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_CURRENT = _CurrentDevice()


def on_device(t: torch.Tensor):
    """Context making ``t``'s device current for a library call (the library
    keeps its tables per device); a no-op when it already is."""
    idx = t.get_device()
    if idx == _current_device():
        return _CURRENT
    return torch.cuda.device(idx)


def device_info(device: int = 0) -> DeviceInfo:
    info = DeviceInfo()
    check(load().clf_device_info_get(device, ctypes.byref(info)), "clf_device_info_get")
    return info
