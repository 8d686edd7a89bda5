"""The C ABI library loads on a host without a GPU, exports every symbol
include/clifford_hip.h declares, and rejects bad arguments before any HIP
call (no compute is launched here)."""
import ctypes
import os
import re

import pytest

from cliffordcuda_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            names |= set(re.findall(r"^\s*(?:const\s+)?[a-z_]+\*?\s+\*?(clf_[a-z0-9_]+)\s*\(", text, re.M))
    return names


def test_all_declared_symbols_exported():
    lib = _lib.load()
    decl = declared_symbols()
    assert "clf_product_fwd" in decl and len(decl) >= 9
    for name in decl:
        assert hasattr(lib, name), name
    assert decl == set(_lib.SIGNATURES), decl ^ set(_lib.SIGNATURES)


def test_abi_version_and_limits():
    lib = _lib.load()
    assert lib.clf_abi_version() == _lib.ABI_VERSION == 3
    assert lib.clf_product_max_n() >= 10


def test_clock_sample_rejects_bad_arguments():
    lib = _lib.load()
    assert lib.clf_clock_sample(None, 8, None) == 1
    assert "NULL" in lib.clf_last_error().decode()
    for slots in (0, -1, 4097):
        assert lib.clf_clock_sample(16, slots, None) == 1
        assert "slots" in lib.clf_last_error().decode()


def test_stream_probe_rejects_bad_arguments():
    lib = _lib.load()
    ok = 256  # a 16-byte aligned stand-in address; nothing is launched on rejection
    cases = [((0, 1, ok, ok, ok, ok, ok, 16, 1, None), "n_in"), ((4, 1, ok, ok, ok, ok, ok, 16, 1, None), "n_in"),
             ((1, 0, ok, ok, ok, ok, ok, 16, 1, None), "n_out"), ((1, 3, ok, ok, ok, ok, ok, 16, 1, None), "n_out"),
             ((1, 1, ok, ok, ok, ok, ok, 18, 1, None), "multiple of 4"),
             ((1, 1, ok, ok, ok, ok, ok, -4, 1, None), "multiple of 4"),
             ((3, 2, ok, ok, None, ok, ok, 16, 1, None), "null"), ((2, 2, ok, ok, ok, ok, None, 16, 1, None), "null"),
             ((2, 1, ok, ok + 4, ok, ok, ok, 16, 1, None), "aligned")]
    for args, msg in cases:
        assert lib.clf_stream_probe(*args) == 1, args
        assert msg in lib.clf_last_error().decode(), (args, lib.clf_last_error())
    # unused operands are not checked; zero floats launch nothing
    assert lib.clf_stream_probe(1, 1, ok, None, None, ok, None, 0, 0, None) == 0


def test_rotor_state_length_matches_python():
    """The traced-graph state length (computed in Python) equals the library's."""
    from cliffordcuda_amd.rotor import _state_len
    lib = _lib.load()
    for n in range(2, 13):
        assert lib.clf_rotor_state_floats(n) == _state_len(n), n
    assert lib.clf_rotor_state_floats(8) == 64 + 56 + 256
    assert lib.clf_rotor_state_floats(13) == -1
    assert lib.clf_rotor_cs_apply_ws_bytes(13, 4) == 0
    assert lib.clf_rotor_cs_apply_ws_bytes(12, 4) > 0


@pytest.mark.parametrize("args,code,msg", [
    ((9, 5, 0, 0, None, None, None, 4, None), 1, "unknown product op"),
    ((0, 0, 0, 0, None, None, None, 4, None), 1, "n must be in"),
    ((0, 21, 0, 0, None, None, None, 4, None), 1, "n must be in"),
    ((0, 5, 1 << 5, 0, None, None, None, 4, None), 1, "bits above n"),
    ((0, 5, 3, 2, None, None, None, 4, None), 1, "overlap"),
    ((0, 5, 0, 0, None, None, None, -1, None), 1, "batch"),
    ((5, 5, 0, 1, None, None, None, 4, None), 2, "degenerate"),
    ((0, 5, 0, 0, None, None, None, 4, None), 1, "null pointer"),
    ((0, 5, 0, 0, 16, 16, 16, 4, None), 1, "alias"),
    ((0, 5, 0, 0, 16, 32, 8, 4, None), 1, "aligned"),
])
def test_product_fwd_argument_errors(args, code, msg):
    lib = _lib.load()
    assert lib.clf_product_fwd(*args) == code
    assert msg in _lib.last_error()


def test_zero_batch_is_noop_and_clears_error():
    lib = _lib.load()
    lib.clf_product_fwd(9, 5, 0, 0, None, None, None, 4, None)
    assert _lib.last_error()
    assert lib.clf_product_fwd(0, 5, 0, 0, None, None, None, 0, None) == 0
    assert _lib.last_error() == ""
    assert lib.clf_product_bwd(0, 5, 0, 0, None, None, None, None, None, 7, None) == 0  # no grads requested


def test_graded_and_norm_errors():
    lib = _lib.load()
    assert lib.clf_graded(9, 5, 0, 0, 0, None, None, 1, None) == 1
    assert lib.clf_graded(3, 5, 0, 0, 6, None, None, 1, None) == 1
    assert "grade must be in" in _lib.last_error()
    assert lib.clf_graded(4, 5, 0, 1, 0, None, None, 1, None) == 2
    assert lib.clf_graded(4, 5, 0, 0, 0, 16, 16, 1, None) == 1
    assert lib.clf_norm_sq_fwd(5, 0, 0, None, None, 3, None) == 1
    assert lib.clf_norm_sq_bwd(0, 0, 0, None, None, None, 3, None) == 1


def test_status_mapping():
    with pytest.raises(ValueError):
        _lib.check(_lib.CLF_ERR_ARG, "x")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.CLF_ERR_HIP, "x")
    _lib.check(_lib.CLF_OK, "x")


def test_rotor_cs_argument_errors():
    """The cs entry points check n, pointers, aliasing and the workspace before
    any HIP call."""
    lib = _lib.load()
    assert lib.clf_rotor_cs_apply_fwd(13, 16, 16, 32, 4, None) == 1
    assert "n in [2, 12]" in _lib.last_error()
    assert lib.clf_rotor_cs_apply_fwd(8, None, 16, 32, 4, None) == 1
    assert lib.clf_rotor_cs_apply_fwd(8, 16, 32, 32, 4, None) == 1
    assert "alias" in _lib.last_error()
    assert lib.clf_rotor_cs_apply_fwd(8, 16, 32, 48, 0, None) == 0           # empty batch
    assert lib.clf_rotor_cs_apply_bwd(8, 16, 32, 48, None, None, 4, None, 0, None) == 0  # nothing requested
    assert lib.clf_rotor_cs_apply_bwd(8, 16, 32, 48, 64, 80, 4, None, 0, None) == 4      # no workspace
    assert "workspace" in _lib.last_error()
    assert lib.clf_rotor_cs_apply_bwd(8, 16, 32, 48, 48, None, 4, None, 0, None) == 1    # gx aliases gy
    assert lib.clf_rotor_cs_compile_bwd(8, 16, None, 32, None) == 1
    assert lib.clf_rotor_compile_fwd(1, 16, 32, None, None) == 1


def test_autograd_extension_loads_when_built():
    """The products' C++ autograd node, when built, loads on a host without a GPU
    and exports its two entries (products.py falls back to the Python Function
    only when it is absent)."""
    import os
    from cliffordcuda_amd import products
    if not os.path.exists(products._EXT_PATH):
        pytest.skip("the C++ autograd node is not built here")
    ext = products._autograd_ext()
    assert ext is not None and callable(ext.product) and callable(ext.product_fwd)
