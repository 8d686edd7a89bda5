"""The allocation-free layer backward (clf_product_bcast_bwd_noalloc) against
the workspace entry point it mirrors (clf_product_bcast_bwd), called through
the C ABI on the same inputs: gx and gw within 1e-5 normwise, on two calls in
a row with the second on a smaller batch (the shared scratch array keeps the
first call's contents, which must not leak into the second)."""
import pytest
import torch

from cliffordcuda_amd import _lib
from cliffordcuda_amd._validate import metric_masks

pytestmark = pytest.mark.gpu
TOL = 1e-5


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = float(ref.abs().max())
    return float((got - ref).abs().max()) / (den if den > 0 else 1.0)


def run_both(lib, op, side, metric, batch, seed):
    n = len(metric)
    D = 1 << n
    neg, nul = metric_masks(tuple(metric))
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, D, generator=g).cuda()
    w = torch.randn(1, D, generator=g).cuda()
    gy = torch.randn(batch, D, generator=g).cuda()
    stream = _lib.stream_of(x)
    code = _lib.OP_CODES[op]
    gx_ref = torch.empty_like(x)
    gw_ref = torch.empty(D, device="cuda")
    ws_bytes = lib.clf_product_bcast_ws_bytes(n, batch)
    ws = torch.empty(max(1, ws_bytes // 4), device="cuda")
    rc = lib.clf_product_bcast_bwd(code, side, n, neg, nul, x.data_ptr(), w.data_ptr(), gy.data_ptr(),
                                   gx_ref.data_ptr(), gw_ref.data_ptr(), batch, ws.data_ptr(), ws_bytes, stream)
    _lib.check(rc, "clf_product_bcast_bwd")
    gx = torch.full_like(x, float("nan"))
    gw = torch.full((D,), float("nan"), device="cuda")
    rc = lib.clf_product_bcast_bwd_noalloc(code, side, n, neg, nul, x.data_ptr(), w.data_ptr(), gy.data_ptr(),
                                           gx.data_ptr(), gw.data_ptr(), batch, stream)
    _lib.check(rc, "clf_product_bcast_bwd_noalloc")
    torch.cuda.synchronize()
    return (gx, gw), (gx_ref, gw_ref)


CASES = [
    ("geom", 0, (1,) * 8),                    # matrix-representation layer path (C3's)
    ("geom", 1, (1, -1) * 4),                 # same path, weight on the left
    ("wedge", 0, (1,) * 7 + (-1,)),           # MFMA GEMM path, n = 8
    ("lc", 1, (1,) * 6 + (-1, 0)),            # GEMM path with a null generator
    ("geom", 0, (1,) * 9 + (0,)),             # GEMM path at n = 10: split count capped by the array
]


@pytest.mark.parametrize("op,side,metric", CASES, ids=[f"{c[0]}-s{c[1]}-n{len(c[2])}" for c in CASES])
def test_noalloc_matches_workspace_entry_point(op, side, metric):
    lib = _lib.load()
    n = len(metric)
    first, second = (20000, 4099) if n < 10 else (12000, 1500)
    for call, batch in enumerate((first, second)):
        print(f"[case] noalloc op={op} side={side} n={n} batch={batch} call={call}", flush=True)
        (gx, gw), (gx_ref, gw_ref) = run_both(lib, op, side, metric, batch, seed=100 * call + n)
        assert rel_err(gx, gx_ref) <= TOL
        assert rel_err(gw, gw_ref) <= TOL


def test_noalloc_scratch_size_and_errors():
    lib = _lib.load()
    assert lib.clf_product_bcast_bwd_noalloc_scratch_bytes() == 32 << 20
    x = torch.zeros(4, 256, device="cuda")
    rc = lib.clf_product_bcast_bwd_noalloc(9, 0, 8, 0, 0, x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(),
                                           x.data_ptr(), 4, _lib.stream_of(x))
    assert rc == _lib.CLF_ERR_ARG
