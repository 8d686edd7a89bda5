"""clf_stream_probe, the roofline report's streaming calibration: every
(inputs, outputs, nontemporal) combination computes out0 = the sum of its
inputs and out1 = in0 - out0, bit for bit against torch, over a length that
ends inside a workgroup's pass, and leaves the floats after its range alone."""
import pytest
import torch

from cliffordcuda_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nt", [0, 1])
@pytest.mark.parametrize("n_out", [1, 2])
@pytest.mark.parametrize("n_in", [1, 2, 3])
def test_stream_probe_values(n_in, n_out, nt):
    lib = _lib.load()
    n = 4 * (1024 * 3 + 517)
    g = torch.Generator().manual_seed(n_in * 10 + n_out * 2 + nt)
    ins = [torch.randn(n + 64, generator=g).cuda() for _ in range(3)]
    outs = [torch.full((n + 64,), 7.0, device="cuda") for _ in range(2)]
    s = torch.cuda.current_stream().cuda_stream
    print(f"[case] stream probe n_in={n_in} n_out={n_out} nt={nt}", flush=True)
    _lib.check(lib.clf_stream_probe(n_in, n_out, ins[0].data_ptr(), ins[1].data_ptr(), ins[2].data_ptr(),
                                    outs[0].data_ptr(), outs[1].data_ptr(), n, nt, s), "clf_stream_probe")
    torch.cuda.synchronize()
    ref = ins[0][:n].clone()
    for k in range(1, n_in):
        ref = ref + ins[k][:n]
    assert torch.equal(outs[0][:n], ref)
    assert torch.all(outs[0][n:] == 7.0)
    if n_out == 2:
        assert torch.equal(outs[1][:n], ins[0][:n] - ref)
        assert torch.all(outs[1][n:] == 7.0)
    else:
        assert torch.all(outs[1] == 7.0)
