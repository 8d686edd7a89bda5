"""clf_clock_sample: XCD indices and clock counters that give a plausible
engine clock over a stretch of GPU work (the roofline report's clock)."""
import pytest
import torch

from cliffordcuda_amd import _lib

pytestmark = pytest.mark.gpu


def test_clock_sample_gives_a_plausible_engine_clock():
    lib = _lib.load()
    info = _lib.device_info(0)
    assert info.wall_clock_khz > 0 and info.compute_units > 0
    slots = 64
    buf = torch.zeros(2, 3 * slots, dtype=torch.int64, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    x = torch.randn(1 << 24, device="cuda")
    _lib.check(lib.clf_clock_sample(buf[0].data_ptr(), slots, s), "clf_clock_sample")
    for _ in range(50):
        x = x * 1.0001 + 0.5
    _lib.check(lib.clf_clock_sample(buf[1].data_ptr(), slots, s), "clf_clock_sample")
    torch.cuda.synchronize()
    h = buf.cpu().view(2, slots, 3)
    assert int(h[:, :, 0].min()) >= 0 and int(h[:, :, 0].max()) < 16
    xccs = set(h[0, :, 0].tolist())
    assert xccs == set(h[1, :, 0].tolist())
    for xcc in xccs:
        pre = h[0][h[0, :, 0] == xcc]
        post = h[1][h[1, :, 0] == xcc]
        dc = int(post[:, 1].min()) - int(pre[:, 1].min())
        dr = int(post[:, 2].min()) - int(pre[:, 2].min())
        assert dc > 0 and dr > 0
        ghz = dc / (dr / (info.wall_clock_khz * 1e3)) / 1e9
        assert 0.3 < ghz < 4.0, (xcc, ghz)
