"""clf_clock_sample: XCD indices, hardware ids and clock counters that give a
plausible engine clock over a stretch of GPU work (the roofline report's
clock), per compute unit seen in both samples."""
import pytest
import torch

from cliffordcuda_amd import _lib

pytestmark = pytest.mark.gpu


def test_clock_sample_gives_a_plausible_engine_clock():
    lib = _lib.load()
    info = _lib.device_info(0)
    assert info.wall_clock_khz > 0 and info.compute_units > 0
    slots = 4096
    buf = torch.zeros(2, 3 * slots, dtype=torch.int64, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    # keep the GPU busy between the samples (an idle GPU lowers its clock, and
    # the first matrix product of a process spends a while loading its library)
    m = torch.randn(4096, 4096, device="cuda")
    m = torch.mm(m, m) * 1e-2
    torch.cuda.synchronize()
    _lib.check(lib.clf_clock_sample(buf[0].data_ptr(), slots, s), "clf_clock_sample")
    for _ in range(8):
        m = torch.mm(m, m) * 1e-2
    _lib.check(lib.clf_clock_sample(buf[1].data_ptr(), slots, s), "clf_clock_sample")
    torch.cuda.synchronize()
    h = buf.cpu().view(2, slots, 3).tolist()
    first = [{}, {}]
    for k in range(2):
        for loc, cyc, rt in h[k]:
            assert 0 <= (loc & 15) < 16
            if loc not in first[k] or cyc < first[k][loc][0]:
                first[k][loc] = (cyc, rt)
    common = set(first[0]) & set(first[1])
    assert len(common) >= info.compute_units // 2
    ghz = []
    for loc in common:
        (c0, r0), (c1, r1) = first[0][loc], first[1][loc]
        assert r1 > r0
        ghz.append((c1 - c0) / ((r1 - r0) / (info.wall_clock_khz * 1e3)) / 1e9)
    ghz.sort()
    print(f"[clock] {len(common)} compute units, median {ghz[len(ghz) // 2]:.3f} GHz, "
          f"range {ghz[0]:.3f} .. {ghz[-1]:.3f}", flush=True)
    assert 0.5 < ghz[len(ghz) // 2] < 4.0
