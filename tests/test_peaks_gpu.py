"""The device-ceiling probes behind the benchmark's roofline context: they run, report the device, and never
write their sink (the guarded store only keeps the work live)."""
import ctypes

import pytest
import torch

from scratchtape_amd import _lib

pytestmark = pytest.mark.gpu


def test_device_info_reports_the_gpu():
    vals = [ctypes.c_int32() for _ in range(4)]
    _lib.call("st_device_info", *[ctypes.byref(v) for v in vals])
    cus, clk, mclk, bus = (v.value for v in vals)
    assert cus == torch.cuda.get_device_properties(0).multi_processor_count
    assert clk > 0 and mclk > 0 and bus > 0


@pytest.mark.parametrize("kind", [0, 1, 2, 3, 4])
def test_mfma_probe_runs_and_leaves_the_sink(kind):
    sink = torch.zeros(64, device="cuda")
    s = torch.cuda.current_stream()
    _lib.call("st_peak_mfma", kind, 50, 64, sink.data_ptr(), s.cuda_stream)
    torch.cuda.synchronize()
    assert torch.count_nonzero(sink).item() == 0


def test_read_probe_runs_and_leaves_the_sink():
    buf = torch.randn(1 << 20, device="cuda")
    sink = torch.zeros(96, device="cuda")
    s = torch.cuda.current_stream()
    for nbytes in (buf.numel() * 4, 4096 + 16, 16):
        _lib.call("st_peak_read", buf.data_ptr(), nbytes, 96, sink.data_ptr(), s.cuda_stream)
    torch.cuda.synchronize()
    assert torch.count_nonzero(sink).item() == 0


def test_lane_exchanges_match_lane_xor_on_this_device():
    """The DPP / v_permlane exchanges, the DPP wave scan and the readlane broadcast that the probe, scan,
    LayerNorm and attention kernels use in place of ds_bpermute give exactly lane ^ J's value, the running sum
    and lane 37's value."""
    out = torch.zeros(10 * 64, dtype=torch.int32, device="cuda")
    _lib.call("st_lane_selftest", out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    got = out.view(10, 64).cpu().numpy().astype("int64")
    lane = list(range(64))
    for r, j in enumerate((1, 2, 4, 8, 15, 16, 32, 63)):
        assert got[r].tolist() == [1000 + 7 * (l ^ j) for l in lane], j
    run, acc = [], 0
    for l in lane:
        acc += 3 * l + 1 + l % 5
        run.append(acc)
    assert got[8].tolist() == run
    assert got[9].tolist() == [1000 + 7 * 37] * 64
