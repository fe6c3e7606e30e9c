"""The measurement aids bench.py reads the kernels against: the HBM streaming-read rate, the dense
bf16 matrix-core rate, the LDS fragment-read rates, the staging rate and the prefill step in three
wave layouts, each launched through the C ABI; their rates must be physically plausible for an
MI355X (the published peaks bound them from above)."""
import sys

import pytest
import torch

from sparseattentioninfer_amd import _lib

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _time(launch, reps=3):
    launch()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        launch()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / reps


def test_ceilings_are_plausible():
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    cus = int(lib.sa_measure_cus())
    assert 1 <= cus <= 1024
    _say(f"[measure] mfma rate, {cus} CUs")
    iters = 4000
    sink = torch.empty(256 * 2 * cus, dtype=torch.float32, device="cuda")
    t = _time(lambda: _lib.check("sa_mfma_rate", lib.sa_mfma_rate(2, iters, sink.data_ptr(), sink.numel(), stream)))
    pflops = 4 * iters * 32768 * 4 * 2 * cus / t / 1e15   # 4 MFMAs per round, 4 waves per workgroup
    assert torch.isfinite(sink).all()
    assert 0.5 < pflops < 2.6, pflops        # the dense bf16 peak is 2.5 PFLOP/s at 2.4 GHz
    for tr16 in (0, 1):
        _say(f"[measure] lds rate tr16={tr16}")
        sink = torch.empty(512 * cus, dtype=torch.int32, device="cuda")
        t = _time(lambda: _lib.check("sa_lds_read_rate", lib.sa_lds_read_rate(tr16, 1000, sink.data_ptr(), sink.numel(), stream)))
        per_cu = 8 * 16384 * 1000 / t / 1e9     # bytes per ns per CU
        assert 50 < per_cu < 1000, per_cu       # at most 256 B per clock at 2.4 GHz is 614 B/ns
    _say("[measure] staging rate")
    src = torch.ones(1 << 16, dtype=torch.uint8, device="cuda")
    sink = torch.empty(512 * cus, dtype=torch.int32, device="cuda")
    t = _time(lambda: _lib.check("sa_stage_rate", lib.sa_stage_rate(src.data_ptr(), src.numel(), 2000, sink.data_ptr(),
                                                                     sink.numel(), stream)))
    per_cu = 16384 * 2000 / t / 1e9
    assert 5 < per_cu < 400, per_cu             # bytes per ns per CU
    assert (sink == 0x01010101).all()           # the tile landed in LDS
    for layout in (0, 1, 2):
        _say(f"[measure] step rate layout {layout}")
        sink = torch.empty(int(lib.sa_step_rate_threads(layout)) * cus, dtype=torch.float32, device="cuda")
        t = _time(lambda: _lib.check("sa_step_rate", lib.sa_step_rate(layout, src.data_ptr(), src.numel(), 500,
                                                                      sink.data_ptr(), sink.numel(), stream)))
        ns = t / 500 * 1e9
        assert 850 < ns < 20000, (layout, ns)   # 2,048 matrix cycles per step: over 850 ns at 2.4 GHz
    _say("[measure] stream read")
    n = 1 << 28
    buf = torch.ones(n, dtype=torch.uint8, device="cuda")
    sink = torch.empty(int(lib.sa_stream_read_workgroups()), dtype=torch.int32, device="cuda")
    t = _time(lambda: _lib.check("sa_stream_read", lib.sa_stream_read(buf.data_ptr(), n, sink.data_ptr(), stream)))
    assert 1.0 < n / t / 1e12 < 8.5          # TB/s against the 8 TB/s HBM peak
