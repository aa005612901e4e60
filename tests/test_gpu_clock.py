"""The shader-clock trace (clock.hip, spmm_c_shader_clock_trace) on cuda:0.

One wave samples shader cycles and the 100 MHz real-time counter; the clock of
an interval is 100 MHz x delta cycles / delta ticks.  On MI355X it lies
between the lowest DPM level and the 2.4 GHz top one, also while a workload
runs on another stream.  Bad sizes are refused before any launch.
"""
import numpy as np
import pytest

from spmm_amd import SPMM_INVALID

pytestmark = pytest.mark.gpu


def test_clock_trace_alone(S):
    import torch
    assert torch.cuda.is_available()
    out = S.shader_clock_trace(20, 5.0)
    torch.cuda.synchronize()
    ser = S.shader_clock_series(out)
    print(f"shader clock alone: {[round(m) for _, m in ser]}", flush=True)
    assert len(ser) == 19
    ts = [t for t, _ in ser]
    assert all(b > a for a, b in zip(ts, ts[1:]))
    assert ts[-1] >= 19 * 5.0 - 1e-6  # samples at least 5 us apart
    assert all(100.0 < m < 3000.0 for _, m in ser)
    assert 100.0 < S.shader_clock_mhz() < 3000.0


def test_clock_trace_beside_workload(S, O):
    import torch
    from gpu_util import make_config
    A, B = make_config(S, "c3")
    dA = S.DeviceBSR(S.bsr_from_csr_host(A))
    B16 = torch.from_numpy(O.f32_to_f16(B).view(np.int16)).cuda()
    plan = S.BsrTilePlan(dA)
    C = plan.launch(B16)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        out = S.shader_clock_trace(200, 5.0)
    plan.launch_repeat(B16, C, 200)
    torch.cuda.synchronize()
    ser = S.shader_clock_series(out)
    vals = sorted(m for _, m in ser)
    print(f"shader clock beside 200 c3 launches: median {vals[len(vals) // 2]:.0f} MHz, "
          f"min {vals[0]:.0f}, max {vals[-1]:.0f}", flush=True)
    assert len(ser) == 199 and all(100.0 < m < 3000.0 for m in vals)


def test_clock_trace_refusals(S):
    import torch
    out = torch.zeros(8, dtype=torch.int64, device="cuda")
    for samples, interval in ((1, 10), (1 << 21, 10), (4, 0), (4, 200000000),
                              (1 << 20, 10000)):  # the last: over 60 s
        with pytest.raises(S.SpmmError) as e:
            S._check(S.lib().spmm_c_shader_clock_trace(out.data_ptr(), samples, interval, None))
        assert e.value.code == SPMM_INVALID
    with pytest.raises(S.SpmmError):
        S._check(S.lib().spmm_c_shader_clock_trace(None, 4, 10, None))
