"""The device clock stamp (orth_hip_clock_stamp) that bench.py brackets its
timed launches with: every workgroup writes a clock value and an XCD id,
stamps in stream order increase, and the interval across known GPU work
matches the HIP events around the same work."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def stamp(buf, stream):
    from libortho_amd import _lib
    _lib.check(_lib.lib().orth_hip_clock_stamp(ctypes.c_void_p(buf.data_ptr()),
                                               ctypes.c_void_p(stream.cuda_stream)))


def test_clock_stamp_layout_and_order(gpu):
    s = torch.cuda.current_stream()
    buf = torch.zeros(2, 16, dtype=torch.int64, device=gpu)
    stamp(buf[0], s)
    a = torch.randn(2048, 2048, device=gpu)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        a = a @ a
        a = a / a.abs().max()
    e1.record()
    stamp(buf[1], s)
    torch.cuda.synchronize()
    h = buf.cpu()
    xcd0 = {int(h[0, 2 * i + 1]): int(h[0, 2 * i]) for i in range(8)}
    xcd1 = {int(h[1, 2 * i + 1]): int(h[1, 2 * i]) for i in range(8)}
    assert all(0 <= k < 16 for k in list(xcd0) + list(xcd1))
    common = [k for k in xcd0 if k in xcd1]
    assert common, "the two stamps ran on no common XCD"
    for k in common:
        assert xcd1[k] > xcd0[k]
    from bench import _stamp_interval_ms
    ms = _stamp_interval_ms(h[0], h[1])
    ev = e0.elapsed_time(e1)
    # the stamps also cover the two launch gaps around the events' span
    assert ev * 0.9 - 0.01 <= ms <= ev * 1.1 + 0.05, (ms, ev)


def test_clock_stamp_rejects_null_and_misaligned(gpu):
    from libortho_amd import _lib
    L = _lib.lib()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert L.orth_hip_clock_stamp(None, s) != 0
    buf = torch.zeros(20, dtype=torch.int64, device=gpu)
    assert L.orth_hip_clock_stamp(ctypes.c_void_p(buf.data_ptr() + 4), s) != 0
