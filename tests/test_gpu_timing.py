"""Per-dispatch kernel timing (si_kernel_timing_*): the launches that match
the filter are timed, in launch order, with the kernel's name; launches
under stream capture and launches of other kernels are not; the durations
are positive and bounded by the wall time around them."""
import ctypes
import time

import numpy as np
import pytest

import si_amd
from tests.gpu_helpers import dev, empty

pytestmark = pytest.mark.gpu


def _quantize(x, rows, k, qs, d, s, stream=None):
    si_amd.call("si_quantize_q8_rows", si_amd.ptr(x), rows, k, si_amd.ptr(qs), si_amd.ptr(d),
                si_amd.ptr(s), si_amd.stream_handle(stream))


def test_kernel_timing_names_order_and_filter():
    import torch
    rows, k = 64, 4096
    x = dev(np.random.default_rng(5).standard_normal(rows * k).astype(np.float32))
    qs = empty(rows * k, torch.int8)
    d = empty(rows * k // 32, torch.int16)
    s = empty(rows * k // 32, torch.int16)
    out = empty(k, torch.float32)
    torch.cuda.synchronize()

    def work():
        for _ in range(5):
            _quantize(x, rows, k, qs, d, s)
            si_amd.call("si_f16_to_f32", si_amd.ptr(qs), si_amd.ptr(out), k,
                        si_amd.stream_handle(None))

    t0 = time.perf_counter()
    got = si_amd.kernel_times_ms("k_quantize_q8_rows", work)
    wall_ms = (time.perf_counter() - t0) * 1e3
    assert [n for n, _ in got] == ["k_quantize_q8_rows"] * 5
    assert all(0 < ms < wall_ms for _, ms in got)
    # '|'-separated alternatives, launch order kept
    both = si_amd.kernel_times_ms("k_quantize_q8_rows|k_f16_to_f32", work)
    assert [n for n, _ in both] == ["k_quantize_q8_rows", "k_f16_to_f32"] * 5
    # capacity bounds the count
    few = si_amd.kernel_times_ms("k_", work, capacity=3)
    assert len(few) == 3
    # no timing is left on: a start after a stop succeeds, a second start fails
    si_amd.call("si_kernel_timing_start", b"k_", 4)
    with pytest.raises(si_amd.SiError):
        si_amd.call("si_kernel_timing_start", b"k_", 4)
    n = np.zeros(1, np.int32)
    ms = np.zeros(4, np.float32)
    si_amd.call("si_kernel_timing_stop", si_amd.ptr(ms), 4,
                n.ctypes.data_as(ctypes.POINTER(ctypes.c_int)))
    assert n[0] == 0


def test_kernel_timing_skips_captured_launches():
    import torch
    rows, k = 8, 1024
    x = dev(np.ones(rows * k, np.float32))
    qs = empty(rows * k, torch.int8)
    d = empty(rows * k // 32, torch.int16)
    s = empty(rows * k // 32, torch.int16)
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()

    def capture_and_replay():
        with torch.cuda.graph(g, stream=stream):
            _quantize(x, rows, k, qs, d, s, torch.cuda.current_stream())
        g.replay()
        torch.cuda.synchronize()

    got = si_amd.kernel_times_ms("k_quantize_q8_rows", capture_and_replay)
    assert got == []
    assert np.array_equal(qs.cpu().numpy(), np.full(rows * k, 127, np.int8))
