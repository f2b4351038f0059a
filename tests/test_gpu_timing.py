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


@pytest.mark.parametrize("nbytes,wgs,depth", [(16, 1, 4), (4096 * 16 + 48, 7, 8),
                                              (9 << 20, 2048, 16), (9 << 20, 100, 8)])
def test_stream_read_checksum(nbytes, wgs, depth):
    """The streaming-read measurement kernel reads every byte once: the XOR
    of its per-workgroup words equals the XOR of the buffer's 32-bit words
    (any grid, depth and tail), and it refuses unaligned sizes."""
    import torch
    rng = np.random.default_rng(nbytes)
    words = rng.integers(0, 1 << 32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    buf = dev(words.view(np.int32))
    sink = dev(np.zeros(wgs, np.int32))  # slices past the buffer write nothing
    si_amd.call("si_stream_read", si_amd.ptr(buf), nbytes, si_amd.ptr(sink), wgs, depth, None)
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(words)
    with pytest.raises(si_amd.SiError):
        si_amd.call("si_stream_read", si_amd.ptr(buf), nbytes - 4 if nbytes > 16 else 8,
                    si_amd.ptr(sink), wgs, depth, None)
