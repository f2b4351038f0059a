"""Exhaustive device check of the fp16 conversions every bit-exact kernel
uses (src: simple-inference_amd/csrc/si_device.hpp), against the oracle's
f16_to_f32 / f32_to_f16 (qwen_one_layer.c:42-86), which are themselves pinned
against numpy's IEEE conversions and the reference build
(test_oracle_math.py, test_oracle_vs_reference.py):
  * h2f (software) on all 65,536 halves, bit for bit (NaN payloads kept);
  * h2f_fast (hardware) on every finite half, bit for bit;
  * f2h on a strided sweep of all 2^32 fp32 patterns (stride 257: every
    exponent, both signs, 16.7 M patterns) plus the full neighbourhoods of
    the rounding edges: zero, the subnormal underflow threshold (2^-25), the
    smallest normal half (2^-14), the overflow threshold (65520) and the
    infinities / NaNs."""
import numpy as np
import pytest

import si_amd  # noqa: F401  (loads torch's HIP runtime first)
from tests.gpu_helpers import dev, empty, host
from tests.probe import call as probe_call

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def test_h2f_all_halves(oracle):
    torch = _torch()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    exact, fast = empty(65536, torch.float32), empty(65536, torch.float32)
    probe_call("si_probe_h2f", si_amd.ptr(dev(h.view(np.int16))), si_amd.ptr(exact),
               si_amd.ptr(fast), 65536, None)
    want = oracle.f16_to_f32(h)
    got = host(exact)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    finite = (h & 0x7c00) != 0x7c00
    assert np.array_equal(host(fast).view(np.uint32)[finite], want.view(np.uint32)[finite])


def _sweep(oracle, start, stride, n):
    torch = _torch()
    out = empty(n, torch.int16)
    probe_call("si_probe_f2h_sweep", start, stride, n, si_amd.ptr(out), None)
    bits = (np.uint64(start) + np.arange(n, dtype=np.uint64) * np.uint64(stride)) \
        & np.uint64(0xffffffff)
    want = oracle.f32_to_f16(bits.astype(np.uint32).view(np.float32))
    got = host(out).view(np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (f"{bad.size} patterns differ, first 0x{int(bits[bad[0]]):08x}: "
                           f"got 0x{int(got[bad[0]]):04x} want 0x{int(want[bad[0]]):04x}")


def test_f2h_strided_sweep(oracle):
    _sweep(oracle, 0, 257, (1 << 32) // 257 + 1)


@pytest.mark.parametrize("center", [
    0x00000000,    # +-0 and the smallest fp32 subnormals
    0x33000000,    # 2^-25: half of the smallest half subnormal (ties to zero/one)
    0x33800000,    # 2^-24: the smallest half subnormal
    0x387fc000,    # the largest half subnormal
    0x38800000,    # 2^-14: the smallest normal half
    0x477fe000,    # 65504: the largest finite half
    0x477ff000,    # 65520: the overflow threshold
    0x7f800000,    # infinity and the NaNs above it
])
@pytest.mark.parametrize("sign", [0, 0x80000000])
def test_f2h_edge_neighbourhoods(oracle, center, sign):
    n = 1 << 17
    start = (center - n // 2) & 0x7fffffff if center >= n // 2 else 0
    _sweep(oracle, (start | sign) & 0xffffffff, 1, n)


def test_abi_f16_conversions(oracle):
    """si_f16_to_f32 / si_f32_to_f16 through the C ABI (the mirror's
    f16_to_f32 / f32_to_f16, qwen_one_layer.c:42-86): every half widened bit
    for bit, and a strided sweep of fp32 patterns plus the rounding edges
    narrowed bit for bit.  One call spans several grid-stride rounds (the
    grid is capped at 8192 workgroups of 256 threads)."""
    torch = _torch()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    wide = empty(65536, torch.float32)
    si_amd.call("si_f16_to_f32", si_amd.ptr(dev(h.view(np.int16))), si_amd.ptr(wide), 65536,
                None)
    assert np.array_equal(host(wide).view(np.uint32), oracle.f16_to_f32(h).view(np.uint32))
    stride = 1021
    bits = np.arange(0, 1 << 32, stride, dtype=np.uint64).astype(np.uint32)
    edges = [0x00000000, 0x33000000, 0x33800000, 0x387fc000, 0x38800000, 0x477fe000,
             0x477ff000, 0x7f800000]
    near = np.concatenate([(np.uint32(c) + np.arange(-2048, 2048, dtype=np.int64)
                            .astype(np.uint32)) for c in edges])
    bits = np.concatenate([bits, near, near | np.uint32(0x80000000)])
    n = bits.size
    assert n > 8192 * 256  # more than one grid-stride round
    narrow = empty(n, torch.int16)
    si_amd.call("si_f32_to_f16", si_amd.ptr(dev(bits.view(np.float32))), si_amd.ptr(narrow), n,
                None)
    got = host(narrow).view(np.uint16)
    want = oracle.f32_to_f16(bits.view(np.float32))
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (f"{bad.size} patterns differ, first 0x{int(bits[bad[0]]):08x}: "
                           f"got 0x{int(got[bad[0]]):04x} want 0x{int(want[bad[0]]):04x}")
