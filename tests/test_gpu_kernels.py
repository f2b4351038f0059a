"""GPU parity of each hot-path kernel against the oracle, through the C ABI.

Bar: bit-exact for Q8_0 quantization (on identical fp32 input), Q4_0 repack
and per-block int32 dots, and for the single-range mat-vec (the reference's
own summation order); fp32 within 1e-3 (attention 2e-3) otherwise."""
import ctypes
import os

import numpy as np
import pytest

import si_amd
from oracle.oracle_py import Q8_DTYPE, make_shape as or_shape
from tests.gpu_helpers import (aos_to_planar, close, dequant_q4, dequant_q8, dev, empty, host,
                               kv_history, q4, q8_tiled, zeros)

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_golden.npz")


def _torch():
    import torch
    return torch


def _q8_inputs(case, n=32 * 96):
    rng = np.random.default_rng(11)
    if case == "normal":
        return rng.standard_normal(n).astype(np.float32)
    if case == "tiny":
        return (rng.standard_normal(n) * 10.0 ** rng.integers(-44, -3, n)).astype(np.float32)
    if case == "ties":
        x = (rng.integers(-254, 255, n) / 2.0).astype(np.float32)
        x[::32] = 127.0
        return x
    if case == "zeros":
        x = np.zeros(n, np.float32)
        x[64:96] = rng.standard_normal(32)
        return x
    if case == "huge":
        x = (rng.standard_normal(n) * 1e6).astype(np.float32)
        x[:32] *= np.float32(1e30)
        return x
    if case == "nonfinite":
        x = rng.standard_normal(n).astype(np.float32)
        x[5], x[40], x[100] = np.nan, np.inf, -np.inf
        x[128:160] = np.nan
        return x
    return (rng.standard_normal(n) * np.repeat(10.0 ** rng.uniform(-6, 6, n // 32), 32)
            ).astype(np.float32)


@pytest.mark.parametrize("case", ["normal", "tiny", "ties", "zeros", "huge", "mixed",
                                  "nonfinite"])
def test_quantize_q8_aos_bit_exact(oracle, case):
    x = _q8_inputs(case)
    want = oracle.quantize_q8(x)
    out = empty(x.size // 32 * 34, _torch().uint8)
    si_amd.call("si_quantize_q8", si_amd.ptr(dev(x)), si_amd.ptr(out), x.size, None)
    got = host(out).view(Q8_DTYPE)
    assert got.tobytes() == want.tobytes()


def test_quantize_q8_golden_fixture():
    g = np.load(GOLDEN, allow_pickle=False)
    torch = _torch()
    for x, want in zip(g["q8_in"], g["q8_out"]):
        out = empty(x.size // 32 * 34, torch.uint8)
        si_amd.call("si_quantize_q8", si_amd.ptr(dev(x)), si_amd.ptr(out), x.size, None)
        assert host(out).tobytes() == want.tobytes()


def test_quantize_q8_rows_planar(oracle):
    torch = _torch()
    rows, k = 7, 4864
    x = (np.random.default_rng(3).standard_normal((rows, k)) * 3).astype(np.float32)
    qs, d, s = empty(rows * k, torch.int8), empty(rows * k // 32, torch.int16), \
        empty(rows * k // 32, torch.int16)
    si_amd.call("si_quantize_q8_rows", si_amd.ptr(dev(x)), rows, k, si_amd.ptr(qs),
                si_amd.ptr(d), si_amd.ptr(s), None)
    want = oracle.quantize_q8(x)
    wq, wd, ws = aos_to_planar(want)
    assert np.array_equal(host(qs), wq)
    assert np.array_equal(host(d).view(np.uint16), wd)
    assert np.array_equal(host(s), ws)


@pytest.mark.parametrize("n,gain", [(896, True), (1536, False), (3584, True)])
def test_rmsnorm_q8(oracle, n, gain):
    torch = _torch()
    rows = 256
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((rows, n)) * rng.uniform(0.01, 50, (rows, 1))).astype(np.float32)
    w = rng.normal(1, 0.1, n).astype(np.float32) if gain else None
    normed = empty(rows * n, torch.float32)
    qs, d, s = empty(rows * n, torch.int8), empty(rows * n // 32, torch.int16), \
        empty(rows * n // 32, torch.int16)
    si_amd.call("si_rmsnorm_q8", si_amd.ptr(dev(x)), si_amd.ptr(None if w is None else dev(w)),
                rows, n, 1e-6, si_amd.ptr(normed), si_amd.ptr(qs), si_amd.ptr(d),
                si_amd.ptr(s), None)
    got = host(normed).reshape(rows, n)
    for r in range(rows):
        want = oracle.rmsnorm(x[r], w)
        # bit-exact: the correctly rounded sqrtf and division of the
        # reference (a 1-ulp hardware sqrt moved ~5 % of the rows)
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), f"rmsnorm row {r}"
    # the quantizer is bit-exact on the device's own normed values
    wq, wd, ws = aos_to_planar(oracle.quantize_q8(got))
    assert np.array_equal(host(qs), wq) and np.array_equal(host(d).view(np.uint16), wd)
    assert np.array_equal(host(s), ws)


def test_rmsnorm_bit_exact_on_golden():
    g = np.load(GOLDEN, allow_pickle=False)
    torch = _torch()
    n = g["rms_in"].size
    normed = empty(n, torch.float32)
    qs, d = empty(n, torch.int8), empty(n // 32, torch.int16)
    si_amd.call("si_rmsnorm_q8", si_amd.ptr(dev(g["rms_in"])), si_amd.ptr(dev(g["rms_w"])), 1,
                n, 1e-6, si_amd.ptr(normed), si_amd.ptr(qs), si_amd.ptr(d), None, None)
    assert np.array_equal(host(normed).view(np.uint32), g["rms_out"].view(np.uint32))


def test_residual_rmsnorm_q8(oracle):
    torch = _torch()
    rows, n = 3, 896
    rng = np.random.default_rng(9)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    y = rng.standard_normal((rows, n)).astype(np.float32)
    w = rng.normal(1, 0.1, n).astype(np.float32)
    h, normed = empty(rows * n, torch.float32), empty(rows * n, torch.float32)
    qs, d = empty(rows * n, torch.int8), empty(rows * n // 32, torch.int16)
    si_amd.call("si_residual_rmsnorm_q8", si_amd.ptr(dev(x)), si_amd.ptr(dev(y)),
                si_amd.ptr(dev(w)), rows, n, 1e-6, si_amd.ptr(h), si_amd.ptr(normed),
                si_amd.ptr(qs), si_amd.ptr(d), None, None)
    assert np.array_equal(host(h).reshape(rows, n), x + y)
    got = host(normed).reshape(rows, n)
    for r in range(rows):
        want = oracle.rmsnorm(x[r] + y[r], w)
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), f"post-norm row {r}"


def test_swiglu_q8(oracle):
    torch = _torch()
    rows, f = 4, 4864
    rng = np.random.default_rng(1)
    gu = (rng.standard_normal((rows, 2 * f)) * 3).astype(np.float32)
    act = empty(rows * f, torch.float32)
    qs, d, s = empty(rows * f, torch.int8), empty(rows * f // 32, torch.int16), \
        empty(rows * f // 32, torch.int16)
    si_amd.call("si_swiglu_q8", si_amd.ptr(dev(gu)), rows, f, si_amd.ptr(act), si_amd.ptr(qs),
                si_amd.ptr(d), si_amd.ptr(s), None)
    got = host(act).reshape(rows, f)
    for r in range(rows):
        close(got[r], oracle.swiglu(gu[r, :f], gu[r, f:]), 1e-5, "swiglu")
    wq, wd, ws = aos_to_planar(oracle.quantize_q8(got))
    assert np.array_equal(host(qs), wq) and np.array_equal(host(d).view(np.uint16), wd)


def _upload_q4(w_rowmajor, n, k, tile=None):
    """Repack row-major Q4_0 on the device; returns (qs, d, tile)."""
    torch = _torch()
    L = si_amd.lib()
    tile = tile or L.si_q4_tile(n, k)
    qs = empty(n * k // 2, torch.uint8)
    d = zeros(L.si_q4_scale_count(n, k, tile), torch.int16)
    si_amd.call("si_q4_repack", si_amd.ptr(dev(w_rowmajor)), n, k, tile, si_amd.ptr(qs),
                si_amd.ptr(d), None)
    return qs, d, tile


@pytest.mark.parametrize("tile", [8, 16, 32, 64])
def test_q4_repack_round_trip(oracle, tile):
    torch = _torch()
    rng = np.random.default_rng(2)
    n, k = 300, 1024  # 300 rows: the last scale tile is partial for every tile size
    w = q4(oracle, rng, n, k)
    qs, d, _ = _upload_q4(w, n, k, tile)
    back = empty(w.size, torch.uint8)
    si_amd.call("si_q4_unpack", si_amd.ptr(qs), si_amd.ptr(d), n, k, tile, si_amd.ptr(back),
                None)
    assert np.array_equal(host(back), w.reshape(-1))
    # the repacked layout: block-major nibbles, tile-major scales
    nb = k // 32
    hq = host(qs).reshape(nb, n, 16)
    blocks = w.reshape(n, nb, 18)
    assert np.array_equal(hq, blocks[:, :, 2:].transpose(1, 0, 2))
    scales = blocks[:, :, :2].copy().view(np.uint16)[..., 0]  # [n][nb]
    npad = -(-n // tile) * tile
    padded = np.zeros((npad, nb), np.uint16)
    padded[:n] = scales
    want = padded.reshape(npad // tile, tile, nb).transpose(0, 2, 1).reshape(-1)
    assert np.array_equal(host(d).view(np.uint16), want)


def _q8_dev(oracle, x):
    xq = oracle.quantize_q8(x)
    qs, d, s = aos_to_planar(xq)
    return xq, dev(qs), dev(d.view(np.int16)), dev(s)


@pytest.mark.parametrize("n,k", [(1152, 896), (64, 32), (200, 4864)])
def test_block_dots_bit_exact(oracle, n, k):
    torch = _torch()
    rng = np.random.default_rng(n + k)
    w = rng.integers(0, 256, (n, k // 32 * 18), dtype=np.uint8)
    w.reshape(n, k // 32, 18)[:, :, 1] &= 0x3b  # keep scales finite
    x = (rng.standard_normal(k) * 2).astype(np.float32)
    x[:32] = 1000.0  # q = +127 block
    xq, xqs, xd, xs = _q8_dev(oracle, x)
    wqs, wd, tile = _upload_q4(w, n, k)
    dots = empty(n * (k // 32), torch.int32)
    si_amd.call("si_q4q8_block_dots", si_amd.ptr(wqs), si_amd.ptr(wd), n, k, si_amd.ptr(xqs),
                si_amd.ptr(xs), si_amd.ptr(dots), None)
    assert np.array_equal(host(dots).reshape(n, k // 32), oracle.block_dots(w, xq, k, n))


@pytest.mark.parametrize("n,k,bias", [(1152, 896, True), (896, 896, False), (9728, 896, False),
                                      (896, 4864, False), (4608, 3584, True),
                                      (3584, 18944, False), (77, 96, True)])
def test_matvec_exact_single_range(oracle, n, k, bias):
    """One K range per row: the reference's block order and roundings."""
    torch = _torch()
    rng = np.random.default_rng(n * 7 + k)
    w = q4(oracle, rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    b = rng.normal(0, 0.02, n).astype(np.float32) if bias else None
    xq, xqs, xd, xs = _q8_dev(oracle, x)
    wqs, wd, tile = _upload_q4(w, n, k)
    out = empty(n, torch.float32)
    si_amd.call("si_matvec_q4q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, n, k, si_amd.ptr(xqs),
                si_amd.ptr(xd), si_amd.ptr(xs), si_amd.ptr(None if b is None else dev(b)), None,
                si_amd.ptr(out), si_amd.SI_GEMM_EXACT, None)
    want = oracle.matvec(w, xq, k, n, b)
    assert np.array_equal(host(out).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n,k,tile", [(1152, 896, 8), (896, 4864, 8), (3584, 18944, 8),
                                      (37888, 3584, 32), (4608, 3584, 16), (9728, 896, 64),
                                      (96, 64, 8), (200, 96, 64), (77, 160, 16)])
def test_matvec_parallel_k(oracle, n, k, tile):
    """K spread over the workgroup (every row-count variant): fp32 rounding of
    the reference, identical results on repeated calls (fixed order)."""
    torch = _torch()
    rng = np.random.default_rng(n + k)
    w = q4(oracle, rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    b = rng.normal(0, 0.02, n).astype(np.float32)
    res = rng.standard_normal(n).astype(np.float32)
    xq, xqs, xd, xs = _q8_dev(oracle, x)
    wqs, wd, tile = _upload_q4(w, n, k, tile)
    want = res + oracle.matvec(w, xq, k, n, b)
    first = None
    for rep in range(2):
        out = empty(n, torch.float32)
        si_amd.call("si_matvec_q4q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, n, k, si_amd.ptr(xqs),
                    si_amd.ptr(xd), si_amd.ptr(xs), si_amd.ptr(dev(b)), si_amd.ptr(dev(res)),
                    si_amd.ptr(out), 0, None)
        got = host(out)
        close(got, want, 1e-5, f"matvec call {rep}")
        if first is None:
            first = got
        else:
            assert np.array_equal(first.view(np.uint32), got.view(np.uint32)), "not deterministic"


@pytest.mark.parametrize("m,n,k", [(1, 64, 64), (5, 200, 96), (64, 1152, 896),
                                   (130, 896, 4864), (512, 384, 896)])
def test_gemm_matches_oracle_rows(oracle, m, n, k):
    torch = _torch()
    rng = np.random.default_rng(m * 31 + n)
    w = q4(oracle, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.normal(0, 0.02, n).astype(np.float32)
    xq = oracle.quantize_q8(x)
    qs, d, _ = aos_to_planar(xq)
    wqs, wd, tile = _upload_q4(w, n, k)
    out = empty(m * n, torch.float32)
    si_amd.call("si_gemm_q4q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, n, k, si_amd.ptr(dev(qs)),
                si_amd.ptr(dev(d.view(np.int16))), m, si_amd.ptr(dev(b)), None,
                si_amd.ptr(out), n, 0, None, 0, None)
    got = host(out).reshape(m, n)
    nb = k // 32
    for r in sorted({0, m // 2, m - 1}):
        want = oracle.matvec(w, xq[r * nb:(r + 1) * nb], k, n, b)
        close(got[r], want, 1e-5, f"gemm row {r}")


@pytest.mark.parametrize("m,n,k", [(512, 1152, 896), (64, 4608, 3584), (130, 896, 4864),
                                   (100, 9728, 896), (64, 3584, 18944), (2048, 384, 896),
                                   (130, 200, 96), (1, 4608, 3584), (200, 1152, 896),
                                   (384, 3584, 3584)])
@pytest.mark.parametrize("split", [False, True])
def test_gemm_every_row_vs_float64(oracle, m, n, k, split):
    """Every output row of the layer-shaped GEMMs against the float64 product
    of the dequantized operands (the value the fp32 path approximates), in
    one pass over K and with K split over workgroups (twice: the split sums
    are added in a fixed order, so both calls give the same bits)."""
    torch = _torch()
    rng = np.random.default_rng(m + n + k)
    w = q4(oracle, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    xq = oracle.quantize_q8(x)
    qs, d, _ = aos_to_planar(xq)
    wqs, wd, tile = _upload_q4(w, n, k)
    wsb = si_amd.lib().si_gemm_workspace(m, n, k) if split else 0
    ws = empty(max(wsb, 4), torch.uint8) if split else None
    want = dequant_q8(xq, m, k) @ dequant_q4(w, n, k).T
    rms = np.sqrt(np.mean(want ** 2))
    prev = None
    for rep in range(2 if split else 1):
        out = empty(m * n, torch.float32)
        si_amd.call("si_gemm_q4q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, n, k,
                    si_amd.ptr(dev(qs)), si_amd.ptr(dev(d.view(np.int16))), m, None, None,
                    si_amd.ptr(out), n, 0, si_amd.ptr(ws), wsb, None)
        got = host(out).reshape(m, n)
        err = np.abs(got - want).max(axis=1) / rms
        bad = np.nonzero(err > 1e-5)[0]
        assert bad.size == 0, f"rows off (row mod 64 -> {sorted(set((bad % 64).tolist()))[:16]}), " \
                              f"first {bad[:8].tolist()}, worst {err.max():.3g}"
        if prev is not None:
            assert np.array_equal(prev.view(np.uint32), got.view(np.uint32)), "not deterministic"
        prev = got


def test_gemm_residual(oracle):
    torch = _torch()
    m, n, k = 70, 256, 512
    rng = np.random.default_rng(5)
    w = q4(oracle, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    res = rng.standard_normal((m, n)).astype(np.float32)
    xq = oracle.quantize_q8(x)
    qs, d, _ = aos_to_planar(xq)
    wqs, wd, tile = _upload_q4(w, n, k)
    out = empty(m * n, torch.float32)
    si_amd.call("si_gemm_q4q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, n, k, si_amd.ptr(dev(qs)),
                si_amd.ptr(dev(d.view(np.int16))), m, None, si_amd.ptr(dev(res)),
                si_amd.ptr(out), n, 0, None, 0, None)
    got = host(out).reshape(m, n)
    nb = k // 32
    for r in (0, 69):
        close(got[r], res[r] + oracle.matvec(w, xq[r * nb:(r + 1) * nb], k, n), 1e-5, "res")


@pytest.mark.parametrize("m,n,k,ldo", [
    (64, 256, 512, 256),     # batched-decode GEMM, one column tile per workgroup
    (33, 9000, 256, 9008),   # three or more tiles per workgroup, a ragged last tile, ldo > n
    (5, 200, 3872, 200),     # K longer than one LDS range: range partials, then their sum
    (300, 896, 896, 904),    # past 64 rows: ten 32-row halves, two tiles per slot
    (200, 896, 4864, 896),   # past 64 rows with two K ranges (no workspace: the tile kernel)
])
def test_gemm_bias_residual_batched(oracle, m, n, k, ldo):
    """out = residual + (GEMM + bias) on k_gemm_bd (every projection of up to
    64 rows, one-tile projections of up to 512), every row against the
    float64 product of the dequantized operands, with and without
    workspace."""
    torch = _torch()
    rng = np.random.default_rng(m + n + k)
    w = q4(oracle, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.normal(0, 0.02, n).astype(np.float32)
    res = rng.standard_normal((m, ldo)).astype(np.float32)
    xq = oracle.quantize_q8(x)
    qs, d, _ = aos_to_planar(xq)
    wqs, wd, tile = _upload_q4(w, n, k)
    want = res[:, :n] + (dequant_q8(xq, m, k) @ dequant_q4(w, n, k).T + b)
    rms = np.sqrt(np.mean(want ** 2))
    wsb = si_amd.lib().si_gemm_workspace(m, n, k)
    for ws_bytes in sorted({0, wsb}):
        ws = empty(max(ws_bytes, 4), torch.uint8)
        out = dev(np.full((m, ldo), 7.0, np.float32))
        si_amd.call("si_gemm_q4q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, n, k,
                    si_amd.ptr(dev(qs)), si_amd.ptr(dev(d.view(np.int16))), m, si_amd.ptr(dev(b)),
                    si_amd.ptr(dev(res)), si_amd.ptr(out), ldo, 0,
                    si_amd.ptr(ws) if ws_bytes else None, ws_bytes, None)
        got = host(out).reshape(m, ldo)
        err = np.abs(got[:, :n] - want).max() / rms
        assert err <= 1e-5, f"workspace {ws_bytes}: worst {err:.3g}"
        assert np.all(got[:, n:] == 7.0), "columns past n written"


@pytest.mark.parametrize("m", [1, 5, 32, 33, 64, 100])
def test_q8_tile_layout(m):
    """si_q8_tile against the layout restated on the host (q8_tiled), padding
    rows included (zero)."""
    torch = _torch()
    k = 384
    rng = np.random.default_rng(m)
    qs = rng.integers(-127, 128, m * k).astype(np.int8)
    d = rng.integers(0, 1 << 16, m * k // 32).astype(np.uint16)
    P = (m + 31) // 32
    tq = dev(np.full(P * 32 * k, 99, np.int8))
    td = dev(np.full(P * 32 * k // 32, 7, np.uint16).view(np.int16))
    si_amd.call("si_q8_tile", si_amd.ptr(dev(qs)), si_amd.ptr(dev(d.view(np.int16))), m, k,
                si_amd.ptr(tq), si_amd.ptr(td), None)
    wq, wd = q8_tiled(qs, d, m, k)
    assert np.array_equal(host(tq), wq)
    assert np.array_equal(host(td).view(np.uint16), wd)


@pytest.mark.parametrize("m,n,k,bias,res", [
    (64, 3584, 18944, False, True),   # config 5's down projection (+ residual)
    (64, 4608, 3584, True, False),    # config 5's Q|K|V (+ bias)
    (64, 3584, 3584, False, False),   # config 5's W_O
    (33, 200, 3872, True, True),      # ragged panel and columns, K past one LDS range
    (5, 256, 512, True, False),
    (1, 1152, 896, False, True),
    (512, 896, 4864, False, True),    # config 3's down projection (+ residual)
    (200, 1152, 896, True, False),    # ragged panel past 64 rows
])
def test_gemm_tiled_a(oracle, m, n, k, bias, res):
    """SI_GEMM_TILED_A (operand-tiled activations streamed with the weights,
    one pass over K) against the float64 product of the dequantized operands
    on every row, and against the default path (planar activations) within
    fp32 summation-order differences: the streamed kernel spreads K over 12
    (or 8) wavefronts, the default over 16 and, for long K, over workgroups."""
    torch = _torch()
    rng = np.random.default_rng(m * 7 + n + k)
    w = q4(oracle, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.normal(0, 0.02, n).astype(np.float32) if bias else None
    r = rng.standard_normal((m, n)).astype(np.float32) if res else None
    xq = oracle.quantize_q8(x)
    qs, d, _ = aos_to_planar(xq)
    wqs, wd, tile = _upload_q4(w, n, k)
    P = (m + 31) // 32
    tq = empty(P * 32 * k, torch.int8)
    td = empty(P * k, torch.int16)
    si_amd.call("si_q8_tile", si_amd.ptr(dev(qs)), si_amd.ptr(dev(d.view(np.int16))), m, k,
                si_amd.ptr(tq), si_amd.ptr(td), None)
    b_d = dev(b) if bias else None
    r_d = dev(r) if res else None

    def gemm(xa, xs, flags, ws=None, wsb=0):
        out = empty(m * n, torch.float32)
        si_amd.call("si_gemm_q4q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, n, k, si_amd.ptr(xa),
                    si_amd.ptr(xs), m, si_amd.ptr(b_d), si_amd.ptr(r_d), si_amd.ptr(out), n, flags,
                    si_amd.ptr(ws), wsb, None)
        return out

    outs = []
    ran = [kn for kn, _ in si_amd.kernel_times_ms(
        "k_gemm", lambda: outs.append(gemm(tq, td, si_amd.SI_GEMM_TILED_A)))]
    # more 32-row halves than the 256 CUs: one unit per 8-wavefront
    # workgroup, two per CU; otherwise the pipelined 12
    wide = -(-n // 32) * -(-m // 32) > 256
    assert ran == ["k_gemm_bd<1, 2, 0, 8, true, false>" if wide
                   else "k_gemm_bd<1, 2, 0, 12, true, true>"], ran
    got = host(outs[0]).reshape(m, n)
    want = dequant_q8(xq, m, k) @ dequant_q4(w, n, k).T
    if bias:
        want = want + b[None, :].astype(np.float64)
    if res:
        want = want + r.astype(np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    err = np.abs(got - want).max(axis=1) / rms
    bad = np.nonzero(err > 1e-5)[0]
    assert bad.size == 0, f"rows off, first {bad[:8].tolist()}, worst {err.max():.3g}"
    wsb = si_amd.lib().si_gemm_workspace(m, n, k)
    ws = empty(max(wsb, 4), torch.uint8)
    ref = host(gemm(dev(qs), dev(d.view(np.int16)), 0, ws, wsb)).reshape(m, n)
    assert np.abs(got - ref).max() / rms <= 2e-6
    again = host(gemm(tq, td, si_amd.SI_GEMM_TILED_A)).reshape(m, n)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), "not deterministic"


def test_gemm_tiled_a_other_panel_nonfinite(oracle):
    """Streamed activations, 64 rows, K = 896 (28 blocks over 12 wavefronts,
    so some steps fall past the range and read the next panel's blocks):
    panel 1 given infinite / NaN scales must leave panel 0's rows exactly as
    with finite ones (an out-of-range block's products carry zero scales)."""
    torch = _torch()
    m, n, k = 64, 128, 896
    rng = np.random.default_rng(5)
    w = q4(oracle, rng, n, k)
    xq = oracle.quantize_q8(rng.standard_normal((m, k)).astype(np.float32))
    qs, d, _ = aos_to_planar(xq)
    wqs, wd, tile = _upload_q4(w, n, k)
    tq = empty(2 * 32 * k, torch.int8)
    td = empty(2 * k, torch.int16)
    si_amd.call("si_q8_tile", si_amd.ptr(dev(qs)), si_amd.ptr(dev(d.view(np.int16))), m, k,
                si_amd.ptr(tq), si_amd.ptr(td), None)

    def gemm(tdv):
        out = empty(m * n, torch.float32)
        si_amd.call("si_gemm_q4q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, n, k,
                    si_amd.ptr(tq), si_amd.ptr(tdv), m, None, None, si_amd.ptr(out), n,
                    si_amd.SI_GEMM_TILED_A, None, 0, None)
        return host(out).reshape(m, n)

    base = gemm(td)
    bad_td = host(td).copy()
    half = k // 32 * 32  # panel 1's scales: [panel][block][row]
    bad_td[half:] = np.where(np.arange(bad_td.size - half) % 2 == 0, 0x7C00, 0x7E00)  # inf, NaN
    got = gemm(dev(bad_td))
    assert np.isfinite(base).all()
    assert np.array_equal(got[:32].view(np.uint32), base[:32].view(np.uint32))


@pytest.mark.parametrize("shape,ntok,pos0", [("0.5b", 1, 1023), ("7b", 5, 0), ("7b", 3, 4093)])
def test_rope_kv_append_bit_exact(oracle, shape, ntok, pos0):
    torch = _torch()
    sd = si_amd.SHAPES[shape]
    s = si_amd.make_shape(**sd)
    D, QD, KVD = s.hdim, s.qheads * s.hdim, s.kvheads * s.hdim
    NQ = QD + 2 * KVD
    rng = np.random.default_rng(ntok)
    qkv = rng.standard_normal((ntok, NQ)).astype(np.float32)
    maxpos = pos0 + ntok
    c = np.empty((maxpos, D // 2), np.float32)
    sn = np.empty_like(c)
    si_amd.call("si_rope_table", maxpos, D, 1e6, si_amd.ptr(c), si_amd.ptr(sn))
    kc = dev(np.zeros(maxpos * KVD, np.uint16).view(np.int16))
    vc = dev(np.zeros(maxpos * KVD, np.uint16).view(np.int16))
    qo = empty(ntok * QD, torch.float32)
    si_amd.call("si_rope_kv_append", ctypes.byref(s), si_amd.ptr(dev(qkv)), NQ, ntok, pos0, 1,
                maxpos, None, si_amd.ptr(dev(c)), si_amd.ptr(dev(sn)), si_amd.ptr(qo), si_amd.ptr(kc),
                si_amd.ptr(vc), 0, None)
    gq = host(qo).reshape(ntok, QD)
    gk = host(kc).view(np.uint16).reshape(maxpos, KVD)
    gv = host(vc).view(np.uint16).reshape(maxpos, KVD)
    for t in range(ntok):
        wq = oracle.rope(qkv[t, :QD], s.qheads, D, pos0 + t)
        wk = oracle.rope(qkv[t, QD:QD + KVD], s.kvheads, D, pos0 + t)
        assert np.array_equal(gq[t].view(np.uint32), wq.view(np.uint32))
        assert np.array_equal(gk[pos0 + t], oracle.f32_to_f16(wk))
        assert np.array_equal(gv[pos0 + t], oracle.f32_to_f16(qkv[t, QD + KVD:]))


def _attention_case(oracle, shape_name, ctx, kmul=1.0, seed=0):
    sd = si_amd.SHAPES[shape_name]
    s = si_amd.make_shape(**sd)
    os_ = or_shape(**sd)
    rng = np.random.default_rng(seed + ctx)
    KVD = s.kvheads * s.hdim
    q = rng.standard_normal(s.qheads * s.hdim).astype(np.float32)
    kc = kv_history(oracle, rng, ctx, KVD, kmul)
    vc = kv_history(oracle, rng, ctx, KVD)
    return s, os_, q, kc, vc


@pytest.mark.parametrize("shape,ctx,kmul", [("0.5b", 1, 1.0), ("0.5b", 2, 0.0125),
                                            ("0.5b", 17, 1.0), ("0.5b", 64, 0.0),
                                            ("0.5b", 1024, 1.0), ("7b", 4096, 1.0),
                                            ("7b", 300, 3.0), ("1.5b_ref", 1000, 0.5),
                                            ("7b", 4097, 1.0)])
def test_attention_decode(oracle, shape, ctx, kmul):
    torch = _torch()
    s, os_, q, kc, vc = _attention_case(oracle, shape, ctx, kmul)
    QD = s.qheads * s.hdim
    ws_bytes = si_amd.lib().si_attention_workspace(ctypes.byref(s), 1, ctx)
    ws = empty(ws_bytes, torch.uint8)
    out = empty(QD, torch.float32)
    qs, d = empty(QD, torch.int8), empty(QD // 32, torch.int16)
    si_amd.call("si_attention", ctypes.byref(s), si_amd.ptr(dev(q)), 1,
                si_amd.ptr(dev(kc.view(np.int16))), si_amd.ptr(dev(vc.view(np.int16))), 0, None,
                ctx, 0, ctx, si_amd.ptr(out), si_amd.ptr(qs), si_amd.ptr(d), None,
                si_amd.ptr(ws), ws_bytes, None)
    got = host(out)
    close(got, oracle.attention_flash(os_, q, kc, vc, ctx), 2e-3, "attention")
    wq, wd, _ = aos_to_planar(oracle.quantize_q8(got))
    assert np.array_equal(host(qs), wq) and np.array_equal(host(d).view(np.uint16), wd)


def test_attention_batched_sequences(oracle):
    """nq sequences, each with its own cache (kv_seq_stride) and context."""
    torch = _torch()
    sd = si_amd.SHAPES["7b"]
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    nseq, maxctx = 6, 700
    KVD, QD = s.kvheads * s.hdim, s.qheads * s.hdim
    rng = np.random.default_rng(42)
    ctxs = np.array([1, 2, 37, 256, 257, 700], np.int32)
    q = rng.standard_normal((nseq, QD)).astype(np.float32)
    kc = kv_history(oracle, rng, nseq * maxctx, KVD).reshape(nseq, maxctx * KVD)
    vc = kv_history(oracle, rng, nseq * maxctx, KVD).reshape(nseq, maxctx * KVD)
    ws_bytes = si_amd.lib().si_attention_workspace(ctypes.byref(s), nseq, maxctx)
    ws = empty(ws_bytes, torch.uint8)
    out = empty(nseq * QD, torch.float32)
    si_amd.call("si_attention", ctypes.byref(s), si_amd.ptr(dev(q)), nseq,
                si_amd.ptr(dev(kc.view(np.int16))), si_amd.ptr(dev(vc.view(np.int16))),
                maxctx * KVD, si_amd.ptr(dev(ctxs)), 0, 0, maxctx, si_amd.ptr(out), None, None,
                None, si_amd.ptr(ws), ws_bytes, None)
    got = host(out).reshape(nseq, QD)
    for i in range(nseq):
        want = oracle.attention_flash(os_, q[i], kc[i], vc[i], int(ctxs[i]))
        close(got[i], want, 2e-3, f"seq {i}")


# query heads per KV group beyond one workgroup's 8 (two head subsets) and
# an odd group width, besides the BASELINE shapes
_WIDE_GROUPS = {"wide16": dict(hidden=2048, qheads=32, kvheads=2, hdim=64),
                "odd3": dict(hidden=1152, qheads=9, kvheads=3, hdim=128)}


@pytest.mark.parametrize("shape,ntok,prefix", [("0.5b", 40, 300), ("7b", 45, 17),
                                               ("wide16", 70, 33), ("odd3", 33, 64)])
def test_attention_causal_prefill(oracle, shape, ntok, prefix):
    """nq query rows over one cache (the flash prefill kernel): row t attends
    to prefix+t+1 positions; every row and its Q8_0."""
    torch = _torch()
    sd = si_amd.SHAPES.get(shape) or _WIDE_GROUPS[shape]
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    KVD, QD = s.kvheads * s.hdim, s.qheads * s.hdim
    rng = np.random.default_rng(7)
    total = prefix + ntok
    q = rng.standard_normal((ntok, QD)).astype(np.float32)
    kc = kv_history(oracle, rng, total, KVD)
    vc = kv_history(oracle, rng, total, KVD)
    ws_bytes = si_amd.lib().si_attention_workspace(ctypes.byref(s), ntok, total)
    ws = empty(ws_bytes, torch.uint8)
    out = empty(ntok * QD, torch.float32)
    aq, ad = empty(ntok * QD, torch.int8), empty(ntok * QD // 32, torch.int16)
    si_amd.call("si_attention", ctypes.byref(s), si_amd.ptr(dev(q)), ntok,
                si_amd.ptr(dev(kc.view(np.int16))), si_amd.ptr(dev(vc.view(np.int16))), 0, None,
                prefix + 1, 1, total, si_amd.ptr(out), si_amd.ptr(aq), si_amd.ptr(ad), None,
                si_amd.ptr(ws), ws_bytes, None)
    got = host(out).reshape(ntok, QD)
    for t in range(ntok):
        want = oracle.attention_flash(os_, q[t], kc, vc, prefix + t + 1)
        close(got[t], want, 2e-3, f"row {t}")
    want_q, want_d, _ = aos_to_planar(oracle.quantize_q8(got.reshape(-1)))
    assert np.array_equal(host(aq), want_q)
    assert np.array_equal(host(ad).view(np.uint16), want_d)


def test_mfma_f16_lane_layouts():
    """The fp16 16x16 matrix-core layouts assumed by the attention kernels."""
    torch = _torch()
    rng = np.random.default_rng(0)
    a = rng.integers(-8, 8, (16, 32)).astype(np.float16)
    b = rng.integers(-8, 8, (32, 16)).astype(np.float16)
    d32, d16 = empty(256, torch.float32), empty(256, torch.float32)
    from tests.probe import call as probe_call
    probe_call("si_probe_mfma_f16", si_amd.ptr(dev(a.view(np.int16))),
               si_amd.ptr(dev(b.view(np.int16))), si_amd.ptr(d32), si_amd.ptr(d16), None)
    af, bf = a.astype(np.float64), b.astype(np.float64)
    assert np.array_equal(host(d32).reshape(16, 16), af @ bf)
    assert np.array_equal(host(d16).reshape(16, 16), af[:, :16] @ bf[:16, :])


def test_cross_lane_ops_layouts():
    """The DPP / permlane moves behind every in-kernel reduction, checked
    against their documented lane maps."""
    torch = _torch()
    out = zeros(19 * 64, torch.int32)
    from tests.probe import call as probe_call
    probe_call("si_probe_lane_ops", si_amd.ptr(out), None)
    got = host(out).reshape(19, 64)
    lane = np.arange(64)
    row0 = lane & ~15
    expect = {
        0: lane ^ 1, 1: lane ^ 2,
        2: row0 + ((lane - 4) & 15), 3: row0 + ((lane - 8) & 15),
        4: (lane & ~7) + 7 - (lane & 7),
        5: lane ^ 16, 6: lane ^ 32,
    }
    for k, want in expect.items():
        assert np.array_equal(got[k], want), f"op {k}: {got[k]}"
    grp = lambda size: np.repeat(lane.reshape(-1, size).sum(1), size)
    gmax = lambda size: np.repeat(lane.reshape(-1, size).max(1), size)
    assert np.array_equal(got[7], grp(8)), "oct_sum"
    assert np.array_equal(got[8], grp(32)), "half_wave_sum"
    assert np.array_equal(got[9], grp(64)), "wave_sum"
    assert np.array_equal(got[10], gmax(32)), "half_wave_max"
    assert np.array_equal(got[11], gmax(64)), "wave_max"
    assert np.array_equal(got[12], gmax(8)), "oct_max"
    for k, r in ((13, 4), (14, 8), (15, 16), (16, 32)):
        want = np.array([lane[lane % r == l % r].sum() for l in lane])
        assert np.array_equal(got[k], want), f"fold_rows<{r}>"
    assert np.array_equal(got[17], grp(64)), "wave_sum_d"
    # row_shl:1 of lane + 1: lane i gets lane i + 1's value, a row's last lane 0
    assert np.array_equal(got[18], np.where(lane % 16 != 15, lane + 2, 0)), "DPP_SHL1"


@pytest.mark.parametrize("shape,flags", [("0.5b", 0), ("0.5b", si_amd.SI_GEMM_EXACT),
                                         ("7b", 0)])
def test_ffn_gateup_q8(oracle, shape, flags):
    """The fused decode FFN front half against the oracle, chained: the
    projections of the GPU's own quantized input (bit-exact with EXACT),
    SwiGLU within 1e-6, its Q8 bit-exact on the GPU's own activations."""
    torch = _torch()
    from oracle.oracle_py import make_shape as or_shape
    os_ = or_shape(**si_amd.SHAPES[shape])
    H, F = os_.hidden, os_.ffn
    rng = np.random.default_rng(F + flags)
    wg, wu = q4(oracle, rng, F, H), q4(oracle, rng, F, H)
    gain = rng.normal(1, 0.1, H).astype(np.float32)
    h = rng.standard_normal(H).astype(np.float32)
    wqs, wd, _ = _upload_q4(np.concatenate([wg, wu]), 2 * F, H, 32)
    act = empty(F, torch.float32)
    aq, ad, asum = empty(F, torch.int8), empty(F // 32, torch.int16), empty(F // 32, torch.int16)
    si_amd.call("si_ffn_gateup_q8", si_amd.ptr(dev(h)), si_amd.ptr(dev(gain)), H, 1e-6,
                si_amd.ptr(wqs), si_amd.ptr(wd), 32, F, si_amd.ptr(act), si_amd.ptr(aq),
                si_amd.ptr(ad), si_amd.ptr(asum), flags, None)
    xq = oracle.quantize_q8(oracle.rmsnorm(h, gain))
    g = oracle.matvec(wg, xq, H, F)
    u = oracle.matvec(wu, xq, H, F)
    got = host(act)
    close(got, oracle.swiglu(g, u), 1e-5 if flags == 0 else 1e-6, "SwiGLU")
    want_q, want_d, want_s = aos_to_planar(oracle.quantize_q8(got))
    assert np.array_equal(host(aq), want_q)
    assert np.array_equal(host(ad).view(np.uint16), want_d)
    assert np.array_equal(host(asum), want_s)


@pytest.mark.parametrize("m,f,k,tile,flags,act_out", [
    (130, 96, 256, 8, 0, True),          # ragged rows, f an odd number of 32-blocks
    (64, 4864, 896, 32, 0, True),        # 0.5B batched-decode shape (64-row tiles)
    (512, 4864, 896, 32, 0, False),      # 0.5B prefill shape; also without act and sums
    (128, 4864, 896, 32, 0, True),       # one-pass plan where the tile kernel would split K
    (2, 160, 96, 16, 0, True),           # tiny: the plan splits K (GEMM + SwiGLU kernel)
    (300, 4864, 896, 32, si_amd.SI_GEMM_EXACT, True),
    (600, 4864, 896, 32, 0, True),       # past 512 rows: 128-row tiles
    (2048, 18944, 3584, 32, 0, True),    # 7B 2048-token prefill, the instance config 4 times
    (33, 96, 3840, 8, 0, True),          # batched decode, the longest K of one LDS range
    (64, 256, 4096, 32, 0, True),        # batched decode, longer K: range partials + reduce
])
def test_gemm_gateup_q8(oracle, m, f, k, tile, flags, act_out):
    """gate|up GEMM with the SwiGLU + Q8_0 epilogue: every row's gate|up
    against the float64 product of the dequantized operands (bit-exact with
    the reference's matvec under SI_GEMM_EXACT), SwiGLU on the GPU's own
    gate|up within 1e-6, and its Q8_0 bit-exact."""
    torch = _torch()
    rng = np.random.default_rng(m + f + k)
    wg, wu = q4(oracle, rng, f, k), q4(oracle, rng, f, k)
    w = np.concatenate([wg, wu])
    x = rng.standard_normal((m, k)).astype(np.float32)
    xq = oracle.quantize_q8(x)
    qs, d, _ = aos_to_planar(xq)
    wqs, wd, _ = _upload_q4(w, 2 * f, k, tile)
    wsb = si_amd.lib().si_gemm_workspace(m, 2 * f, k)
    ws = empty(max(wsb, 4), torch.uint8)
    xqs_d, xd_d = dev(qs), dev(d.view(np.int16))

    def run(with_act, with_gu=True):
        gu = empty(m * 2 * f, torch.float32) if with_gu else None
        act = empty(m * f, torch.float32) if with_act else None
        aq, ad = empty(m * f, torch.int8), empty(m * f // 32, torch.int16)
        asum = empty(m * f // 32, torch.int16) if with_act else None
        si_amd.call("si_gemm_gateup_q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, f, k,
                    si_amd.ptr(xqs_d), si_amd.ptr(xd_d), m, si_amd.ptr(gu), si_amd.ptr(act),
                    si_amd.ptr(aq), si_amd.ptr(ad), si_amd.ptr(asum), flags, si_amd.ptr(ws),
                    wsb, None)
        return gu, act, aq, ad, asum

    gu, act, aq, ad, asum = run(True)
    if not flags:  # gu is optional given the workspace: the same Q8_0 without it
        _, _, aq3, ad3, _ = run(True, with_gu=False)
        assert np.array_equal(host(aq3), host(aq)) and np.array_equal(host(ad3), host(ad))
    if not act_out:  # NULL act and block sums: the same gate|up and Q8_0
        gu2, _, aq2, ad2, _ = run(False)
        assert np.array_equal(host(gu2).view(np.uint32), host(gu).view(np.uint32))
        assert np.array_equal(host(aq2), host(aq))
        assert np.array_equal(host(ad2), host(ad))
    g = host(gu).reshape(m, 2 * f)
    nb = k // 32
    if flags:
        for r in sorted({0, m // 2, m - 1}):
            want = oracle.matvec(w, xq[r * nb:(r + 1) * nb], k, 2 * f)
            assert np.array_equal(g[r].view(np.uint32), want.view(np.uint32)), f"row {r}"
    else:
        # float64 product of the dequantized operands, on the GPU (rocBLAS
        # dgemm) because at 2048 x 37888 x 3584 a host product takes minutes
        a64 = torch.from_numpy(dequant_q8(xq, m, k)).cuda()
        w64 = torch.from_numpy(dequant_q4(w, 2 * f, k)).cuda()
        want = (a64 @ w64.T).cpu().numpy()
        del a64, w64
        rms = np.sqrt(np.mean(want ** 2))
        err = np.abs(g - want).max(axis=1) / rms
        assert err.max() <= 1e-5, f"gate|up rows off: worst {err.max():.3g} at {int(err.argmax())}"
    sw = np.stack([oracle.swiglu(g[r, :f], g[r, f:]) for r in range(m)])
    close(host(act), sw, 1e-6, "SwiGLU")
    want_q, want_d, want_s = aos_to_planar(oracle.quantize_q8(host(act)))
    assert np.array_equal(host(aq), want_q)
    assert np.array_equal(host(ad).view(np.uint16), want_d)
    assert np.array_equal(host(asum), want_s)


@pytest.mark.parametrize("m,f,k", [(64, 18944, 3584), (33, 4864, 896), (2, 256, 512),
                                   (64, 160, 3840)])
def test_gemm_gateup_tiled_a_bit_identical(oracle, m, f, k):
    """SI_GEMM_TILED_A on the gate|up GEMM (operand-tiled activations
    streamed with the weights; the wavefronts' partial sums reduced in LDS
    per tile, SwiGLU + Q8_0 of all a workgroup's tiles at its end) gives the
    default's gate|up, SwiGLU and Q8_0 bit for bit: the same blocks per
    wavefront and the same order of sums.  Ragged row panels included;
    shapes it does not take are refused."""
    torch = _torch()
    rng = np.random.default_rng(m + 5 * f)
    w = np.concatenate([q4(oracle, rng, f, k), q4(oracle, rng, f, k)])
    x = rng.standard_normal((m, k)).astype(np.float32)
    qs, d, _ = aos_to_planar(oracle.quantize_q8(x))
    wqs, wd, _ = _upload_q4(w, 2 * f, k, 32)
    P = (m + 31) // 32
    tq = empty(P * 32 * k, torch.int8)
    td = empty(P * k, torch.int16)
    si_amd.call("si_q8_tile", si_amd.ptr(dev(qs)), si_amd.ptr(dev(d.view(np.int16))), m, k,
                si_amd.ptr(tq), si_amd.ptr(td), None)
    ins = {0: (dev(qs), dev(d.view(np.int16))), si_amd.SI_GEMM_TILED_A: (tq, td)}
    outs = []
    for flags, (xa, xs) in ins.items():
        gu = empty(m * 2 * f, torch.float32)
        act = empty(m * f, torch.float32)
        aq, ad = empty(m * f, torch.int8), empty(m * f // 32, torch.int16)
        asum = empty(m * f // 32, torch.int16)

        def run():
            si_amd.call("si_gemm_gateup_q8", si_amd.ptr(wqs), si_amd.ptr(wd), 32, f, k,
                        si_amd.ptr(xa), si_amd.ptr(xs), m, si_amd.ptr(gu), si_amd.ptr(act),
                        si_amd.ptr(aq), si_amd.ptr(ad), si_amd.ptr(asum), flags, None, 0, None)
        ran = [kn for kn, _ in si_amd.kernel_times_ms("k_gemm", run)]
        assert len(ran) == 1 and ran[0].startswith("k_gemm_bd<2,") and \
            ran[0].endswith(", true, false>" if flags else ", false, false>"), ran
        outs.append([host(t) for t in (gu, act, aq, ad, asum)])
    for name, a, b in zip(("gate|up", "SwiGLU", "Q8", "scales", "block sums"), *outs):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), name
    L = si_amd.lib()
    a16 = 1 << 12
    assert L.si_gemm_gateup_q8(a16, a16, 32, 64, 64, a16, a16, 65, None, None, a16, a16, None,
                               si_amd.SI_GEMM_TILED_A, None, 0, None) == si_amd.SI_ERR_ARG
    assert L.si_gemm_gateup_q8(a16, a16, 32, 64, 3872, a16, a16, 8, None, None, a16, a16, None,
                               si_amd.SI_GEMM_TILED_A, None, 0, None) == si_amd.SI_ERR_ARG


@pytest.mark.parametrize("m,f,k", [(130, 96, 256), (600, 4864, 896), (2048, 18944, 3584),
                                   (77, 160, 3840)])
def test_gemm_gateup_f16_formulation_bit_identical(oracle, m, f, k):
    """SI_GEMM_F16 (f16 matrix-core products of the integer-valued operands,
    converted once per LDS stage) gives the default int8 formulation's
    gate|up, SwiGLU and Q8_0 bit for bit: both form each block's exact dot
    and apply the same fused multiply-adds in the same order.  Ragged rows
    and columns included; SI_GEMM_EXACT with it is refused."""
    torch = _torch()
    rng = np.random.default_rng(m + 3 * f)
    w = np.concatenate([q4(oracle, rng, f, k), q4(oracle, rng, f, k)])
    x = rng.standard_normal((m, k)).astype(np.float32)
    qs, d, _ = aos_to_planar(oracle.quantize_q8(x))
    wqs, wd, _ = _upload_q4(w, 2 * f, k, 32)
    xqs_d, xd_d = dev(qs), dev(d.view(np.int16))
    outs = []
    for flags in (0, si_amd.SI_GEMM_F16):
        gu = empty(m * 2 * f, torch.float32)
        act = empty(m * f, torch.float32)
        aq, ad = empty(m * f, torch.int8), empty(m * f // 32, torch.int16)
        asum = empty(m * f // 32, torch.int16)
        # no workspace: the default formulation also runs one pass over K
        # (a K split would add its partial sums in another order)
        si_amd.call("si_gemm_gateup_q8", si_amd.ptr(wqs), si_amd.ptr(wd), 32, f, k,
                    si_amd.ptr(xqs_d), si_amd.ptr(xd_d), m, si_amd.ptr(gu), si_amd.ptr(act),
                    si_amd.ptr(aq), si_amd.ptr(ad), si_amd.ptr(asum), flags, None, 0, None)
        outs.append([host(t) for t in (gu, act, aq, ad, asum)])
    for name, a, b in zip(("gate|up", "act", "q", "d", "sums"), *outs):
        assert np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8)), name
    with pytest.raises(si_amd.SiError):
        si_amd.call("si_gemm_gateup_q8", si_amd.ptr(wqs), si_amd.ptr(wd), 32, f, k,
                    si_amd.ptr(xqs_d), si_amd.ptr(xd_d), m, si_amd.ptr(gu), None, si_amd.ptr(aq),
                    si_amd.ptr(ad), None, si_amd.SI_GEMM_EXACT | si_amd.SI_GEMM_F16, None, 0,
                    None)
