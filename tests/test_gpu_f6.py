"""The fp6 formulation of the prefill GEMMs (SI_GEMM_F6, k_gemm_f6), which the
layer runs past 512 rows.

Each Q8 value q is split as 16 (q >> 4) + (q & 15) and every part, like
every weight nibble - 8, is stored as the fp6 e2m3 code of half its value;
one scaled fp6 matrix instruction per 32 x 32 tile and block then yields the
block's integer dot exactly.  The epilogue is the default tile kernel's fma
on the same blocks in the same order, so wherever the default runs that
kernel (more than 512 rows) the outputs must agree bit for bit: checked at
config 4's exact shapes (Q|K|V with bias, O, down with residual and a 5-way
K split, the fused gate|up + SwiGLU + Q8), on ragged shapes (odd m: the
converted activations' regions then start only 8-byte aligned; n not a
multiple of the 128-wide tile; K in one stage; 3- and 11-way K splits, the
last part shorter) and against the float64 product of the dequantized
operands.  The reference's contract for these products is matvec_q4q8 per
token (qwen_one_layer.c:148-162)."""
import numpy as np
import pytest

import si_amd
from tests.gpu_helpers import aos_to_planar, dequant_q4, dequant_q8, dev, empty, host, q4

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _upload_q4(w_rowmajor, n, k, tile=None):
    torch = _torch()
    L = si_amd.lib()
    tile = tile or L.si_q4_tile(n, k)
    qs = empty(n * k // 2, torch.uint8)
    d = empty(L.si_q4_scale_count(n, k, tile), torch.int16)
    d.zero_()
    si_amd.call("si_q4_repack", si_amd.ptr(dev(w_rowmajor)), n, k, tile, si_amd.ptr(qs),
                si_amd.ptr(d), None)
    return qs, d, tile


def _f64_product(xq, w, m, n, k):
    """float64 product of the dequantized operands (on the GPU past a size a
    host product would take long over)."""
    torch = _torch()
    if m * n * k > 1 << 31:
        a64 = torch.from_numpy(dequant_q8(xq, m, k)).cuda()
        w64 = torch.from_numpy(dequant_q4(w, n, k)).cuda()
        return (a64 @ w64.T).cpu().numpy()
    return dequant_q8(xq, m, k) @ dequant_q4(w, n, k).T


# (m, n, k, bias, residual, kernels in launch order)
SHAPES = [
    (2048, 4608, 3584, True, False, ["k_gemm_f6<2, 2, 2, 2, false>"]),   # config 4 Q|K|V
    (2048, 3584, 3584, False, False, ["k_gemm_f6<2, 2, 2, 2, false>"]),  # config 4 O
    (2048, 3584, 18944, False, True,                                      # config 4 down
     ["k_gemm_f6<2, 2, 2, 2, false>", "k_gemm_reduce4"]),
    (701, 1000, 896, True, True,                                          # ragged m, n; 3 splits
     ["k_gemm_f6<2, 2, 2, 2, false>", "k_gemm_reduce4"]),
    (600, 96, 64, True, False, ["k_gemm_f6<2, 2, 2, 2, false>"]),        # one stage, n < tile
    (1025, 256, 4096, True, True,                                         # 11-way K split
     ["k_gemm_f6<2, 2, 2, 2, false>", "k_gemm_reduce4"]),
]


@pytest.mark.parametrize("m,n,k,bias,residual,kernels", SHAPES,
                         ids=[f"{s[0]}x{s[1]}x{s[2]}" for s in SHAPES])
def test_gemm_f6_bit_identical_to_default(oracle, m, n, k, bias, residual, kernels):
    torch = _torch()
    L = si_amd.lib()
    rng = np.random.default_rng(m * 7 + n + k)
    w = q4(oracle, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.normal(0, 0.02, n).astype(np.float32) if bias else None
    res = rng.standard_normal((m, n)).astype(np.float32) if residual else None
    xq = oracle.quantize_q8(x)
    qs, d, _ = aos_to_planar(xq)
    wqs, wd, tile = _upload_q4(w, n, k)
    xqs_d, xd_d = dev(qs), dev(d.view(np.int16))
    b_d = dev(b) if bias else None
    r_d = dev(res) if residual else None

    def run(flags, wsb):
        ws = empty(max(wsb, 256), torch.uint8)
        out = empty(m * n, torch.float32)
        si_amd.call("si_gemm_q4q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, n, k,
                    si_amd.ptr(xqs_d), si_amd.ptr(xd_d), m, si_amd.ptr(b_d), si_amd.ptr(r_d),
                    si_amd.ptr(out), n, flags, si_amd.ptr(ws), wsb, None)
        return host(out).reshape(m, n)

    base = run(0, L.si_gemm_workspace(m, n, k))
    got = []
    ran = [kn for kn, _ in si_amd.kernel_times_ms(
        "k_gemm", lambda: got.append(run(si_amd.SI_GEMM_F6, L.si_gemm_f6_workspace(m, n, k))))]
    assert ran == kernels, f"kernels {ran}, expected {kernels}"
    f6 = got[0]
    diff = np.nonzero(f6.view(np.uint32) != base.view(np.uint32))
    assert diff[0].size == 0, (f"{diff[0].size} outputs differ from the default path, first "
                               f"(row, col) {list(zip(diff[0][:4].tolist(), diff[1][:4].tolist()))}")
    want = _f64_product(xq, w, m, n, k)
    rms = np.sqrt(np.mean(want ** 2))
    if bias:
        want = want + b[None, :].astype(np.float64)
    if residual:
        want = want + res.astype(np.float64)
    err = np.abs(f6 - want).max(axis=1) / rms
    assert err.max() <= 1e-5, f"rows off the float64 product: worst {err.max():.3g}"


@pytest.mark.parametrize("m,f,k", [(2048, 18944, 3584), (700, 160, 128)],
                         ids=["config4_gateup", "ragged"])
def test_gemm_gateup_f6_bit_identical_to_default(oracle, m, f, k):
    """The fused gate|up + SwiGLU + Q8_0 pass: gate|up, SwiGLU, the Q8_0
    bytes, scales and block sums all equal the default path's."""
    torch = _torch()
    L = si_amd.lib()
    rng = np.random.default_rng(m + f + k)
    w = np.concatenate([q4(oracle, rng, f, k), q4(oracle, rng, f, k)])
    x = rng.standard_normal((m, k)).astype(np.float32)
    xq = oracle.quantize_q8(x)
    qs, d, _ = aos_to_planar(xq)
    wqs, wd, tile = _upload_q4(w, 2 * f, k, 32)
    xqs_d, xd_d = dev(qs), dev(d.view(np.int16))

    def run(flags, wsb):
        ws = empty(max(wsb, 256), torch.uint8)
        gu = empty(m * 2 * f, torch.float32)
        act = empty(m * f, torch.float32)
        aq, ad = empty(m * f, torch.int8), empty(m * f // 32, torch.int16)
        asum = empty(m * f // 32, torch.int16)
        si_amd.call("si_gemm_gateup_q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, f, k,
                    si_amd.ptr(xqs_d), si_amd.ptr(xd_d), m, si_amd.ptr(gu), si_amd.ptr(act),
                    si_amd.ptr(aq), si_amd.ptr(ad), si_amd.ptr(asum), flags, si_amd.ptr(ws),
                    wsb, None)
        return [host(t) for t in (gu, act, aq, ad, asum)]

    base = run(0, L.si_gemm_workspace(m, 2 * f, k))
    got = []
    ran = [kn for kn, _ in si_amd.kernel_times_ms(
        "k_gemm", lambda: got.append(run(si_amd.SI_GEMM_F6, L.si_gemm_f6_workspace(m, 2 * f, k))))]
    assert ran == ["k_gemm_f6<2, 2, 2, 2, true>"], f"kernels {ran}"
    for what, a, b in zip(("gate|up", "SwiGLU", "Q8 values", "Q8 scales", "Q8 block sums"),
                          got[0], base):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{what} differ"
    g = got[0][0].reshape(m, 2 * f)
    want = _f64_product(xq, w, m, 2 * f, k)
    err = np.abs(g - want).max(axis=1) / np.sqrt(np.mean(want ** 2))
    assert err.max() <= 1e-5, f"gate|up rows off the float64 product: worst {err.max():.3g}"


@pytest.mark.parametrize("m,n,k", [(100, 256, 512), (64, 3584, 18944)],
                         ids=["100x256x512", "config5_down"])
def test_gemm_f6_small_m(oracle, m, n, k):
    """Below 513 rows the default path streams with another summation order;
    the fp6 tile pass (64-row tiles) is checked against float64 there, also
    at config 5's down projection (a 21-way K split and its reduce)."""
    torch = _torch()
    L = si_amd.lib()
    rng = np.random.default_rng(m + n + k)
    w = q4(oracle, rng, n, k)
    xq = oracle.quantize_q8(rng.standard_normal((m, k)).astype(np.float32))
    qs, d, _ = aos_to_planar(xq)
    wqs, wd, tile = _upload_q4(w, n, k)
    wsb = L.si_gemm_f6_workspace(m, n, k)
    ws = empty(wsb, torch.uint8)
    out = empty(m * n, torch.float32)
    ran = [kn for kn, _ in si_amd.kernel_times_ms("k_gemm", lambda: si_amd.call(
        "si_gemm_q4q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, n, k, si_amd.ptr(dev(qs)),
        si_amd.ptr(dev(d.view(np.int16))), m, None, None, si_amd.ptr(out), n,
        si_amd.SI_GEMM_F6, si_amd.ptr(ws), wsb, None))]
    assert ran[0] == "k_gemm_f6<1, 4, 2, 1, false>", ran
    want = _f64_product(xq, w, m, n, k)
    err = np.abs(host(out).reshape(m, n) - want).max(axis=1) / np.sqrt(np.mean(want ** 2))
    assert err.max() <= 1e-5, f"worst {err.max():.3g}"
