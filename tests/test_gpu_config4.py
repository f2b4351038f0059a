"""Parity of the kernels BASELINE config 4 times (7B layer, 2048-token
prefill, default flags), each at its exact shape and instance.

The layer's four projections at 2048 rows run the 128 x 128 tile kernel
k_gemm_fast<2, 2, 2, 2, ...> in one pass (Q|K|V with bias, O) or with K
split over workgroups and the float4 split reduce (down, with the residual
added in the reduce); gate|up runs the fused SwiGLU + Q8 instance (checked
in test_gpu_kernels.py::test_gemm_gateup_q8).  Each output row is compared
with the float64 product of the dequantized operands, computed on the GPU
(rocBLAS dgemm): a host product at these sizes takes minutes.  The
reference's contract for these products is matvec_q4q8 applied per token
(qwen_one_layer.c:148-162, prefill_weight_stationary.h:183-311)."""
import numpy as np
import pytest

import si_amd
from tests.gpu_helpers import aos_to_planar, dequant_q4, dequant_q8, dev, empty, host, q4

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _upload_q4(w_rowmajor, n, k):
    torch = _torch()
    L = si_amd.lib()
    tile = L.si_q4_tile(n, k)
    qs = empty(n * k // 2, torch.uint8)
    d = empty(L.si_q4_scale_count(n, k, tile), torch.int16)
    d.zero_()
    si_amd.call("si_q4_repack", si_amd.ptr(dev(w_rowmajor)), n, k, tile, si_amd.ptr(qs),
                si_amd.ptr(d), None)
    return qs, d, tile


# (name, n, k, bias, residual, kernels expected in launch order)
CASES = [
    ("qkv", 4608, 3584, True, False, ["k_gemm_fast<2, 2, 2, 2, false>"]),
    ("o", 3584, 3584, False, False, ["k_gemm_fast<2, 2, 2, 2, false>"]),
    ("down", 3584, 18944, False, True, ["k_gemm_fast<2, 2, 2, 2, false>", "k_gemm_reduce4"]),
]


@pytest.mark.parametrize("name,n,k,bias,residual,kernels", CASES, ids=[c[0] for c in CASES])
def test_gemm_config4_fast_shapes(oracle, name, n, k, bias, residual, kernels):
    torch = _torch()
    m = 2048
    rng = np.random.default_rng(n + k + m)
    w = q4(oracle, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.normal(0, 0.02, n).astype(np.float32) if bias else None
    res = rng.standard_normal((m, n)).astype(np.float32) if residual else None
    xq = oracle.quantize_q8(x)
    qs, d, _ = aos_to_planar(xq)
    wqs, wd, tile = _upload_q4(w, n, k)
    wsb = si_amd.lib().si_gemm_workspace(m, n, k)
    ws = empty(max(wsb, 4), torch.uint8)
    xqs_d, xd_d = dev(qs), dev(d.view(np.int16))
    b_d = dev(b) if bias else None
    r_d = dev(res) if residual else None
    outs = []

    def run():
        out = empty(m * n, torch.float32)
        si_amd.call("si_gemm_q4q8", si_amd.ptr(wqs), si_amd.ptr(wd), tile, n, k,
                    si_amd.ptr(xqs_d), si_amd.ptr(xd_d), m, si_amd.ptr(b_d), si_amd.ptr(r_d),
                    si_amd.ptr(out), n, 0, si_amd.ptr(ws), wsb, None)
        outs.append(out)

    ran = [kn for kn, _ in si_amd.kernel_times_ms("k_gemm", run)]
    assert ran == kernels, f"{name}: kernels {ran}, expected {kernels}"
    run()  # a second call: the split sums are added in a fixed order
    got = host(outs[0]).reshape(m, n)
    assert np.array_equal(got.view(np.uint32), host(outs[1]).reshape(m, n).view(np.uint32)), \
        f"{name}: not deterministic"
    a64 = torch.from_numpy(dequant_q8(xq, m, k)).cuda()
    w64 = torch.from_numpy(dequant_q4(w, n, k)).cuda()
    prod = (a64 @ w64.T).cpu().numpy()
    del a64, w64
    rms = np.sqrt(np.mean(prod ** 2))
    want = prod
    if bias:
        want = want + b[None, :].astype(np.float64)
    if residual:
        want = want + res.astype(np.float64)
    err = np.abs(got - want).max(axis=1) / rms
    bad = np.nonzero(err > 1e-5)[0]
    assert bad.size == 0, f"{name}: rows off, first {bad[:8].tolist()}, worst {err.max():.3g}"
