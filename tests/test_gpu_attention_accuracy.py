"""Accuracy of the GPU attention against a float64 textbook softmax, next to
the oracle's own fp32 error, at the decode/batched/prefill split shapes."""
import ctypes

import numpy as np
import pytest

import si_amd
from oracle.oracle_py import make_shape as or_shape
from tests.gpu_helpers import dev, empty, host, kv_history

pytestmark = pytest.mark.gpu


def _f64_attention(q, kc, vc, s, ctx, f16_to_f32):
    D, per = s.hdim, s.qheads // s.kvheads
    K = f16_to_f32(kc[:ctx * s.kvheads * D]).astype(np.float64).reshape(ctx, s.kvheads, D)
    V = f16_to_f32(vc[:ctx * s.kvheads * D]).astype(np.float64).reshape(ctx, s.kvheads, D)
    out = np.zeros((s.qheads, D))
    for h in range(s.qheads):
        sc = K[:, h // per] @ q[h * D:(h + 1) * D].astype(np.float64) / np.sqrt(D)
        p = np.exp(sc - sc.max())
        out[h] = (p / p.sum()) @ V[:, h // per]
    return out.reshape(-1)


@pytest.mark.parametrize("shape,nq,ctx", [("7b", 64, 300), ("7b", 64, 4096), ("7b", 1, 300),
                                          ("0.5b", 1, 1024), ("7b", 1, 17)])
def test_attention_error_vs_float64(oracle, shape, nq, ctx):
    import torch
    sd = si_amd.SHAPES[shape]
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    QD, KVD = s.qheads * s.hdim, s.kvheads * s.hdim
    rng = np.random.default_rng(ctx + nq)
    q = (rng.standard_normal((nq, QD)) * 1.2).astype(np.float32)
    kc = kv_history(oracle, rng, nq * ctx, KVD)
    vc = kv_history(oracle, rng, nq * ctx, KVD)
    wsb = si_amd.lib().si_attention_workspace(ctypes.byref(s), nq, ctx)
    ws = empty(wsb, torch.uint8)
    out = empty(nq * QD, torch.float32)
    si_amd.call("si_attention", ctypes.byref(s), si_amd.ptr(dev(q)), nq,
                si_amd.ptr(dev(kc.view(np.int16))), si_amd.ptr(dev(vc.view(np.int16))),
                ctx * KVD, None, ctx, 0, ctx, si_amd.ptr(out), None, None, None, si_amd.ptr(ws),
                wsb, None)
    got = host(out).reshape(nq, QD)
    i = nq - 1
    b = i * ctx * KVD
    ref = _f64_attention(q[i], kc[b:], vc[b:], os_, ctx, oracle.f16_to_f32)
    orc = oracle.attention_flash(os_, q[i], kc[b:], vc[b:], ctx)
    rms = np.sqrt(np.mean(ref ** 2))
    e_gpu = np.abs(got[i] - ref).max() / rms
    e_orc = np.abs(orc - ref).max() / rms
    print(f"{shape} nq={nq} ctx={ctx}: gpu-f64 {e_gpu:.3g}  oracle-f64 {e_orc:.3g}  "
          f"gpu-oracle {np.abs(got[i] - orc).max() / rms:.3g}")
    assert e_gpu < 2e-5, (e_gpu, e_orc)
