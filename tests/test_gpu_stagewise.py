"""Stage-by-stage parity of the multi-row layer schedules (prefill and batched
decode): every stage is checked on the GPU's OWN inputs to that stage, so a
failure names the kernel that diverged instead of the end of the layer.

Quantization stages are bit-exact; projection stages are compared with the
float64 product of the dequantized operands; RoPE/K-V append bit-exact;
attention within 2e-3."""
import numpy as np
import pytest

import si_amd
from oracle.oracle_py import Q8_DTYPE, make_shape as or_shape
from tests.gpu_helpers import (close, dequant_q4, dev, device_view, empty, host, kv_history,
                               make_layer, planar_to_aos)

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _buf(L, name, count, dtype):
    return host(device_view(L.buffer(name), count, dtype).clone())


def _q8_rows(L, prefix, rows, k):
    torch = _torch()
    qs = _buf(L, prefix + "_QS", rows * k, torch.int8)
    d = _buf(L, prefix + "_D", rows * k // 32, torch.int16).view(np.uint16)
    return planar_to_aos(qs, d)


def _rows_off(got, want, rtol):
    rms = np.sqrt(np.mean(want.astype(np.float64) ** 2))
    err = np.abs(got.astype(np.float64) - want).max(axis=1) / max(rms, 1e-30)
    return np.nonzero(err > rtol)[0], err


def _check_rows(what, got, want, rtol):
    bad, err = _rows_off(got, want, rtol)
    assert bad.size == 0, (f"{what}: {bad.size} rows off (row mod 64: "
                           f"{sorted(set((bad % 64).tolist()))[:12]}, first {bad[:8].tolist()},"
                           f" worst {err.max():.3g} of rms)")


def _mm(a, w):
    """a @ w.T in float64 on the GPU (rocBLAS dgemm): the reference product
    of dequantized operands, exact to ~1e-16 relative, at sizes (7B x 2048
    rows) where a host float64 product would take minutes."""
    torch = _torch()
    at = torch.from_numpy(np.ascontiguousarray(a, np.float64)).cuda()
    wt = torch.from_numpy(np.ascontiguousarray(w, np.float64)).cuda()
    r = (at @ wt.T).cpu().numpy()
    del at, wt
    return r


def _dequant_act(blocks, rows, k):
    q = blocks["qs"].astype(np.float64).reshape(rows, k // 32, 32)
    d = blocks["d"].view(np.float16).astype(np.float64).reshape(rows, k // 32, 1)
    return (q * d).reshape(rows, k)


def _stagewise(oracle, L, lay, s, os_, x, rows, kc_host, vc_host, positions, ctxs, kv_base,
               out):
    """kc_host/vc_host: fp16 caches after the call (GPU's), positions[t]:
    cache row of token t, ctxs[t]: its attention context, kv_base[t]: element
    offset of its cache."""
    torch = _torch()
    H, D = s.hidden, s.hdim
    QD, KVD, F = s.qheads * D, s.kvheads * D, s.ffn
    NQKV = QD + 2 * KVD
    # 1. RMSNorm -> Q8
    normed = _buf(L, "NORMED", rows * H, torch.float32).reshape(rows, H)
    want = np.stack([oracle.rmsnorm(x[t], lay["norm"]) for t in range(rows)])
    assert np.array_equal(normed.view(np.uint32), want.view(np.uint32)), "rmsnorm"
    xq = _q8_rows(L, "XQ", rows, H)
    assert xq.tobytes() == oracle.quantize_q8(normed).tobytes(), "input Q8"
    # 2. QKV projection (+bias) on the GPU's Q8
    qkv = _buf(L, "QKV", rows * NQKV, torch.float32).reshape(rows, NQKV)
    wqkv = np.concatenate([lay["wq"], lay["wk"], lay["wv"]])
    bias = np.concatenate([lay["bq"], lay["bk"], lay["bv"]]).astype(np.float64)
    want = _mm(_dequant_act(xq, rows, H), dequant_q4(wqkv, NQKV, H)) + bias
    _check_rows("qkv projection", qkv, want, 1e-5)
    # 3. RoPE + fp16 K/V append on the GPU's projections
    q = _buf(L, "Q", rows * QD, torch.float32).reshape(rows, QD)
    for t in range(rows):
        p = int(positions[t])
        wq = oracle.rope(qkv[t, :QD], s.qheads, D, p)
        wk = oracle.rope(qkv[t, QD:QD + KVD], s.kvheads, D, p)
        assert np.array_equal(q[t].view(np.uint32), wq.view(np.uint32)), f"rope q row {t}"
        base = int(kv_base[t]) + p * KVD
        assert np.array_equal(kc_host[base:base + KVD], oracle.f32_to_f16(wk)), f"K row {t}"
        assert np.array_equal(vc_host[base:base + KVD],
                              oracle.f32_to_f16(qkv[t, QD + KVD:])), f"V row {t}"
    # 4. attention over the GPU's cache, sampled rows (incl. every 63 mod 64)
    attn = _buf(L, "ATTN", rows * QD, torch.float32).reshape(rows, QD)
    sample = sorted({0, 1, rows - 1, rows // 2} | {t for t in range(63, rows, 64)})
    for t in sample:
        b = int(kv_base[t])
        want = oracle.attention_flash(os_, q[t], kc_host[b:], vc_host[b:], int(ctxs[t]))
        close(attn[t], want, 2e-3, f"attention row {t}")
    attq = _q8_rows(L, "ATTQ", rows, QD)
    assert attq.tobytes() == oracle.quantize_q8(attn).tobytes(), "attention Q8"
    # 5. W_O
    ao = _buf(L, "ATTN_OUT", rows * H, torch.float32).reshape(rows, H)
    want = _mm(_dequant_act(attq, rows, QD), dequant_q4(lay["wo"], H, QD))
    _check_rows("o projection", ao, want, 1e-5)
    # 6. residual + post-norm -> Q8
    h = _buf(L, "H", rows * H, torch.float32).reshape(rows, H)
    assert np.array_equal(h, x + ao), "residual 1"
    n2 = _buf(L, "NORMED2", rows * H, torch.float32).reshape(rows, H)
    want = np.stack([oracle.rmsnorm(h[t], lay["post_norm"]) for t in range(rows)])
    assert np.array_equal(n2.view(np.uint32), want.view(np.uint32)), "post-norm"
    xq2 = _q8_rows(L, "XQ2", rows, H)
    assert xq2.tobytes() == oracle.quantize_q8(n2).tobytes(), "post-norm Q8"
    # 7. gate|up, SwiGLU -> Q8
    gu = _buf(L, "GU", rows * 2 * F, torch.float32).reshape(rows, 2 * F)
    wgu = np.concatenate([lay["wgate"], lay["wup"]])
    want = _mm(_dequant_act(xq2, rows, H), dequant_q4(wgu, 2 * F, H))
    _check_rows("gate|up projection", gu, want, 1e-5)
    act = _buf(L, "ACT", rows * F, torch.float32).reshape(rows, F)
    want = np.stack([oracle.swiglu(gu[t, :F], gu[t, F:]) for t in range(rows)])
    _check_rows("swiglu", act, want, 1e-5)
    actq = _q8_rows(L, "ACTQ", rows, F)
    assert actq.tobytes() == oracle.quantize_q8(act).tobytes(), "swiglu Q8"
    # 8. down + residual
    want = h + _mm(_dequant_act(actq, rows, F), dequant_q4(lay["wdown"], H, F))
    _check_rows("down projection + residual", out, want, 1e-5)


@pytest.mark.parametrize("shape,ntok,prefix", [
    ("0.5b", 200, 30),    # ragged last tile, cached prefix; RoPE in the Q|K|V epilogue
    ("7b", 100, 7),       # the same fused epilogue at hdim 128
    ("7b", 2048, 0),      # BASELINE config 4 as the bench times it (default flags)
])
def test_prefill_stagewise(shape, ntok, prefix):
    """Causal prefill with the default (fast) flags: at 7B x 2048 this runs
    the 128-row gate|up GEMM with the fused SwiGLU + Q8 epilogue and the
    fast-epilogue QKV/O/down GEMMs the bench times."""
    from oracle.oracle_py import Oracle
    oracle = Oracle()
    torch = _torch()
    sd = si_amd.SHAPES[shape]
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    lay = make_layer(oracle, os_, 21)
    kvd = s.kvheads * s.hdim
    rng = np.random.default_rng(22)
    total = prefix + ntok
    x = rng.standard_normal((ntok, s.hidden)).astype(np.float32)
    kc0 = np.zeros(total * kvd, np.uint16)
    vc0 = np.zeros_like(kc0)
    kc0[:prefix * kvd] = kv_history(oracle, rng, prefix, kvd)
    vc0[:prefix * kvd] = kv_history(oracle, rng, prefix, kvd)
    L = si_amd.Layer(s, lay, ntok, total)
    kc, vc = dev(kc0.view(np.int16)), dev(vc0.view(np.int16))
    out = empty(ntok * s.hidden, torch.float32)
    L.prefill(dev(x), ntok, prefix, kc, vc, out)
    _stagewise(oracle, L, lay, s, os_, x, ntok, host(kc).view(np.uint16),
               host(vc).view(np.uint16), prefix + np.arange(ntok), prefix + 1 + np.arange(ntok),
               np.zeros(ntok, np.int64), host(out).reshape(ntok, s.hidden))
    L.close()


@pytest.mark.parametrize("nseq,ctx", [
    (70, 160),     # ragged 64-row tiles
    (64, 4096),    # BASELINE config 5 as the bench times it (default flags)
])
def test_batched_decode_stagewise_7b(nseq, ctx):
    """Batched decode with the default flags: the M = nseq GEMMs with their
    K-split plans, the split sums folded into the post-norm and SwiGLU
    kernels, and the whole-row batched decode attention."""
    from oracle.oracle_py import Oracle
    oracle = Oracle()
    torch = _torch()
    sd = si_amd.SHAPES["7b"]
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    lay = make_layer(oracle, os_, 23)
    kvd = s.kvheads * s.hdim
    stride = ctx * kvd
    rng = np.random.default_rng(24)
    x = rng.standard_normal((nseq, s.hidden)).astype(np.float32)
    kc0 = kv_history(oracle, rng, nseq * ctx, kvd)
    vc0 = kv_history(oracle, rng, nseq * ctx, kvd)
    L = si_amd.Layer(s, lay, nseq, ctx)
    kc, vc = dev(kc0.view(np.int16)), dev(vc0.view(np.int16))
    out = empty(nseq * s.hidden, torch.float32)
    L.decode_batch(dev(x), nseq, kc, vc, stride, ctx, ctx, out)
    _stagewise(oracle, L, lay, s, os_, x, nseq, host(kc).view(np.uint16),
               host(vc).view(np.uint16), np.full(nseq, ctx - 1), np.full(nseq, ctx),
               np.arange(nseq) * stride, host(out).reshape(nseq, s.hidden))
    L.close()


# Batched decode over ragged per-sequence contexts (ctx_dev), for every KV
# group count and head size the whole-row batched decode attention kernel
# serves (1, 2 or 4 groups; hdim 32..128; up to 16 query heads per group).
# Contexts fall on both sides of the 16-position tiles, the per-step rows and
# the context chunks, and include a context of 1.
_RAGGED = {
    "g1_d32": dict(hidden=256, qheads=8, kvheads=1, hdim=32, ffn=0),
    "0.5b": si_amd.SHAPES["0.5b"],
    "1.5b_ref": si_amd.SHAPES["1.5b_ref"],
    "g4_d96": dict(hidden=768, qheads=8, kvheads=4, hdim=96, ffn=0),
    "g1_d128_16heads": dict(hidden=2048, qheads=16, kvheads=1, hdim=128, ffn=0),
    "7b": si_amd.SHAPES["7b"],
}


_CTXS = {  # max_ctx -> contexts; 60 leaves one chunk (normalised in-kernel)
    333: [1, 2, 15, 16, 17, 63, 64, 65, 128, 129, 200, 331, 332, 333],
    60: [1, 2, 15, 16, 17, 31, 32, 33, 47, 48, 49, 58, 59, 60],
}


@pytest.mark.parametrize("max_ctx", list(_CTXS))
@pytest.mark.parametrize("name", list(_RAGGED))
def test_batched_decode_ragged_attention(name, max_ctx):
    from oracle.oracle_py import Oracle
    oracle = Oracle()
    torch = _torch()
    sd = _RAGGED[name]
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    lay = make_layer(oracle, os_, 31, ffn=s.ffn > 0)
    ctxs = np.array(_CTXS[max_ctx], np.int32)
    nseq = ctxs.size
    D, QD, KVD = s.hdim, s.qheads * s.hdim, s.kvheads * s.hdim
    stride = max_ctx * KVD
    rng = np.random.default_rng(32)
    x = rng.standard_normal((nseq, s.hidden)).astype(np.float32)
    kc0 = kv_history(oracle, rng, nseq * max_ctx, KVD)
    vc0 = kv_history(oracle, rng, nseq * max_ctx, KVD)
    L = si_amd.Layer(s, lay, nseq, max_ctx)
    kc, vc = dev(kc0.view(np.int16)), dev(vc0.view(np.int16))
    out = empty(nseq * s.hidden, torch.float32)
    flags = si_amd.SI_LAYER_FULL if s.ffn > 0 else si_amd.SI_LAYER_ATTN_ONLY
    L.decode_batch(dev(x), nseq, kc, vc, stride, 0, max_ctx, out, ctx_dev=dev(ctxs), flags=flags)
    kh, vh = host(kc).view(np.uint16), host(vc).view(np.uint16)
    NQKV = QD + 2 * KVD
    qkv = _buf(L, "QKV", nseq * NQKV, torch.float32).reshape(nseq, NQKV)
    q = _buf(L, "Q", nseq * QD, torch.float32).reshape(nseq, QD)
    attn = _buf(L, "ATTN", nseq * QD, torch.float32).reshape(nseq, QD)
    for t in range(nseq):
        p, b = int(ctxs[t]) - 1, t * stride
        assert np.array_equal(q[t].view(np.uint32),
                              oracle.rope(qkv[t, :QD], s.qheads, D, p).view(np.uint32)), t
        wk = oracle.f32_to_f16(oracle.rope(qkv[t, QD:QD + KVD], s.kvheads, D, p))
        assert np.array_equal(kh[b + p * KVD:b + (p + 1) * KVD], wk), f"K row of seq {t}"
        assert np.array_equal(vh[b + p * KVD:b + (p + 1) * KVD],
                              oracle.f32_to_f16(qkv[t, QD + KVD:])), f"V row of seq {t}"
        # the rest of the cache is untouched
        rest = np.r_[0:p * KVD, (p + 1) * KVD:stride]
        assert np.array_equal(kh[b:b + stride][rest], kc0[b:b + stride][rest]), t
        want = oracle.attention_flash(os_, q[t], kh[b:b + stride], vh[b:b + stride], int(ctxs[t]))
        close(attn[t], want, 2e-3, f"{name} attention seq {t} (context {ctxs[t]})")
    attq = _q8_rows(L, "ATTQ", nseq, QD)
    assert attq.tobytes() == oracle.quantize_q8(attn).tobytes(), "attention Q8"
    L.close()
