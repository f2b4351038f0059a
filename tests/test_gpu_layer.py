"""Layer-level GPU parity on the benchmark configurations (decode, batched
decode, causal prefill), the reference's prefill == sequential-decode
contract, and the C11 host mirror.  Rows are checked with the chained
oracle check (tests/chain.py); the raw end-to-end difference is printed."""
import ctypes
import os

import numpy as np
import pytest

import si_amd
from oracle.oracle_py import Q8_DTYPE, make_shape as or_shape
from tests.chain import E2E_BOUND, LayerBuffers, check_row, end_to_end_report
from tests.gpu_helpers import (close, dev, device_view, empty, host, kv_history, make_layer,
                               q8_tiled)

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_golden.npz")
EXACT = si_amd.SI_LAYER_EXACT


def _torch():
    import torch
    return torch


# Test-only shapes beside si_amd.SHAPES.  d128_small: hdim 128 with a
# hidden small enough (3 * 128 rows x 512 values = 110,592 B of Q4_0 per
# head) that single-token decode projects Q|K|V inside the attention kernel
# (the hdim-128 instances of the fused path), one KV group of 4 heads.
_TEST_SHAPES = {
    "d128_small": dict(hidden=512, qheads=4, kvheads=1, hdim=128, ffn=1024),
}


def _shapes(name):
    sd = _TEST_SHAPES.get(name) or si_amd.SHAPES[name]
    return si_amd.make_shape(**sd), or_shape(**sd)


@pytest.mark.parametrize("ctx", [1, 17, 64])
def test_attention_sublayer_reference_shape_golden(oracle, ctx):
    """run_layer at the reference's own 1.5B shape against the reference's
    outputs (golden fixture written from the reference build)."""
    from tests.golden.make_golden import layer_weights
    g = np.load(GOLDEN, allow_pickle=False)
    s, os_ = _shapes("1.5b_ref")
    lay = layer_weights(oracle, int(g["layer_seed"][0]), os_)
    L = si_amd.Layer(s, lay, 1, 64)
    torch = _torch()
    kvd = s.kvheads * s.hdim
    kc = dev(g[f"layer_kc_{ctx}"].view(np.int16))
    vc = dev(g[f"layer_vc_{ctx}"].view(np.int16))
    out = empty(s.hidden, torch.float32)
    L.decode(dev(g["layer_x"]), kc, vc, ctx, out, si_amd.SI_LAYER_ATTN_ONLY | EXACT)
    B = LayerBuffers(L, os_, 1)
    hk, hv = host(kc).view(np.uint16), host(vc).view(np.uint16)
    # the appended fp16 K/V rows equal the reference's (audit_fusion_timing.c:192-196)
    assert np.array_equal(hk[(ctx - 1) * kvd:], g[f"layer_newk_{ctx}"])
    assert np.array_equal(hv[(ctx - 1) * kvd:], g[f"layer_newv_{ctx}"])
    close(B.attn[0], g[f"layer_attn_{ctx}"], 2e-3, "attention vs reference")
    got = host(out)
    check_row(oracle, os_, lay, g["layer_x"], 0, B, hk, hv, 0, ctx - 1, ctx, got, True,
              full=False)
    close(got, g[f"layer_out_{ctx}"], 1e-3, "Y vs reference")
    L.close()


@pytest.mark.parametrize("flags", [si_amd.SI_LAYER_FULL, EXACT])
def test_decode_full_layer_0_5b_ctx1024(oracle, flags):
    """full 0.5B layer, one token at context 1024."""
    torch = _torch()
    s, os_ = _shapes("0.5b")
    lay = make_layer(oracle, os_, 2)
    ctx = 1024
    kvd = s.kvheads * s.hdim
    rng = np.random.default_rng(3)
    kc0 = kv_history(oracle, rng, ctx, kvd)
    vc0 = kv_history(oracle, rng, ctx, kvd)
    x = rng.standard_normal(s.hidden).astype(np.float32)
    L = si_amd.Layer(s, lay, 1, ctx)
    kc, vc = dev(kc0.view(np.int16)), dev(vc0.view(np.int16))
    out = empty(s.hidden, torch.float32)
    L.decode(dev(x), kc, vc, ctx, out, flags)
    B = LayerBuffers(L, os_, 1)
    hk, hv = host(kc).view(np.uint16), host(vc).view(np.uint16)
    assert np.array_equal(hk[:(ctx - 1) * kvd], kc0[:(ctx - 1) * kvd])  # history untouched
    got = host(out)
    check_row(oracle, os_, lay, x, 0, B, hk, hv, 0, ctx - 1, ctx, got, flags == EXACT)
    want = oracle.layer_decode(os_, lay, x, kc0.copy(), vc0.copy(), ctx)
    e2e = end_to_end_report(got, want)
    print("end-to-end vs oracle:", e2e)
    assert e2e["max_over_rms"] <= E2E_BOUND["0.5b"], e2e
    L.close()


@pytest.mark.parametrize("shape,ctx", [("0.5b", 1), ("0.5b", 2), ("0.5b", 16), ("0.5b", 17),
                                       ("0.5b", 129), ("0.5b", 500), ("0.5b", 5000), ("7b", 33),
                                       ("7b", 4096), ("d128_small", 1), ("d128_small", 17),
                                       ("d128_small", 300), ("d128_small", 2048),
                                       ("d128_small", 2100)])
def test_decode_contexts(oracle, shape, ctx):
    """Single-token decode over contexts that put the new token at every kind
    of place in the attention chunks (first tile, tile edge, last chunk); at
    0.5B 5000 and 7B 4096 the chunk partials exceed 32 KB and are merged once
    before W_O instead of inside it.  d128_small runs the hdim-128 fused
    Q|K|V + attention kernel up to 2048 positions (one and two tiles in
    flight) and the staged pair past them."""
    torch = _torch()
    s, os_ = _shapes(shape)
    lay = make_layer(oracle, os_, 40 + ctx)
    kvd = s.kvheads * s.hdim
    rng = np.random.default_rng(ctx)
    kc0 = kv_history(oracle, rng, ctx, kvd)
    vc0 = kv_history(oracle, rng, ctx, kvd)
    x = rng.standard_normal(s.hidden).astype(np.float32)
    L = si_amd.Layer(s, lay, 1, ctx)
    for flags in (si_amd.SI_LAYER_FULL, EXACT):
        kc, vc = dev(kc0.view(np.int16)), dev(vc0.view(np.int16))
        out = empty(s.hidden, torch.float32)
        ran = si_amd.kernel_times_ms("k_dec_attn", lambda: L.decode(dev(x), kc, vc, ctx, out,
                                                                    flags))
        if shape == "d128_small" and flags == si_amd.SI_LAYER_FULL:
            fused = [n for n, _ in ran if n.startswith("k_dec_attn<128,") and
                     n.endswith(", true>")]
            assert bool(fused) == (ctx <= 2048), f"ctx {ctx}: kernels {ran}"
        B = LayerBuffers(L, os_, 1)
        hk, hv = host(kc).view(np.uint16), host(vc).view(np.uint16)
        check_row(oracle, os_, lay, x, 0, B, hk, hv, 0, ctx - 1, ctx, host(out), flags == EXACT)
    L.close()


def test_shared_workspace_layers(oracle):
    """Layers created on one workspace give the same bits as layers with
    private workspaces, when their calls interleave."""
    torch = _torch()
    s, os_ = _shapes("0.5b")
    ctx = 300
    kvd = s.kvheads * s.hdim
    rng = np.random.default_rng(9)
    lays = [make_layer(oracle, os_, 70 + i) for i in range(2)]
    ws = si_amd.Workspace(s, 1, ctx)
    shared = [si_amd.Layer(s, lay, workspace=ws) for lay in lays]
    ws.close()  # the layers keep the workspace alive
    private = [si_amd.Layer(s, lay, 1, ctx) for lay in lays]
    caches = [(kv_history(oracle, rng, ctx, kvd), kv_history(oracle, rng, ctx, kvd))
              for _ in range(2)]
    x = rng.standard_normal(s.hidden).astype(np.float32)
    outs = {}
    for name, layers in (("shared", shared), ("private", private)):
        for rep in range(2):
            for i in (0, 1):
                kc, vc = (dev(c.view(np.int16)) for c in caches[i])
                out = empty(s.hidden, torch.float32)
                layers[i].decode(dev(x), kc, vc, ctx, out)
                outs[(name, rep, i)] = (host(out), host(kc), host(vc))
    for rep in range(2):
        for i in (0, 1):
            for a, b in zip(outs[("shared", rep, i)], outs[("private", rep, i)]):
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    for L in shared + private:
        L.close()


def _prefill_case(oracle, shape, ntok, prefix, seed, flags, rows):
    torch = _torch()
    s, os_ = _shapes(shape)
    lay = make_layer(oracle, os_, seed)
    kvd = s.kvheads * s.hdim
    rng = np.random.default_rng(seed + 1)
    total = prefix + ntok
    x = rng.standard_normal((ntok, s.hidden)).astype(np.float32)
    kc0 = np.zeros(total * kvd, np.uint16)
    vc0 = np.zeros_like(kc0)
    kc0[:prefix * kvd] = kv_history(oracle, rng, prefix, kvd)
    vc0[:prefix * kvd] = kv_history(oracle, rng, prefix, kvd)
    L = si_amd.Layer(s, lay, ntok, total)
    kc, vc = dev(kc0.view(np.int16)), dev(vc0.view(np.int16))
    out = empty(ntok * s.hidden, torch.float32)
    L.prefill(dev(x), ntok, prefix, kc, vc, out, flags)
    B = LayerBuffers(L, os_, ntok)
    hk, hv = host(kc).view(np.uint16), host(vc).view(np.uint16)
    got = host(out).reshape(ntok, s.hidden)
    for t in rows:
        check_row(oracle, os_, lay, x[t], t, B, hk, hv, 0, prefix + t, prefix + t + 1, got[t],
                  flags == EXACT)
    return L, s, os_, lay, x, kc0, vc0, hk, hv, got


@pytest.mark.parametrize("shape,ntok,prefix,rows,flags", [
    ("0.5b", 512, 0, [0, 1, 17, 63, 255, 511], EXACT),
    ("0.5b", 512, 0, [0, 63, 255, 511], si_amd.SI_LAYER_FULL),
    ("0.5b", 128, 0, [0, 127], si_amd.SI_LAYER_FULL),        # streaming one-tile GEMMs
    ("0.5b", 37, 100, [0, 36], EXACT),                      # ragged, cached prefix
])
def test_prefill_vs_oracle(oracle, shape, ntok, prefix, rows, flags):
    L, s, os_, lay, x, kc0, vc0, hk, hv, got = _prefill_case(oracle, shape, ntok, prefix, 4,
                                                             flags, rows)
    kr, vr = kc0.copy(), vc0.copy()
    want = oracle.layer_prefill(os_, lay, x, ntok, prefix, kr, vr, rows=rows)
    if flags == EXACT:
        # every appended K/V row equals the oracle's (prefill contract)
        assert np.array_equal(hk, kr) and np.array_equal(hv, vr)
    e2e = [end_to_end_report(got[t], want[i]) for i, t in enumerate(rows)]
    print("end-to-end vs oracle:", e2e)
    assert max(e["max_over_rms"] for e in e2e) <= E2E_BOUND[shape], e2e
    if flags != EXACT and ntok >= 128:
        # the down projection streamed the SwiGLU Q8 operand-tiled: that
        # copy holds the planar one's bytes
        torch = _torch()
        F, P = s.ffn, (ntok + 31) // 32
        qs = host(device_view(L.buffer("ACTQ_QS"), ntok * F, torch.int8).clone())
        d = host(device_view(L.buffer("ACTQ_D"), ntok * F // 32, torch.int16).clone())
        tq = host(device_view(L.buffer("ACTQ_TQ"), P * 32 * F, torch.int8).clone())
        td = host(device_view(L.buffer("ACTQ_TD"), P * F, torch.int16).clone())
        wq, wd = q8_tiled(qs, d.view(np.uint16), ntok, F)
        assert np.array_equal(tq, wq) and np.array_equal(td.view(np.uint16), wd)
    L.close()


@pytest.mark.parametrize("flags", [EXACT, si_amd.SI_LAYER_FULL])
def test_prefill_7b_2048_sampled_rows(oracle, flags):
    """7B layer, 2048-token causal prefill, in the
    reference's block order (EXACT) and with the fast kernels bench.py times
    (default flags: single-pass tile GEMMs for Q|K|V and O, a 5-way K split
    and reduce for down, the fused SwiGLU + Q8 gate|up instance)."""
    rows = [0, 1, 63, 1023, 2047]
    L, s, os_, lay, x, kc0, vc0, hk, hv, got = _prefill_case(oracle, "7b", 2048, 0, 5, flags,
                                                             rows)
    L.close()
    kr, vr = kc0.copy(), vc0.copy()
    want = oracle.layer_prefill(os_, lay, x, 2048, 0, kr, vr, rows=rows)
    if flags == EXACT:
        assert np.array_equal(hk, kr) and np.array_equal(hv, vr)
    e2e = [end_to_end_report(got[t], want[i]) for i, t in enumerate(rows)]
    print("end-to-end vs oracle:", e2e)
    assert max(e["max_over_rms"] for e in e2e) <= E2E_BOUND["7b"], e2e


@pytest.mark.parametrize("shape,ntok,prefix", [
    ("0.5b", 100, 45),      # hdim 64, 7 heads per KV group; ragged last tile
    ("7b", 70, 30),         # hdim 128, 7 heads per group
    ("1.5b_ref", 33, 0),    # hdim 128, 6 heads per group; one token past a tile
    ("0.5b", 1, 0),         # a single token
])
def test_prefill_attention_every_row(oracle, shape, ntok, prefix):
    """Causal prefill attention of every token of the batch (tiles of 32
    tokens, cached prefix rows) against attention_flash on the same q and
    cache, and its Q8_0 quantization bit-exact."""
    torch = _torch()
    s, os_ = _shapes(shape)
    lay = make_layer(oracle, os_, 21, ffn=False)
    kvd, QD = s.kvheads * s.hdim, s.qheads * s.hdim
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
    L.prefill(dev(x), ntok, prefix, kc, vc, out, si_amd.SI_LAYER_ATTN_ONLY)
    B = LayerBuffers(L, os_, ntok)
    hk, hv = host(kc).view(np.uint16), host(vc).view(np.uint16)
    for t in range(ntok):
        want = oracle.attention_flash(os_, B.q[t], hk, hv, prefix + t + 1)
        close(B.attn[t], want, 2e-3, f"row {t} attention")
        assert np.array_equal(B.attq[t].view(np.uint8),
                              oracle.quantize_q8(B.attn[t]).view(np.uint8)), f"row {t} Q8"
    assert QD == B.attn.shape[1]
    L.close()


def test_prefill_equals_sequential_decode(oracle):
    """bench_ai_dma_prefill.c:104-129: a prefill batch and a loop of
    single-token decodes leave bit-identical fp16 K/V for every position and
    agree on every output (EXACT projections)."""
    torch = _torch()
    s, os_ = _shapes("0.5b")
    lay = make_layer(oracle, os_, 11)
    ntok, prefix = 24, 9
    kvd = s.kvheads * s.hdim
    rng = np.random.default_rng(12)
    total = prefix + ntok
    x = rng.standard_normal((ntok, s.hidden)).astype(np.float32)
    k0 = np.zeros(total * kvd, np.uint16)
    v0 = np.zeros_like(k0)
    k0[:prefix * kvd] = kv_history(oracle, rng, prefix, kvd)
    v0[:prefix * kvd] = kv_history(oracle, rng, prefix, kvd)
    L = si_amd.Layer(s, lay, ntok, total)
    kp, vp = dev(k0.view(np.int16)), dev(v0.view(np.int16))
    yp = empty(ntok * s.hidden, torch.float32)
    L.prefill(dev(x), ntok, prefix, kp, vp, yp, EXACT)
    ks, vs = dev(k0.view(np.int16)), dev(v0.view(np.int16))
    ys = empty(ntok * s.hidden, torch.float32)
    xd = dev(x)
    for t in range(ntok):
        L.decode(xd[t], ks, vs, prefix + t + 1, ys[t * s.hidden:(t + 1) * s.hidden], EXACT)
    assert np.array_equal(host(kp), host(ks)) and np.array_equal(host(vp), host(vs))
    close(host(yp), host(ys), 1e-3, "prefill vs sequential decode")
    L.close()


@pytest.mark.parametrize("nseq,ctx,check,flags", [
    (4, 300, [0, 3], EXACT),
    (64, 4096, [0, 31, 63], EXACT),
    (64, 4096, [0, 31, 63], si_amd.SI_LAYER_FULL),  # the flags the bench times
])
def test_batched_decode_7b(oracle, nseq, ctx, check, flags):
    """BASELINE config 5 (64 sequences x 4096 positions) and a small variant;
    each sequence has its own contiguous cache."""
    torch = _torch()
    s, os_ = _shapes("7b")
    lay = make_layer(oracle, os_, 7)
    kvd = s.kvheads * s.hdim
    stride = ctx * kvd
    x = np.random.default_rng(8).standard_normal((nseq, s.hidden)).astype(np.float32)
    L = si_amd.Layer(s, lay, nseq, ctx)
    gen = torch.Generator(device="cuda").manual_seed(9)
    kc = torch.randn(nseq * stride, generator=gen, device="cuda").half().view(torch.int16)
    vc = torch.randn(nseq * stride, generator=gen, device="cuda").half().view(torch.int16)
    for i in check:
        rng = np.random.default_rng(100 + i)
        kc[i * stride:(i + 1) * stride] = dev(kv_history(oracle, rng, ctx, kvd).view(np.int16))
        vc[i * stride:(i + 1) * stride] = dev(kv_history(oracle, rng, ctx, kvd).view(np.int16))
    out = empty(nseq * s.hidden, torch.float32)
    L.decode_batch(dev(x), nseq, kc, vc, stride, ctx, ctx, out, flags=flags)
    B = LayerBuffers(L, os_, nseq)
    if flags != EXACT:
        # the down projection read the SwiGLU Q8 operand-tiled: that copy
        # holds the planar one's bytes (every row, padding zero)
        F, P = s.ffn, (nseq + 31) // 32
        qs = host(device_view(L.buffer("ACTQ_QS"), nseq * F, torch.int8).clone())
        d = host(device_view(L.buffer("ACTQ_D"), nseq * F // 32, torch.int16).clone())
        tq = host(device_view(L.buffer("ACTQ_TQ"), P * 32 * F, torch.int8).clone())
        td = host(device_view(L.buffer("ACTQ_TD"), P * F, torch.int16).clone())
        wq, wd = q8_tiled(qs, d.view(np.uint16), nseq, F)
        assert np.array_equal(tq, wq) and np.array_equal(td.view(np.uint16), wd)
    hk, hv = host(kc).view(np.uint16), host(vc).view(np.uint16)
    got = host(out).reshape(nseq, s.hidden)
    for i in check:
        check_row(oracle, os_, lay, x[i], i, B, hk, hv, i * stride, ctx - 1, ctx, got[i],
                  flags == EXACT)
        # the raw end-to-end difference on this sequence's own cache copy
        rng = np.random.default_rng(100 + i)
        k0, v0 = kv_history(oracle, rng, ctx, kvd), kv_history(oracle, rng, ctx, kvd)
        want = oracle.layer_decode(os_, lay, x[i], k0, v0, ctx)
        e2e = end_to_end_report(got[i], want)
        print(f"sequence {i} end-to-end vs oracle:", e2e)
        assert e2e["max_over_rms"] <= E2E_BOUND["7b"], e2e
    L.close()


def test_host_mirror_run_layer(oracle):
    """The C11 mirror (libsi_host.so run_layer) with captures."""
    from tests.golden.make_golden import layer_weights
    g = np.load(GOLDEN, allow_pickle=False)
    torch = _torch()
    s, os_ = _shapes("1.5b_ref")
    lay = layer_weights(oracle, int(g["layer_seed"][0]), os_)
    H = ctypes.CDLL(si_amd.HOST_SO)

    class Model(ctypes.Structure):
        _fields_ = [("shape", si_amd.Shape), ("layer", ctypes.c_void_p),
                    ("stream", ctypes.c_void_p), ("max_tokens", ctypes.c_int),
                    ("max_pos", ctypes.c_int), ("attn_ws", ctypes.c_void_p),
                    ("attn_ws_bytes", ctypes.c_size_t)]

    class Phase(ctypes.Structure):
        _fields_ = [(n, ctypes.c_float) for n in ("rms", "q8_input", "q_proj", "k_proj",
                                                  "v_proj", "rope_cache", "attention",
                                                  "q8_output", "out_proj")]

    H.si_model_from_host.restype = ctypes.POINTER(Model)
    H.si_model_from_host.argtypes = [ctypes.POINTER(si_amd.Shape),
                                     ctypes.POINTER(si_amd.LayerHost), ctypes.c_int, ctypes.c_int]
    H.run_layer.restype = Phase
    H.run_layer.argtypes = [ctypes.POINTER(Model)] + [ctypes.c_void_p] * 3 + \
        [ctypes.c_int, ctypes.c_void_p, ctypes.c_int] + [ctypes.c_void_p] * 3
    H.free_layer.argtypes = [ctypes.POINTER(Model)]
    keep = {k: np.ascontiguousarray(v) for k, v in lay.items() if v is not None}
    lh = si_amd.LayerHost(**{k: v.ctypes.data for k, v in keep.items()})
    m = H.si_model_from_host(ctypes.byref(s), ctypes.byref(lh), 1, 64)
    ctx = 17
    x = dev(g["layer_x"])
    for method in (1, 0):  # ATTENTION_FLASH, ATTENTION_STANDARD
        kc = dev(g[f"layer_kc_{ctx}"].view(np.int16))
        vc = dev(g[f"layer_vc_{ctx}"].view(np.int16))
        out = empty(s.hidden, torch.float32)
        attn = np.zeros(s.qheads * s.hdim, np.float32)
        q8 = np.zeros(s.qheads * s.hdim // 32, Q8_DTYPE)
        ph = H.run_layer(m, si_amd.ptr(x), si_amd.ptr(kc), si_amd.ptr(vc), ctx,
                         si_amd.ptr(out), method, None, attn.ctypes.data, q8.ctypes.data)
        close(host(out), g[f"layer_out_{ctx}"], 1e-3, f"mirror Y ({method})")
        close(attn, g[f"layer_attn_{ctx}"], 2e-3, f"mirror attention capture ({method})")
        # the captured Q8 is the quantization of the captured attention, bit-exact
        assert oracle.quantize_q8(attn).tobytes() == q8.tobytes()
        assert ph.q_proj > 0 and ph.attention > 0 and ph.out_proj > 0
        # the staged standard order times RoPE + K/V append on its own
        assert (ph.rope_cache > 0) == (method == 0)
    # attention_compute with both methods on the same q and cache
    H.attention_compute.argtypes = [ctypes.POINTER(Model), ctypes.c_int] + \
        [ctypes.c_void_p] * 3 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    rng = np.random.default_rng(9)
    q = rng.standard_normal(s.qheads * s.hdim).astype(np.float32)
    kh, vh = g[f"layer_kc_{ctx}"], g[f"layer_vc_{ctx}"]
    scores = empty(s.qheads * ctx, torch.float32)
    want = oracle.attention_standard(os_, q, kh, vh, ctx)
    qd, kd, vd = dev(q), dev(kh.view(np.int16)), dev(vh.view(np.int16))
    for method in (0, 1):
        o = empty(s.qheads * s.hdim, torch.float32)
        H.attention_compute(m, method, si_amd.ptr(qd), si_amd.ptr(kd), si_amd.ptr(vd), ctx,
                            si_amd.ptr(o), si_amd.ptr(scores))
        torch.cuda.synchronize()
        close(host(o), want, 2e-3, f"attention_compute({method})")
    H.free_layer(m)


@pytest.mark.parametrize("mode", ["decode", "decode_7b", "batch", "prefill"])
def test_capture_flag_leaves_outputs_unchanged(oracle, mode):
    """SI_LAYER_CAPTURE only adds the intermediate buffers: the layer output
    and the appended K/V rows are the same bits with and without it, and a
    call without it leaves the capture buffers untouched."""
    torch = _torch()
    name = "7b" if mode == "decode_7b" else "0.5b"
    s, os_ = _shapes(name)
    lay = make_layer(oracle, os_, 91)
    rng = np.random.default_rng(92)
    kvd = s.kvheads * s.hdim
    rows, ctx = {"decode": (1, 300), "decode_7b": (1, 700), "batch": (6, 150),
                 "prefill": (40, 40)}[mode]
    L = si_amd.Layer(s, lay, rows, ctx)
    x = dev(rng.standard_normal(rows * s.hidden).astype(np.float32))
    hist = kv_history(oracle, rng, rows * ctx, kvd)
    outs = []
    for capture in (True, False):
        kc = dev(hist.view(np.int16).copy())
        vc = dev(hist.view(np.int16)[::-1].copy())
        out = empty(rows * s.hidden, torch.float32)
        gu = si_amd_buffer(L, "GU", rows * 2 * s.ffn)
        gu.fill_(7.0)
        if mode.startswith("decode"):
            L.decode(x, kc, vc, ctx, out, capture=capture)
        elif mode == "batch":
            L.decode_batch(x, rows, kc, vc, ctx * kvd, ctx, ctx, out, capture=capture)
        else:
            L.prefill(x, rows, 0, kc, vc, out, capture=capture)
        torch.cuda.synchronize()
        if capture:
            assert not torch.all(gu == 7.0), "GU capture not written"
        else:
            assert torch.all(gu == 7.0), "GU written without SI_LAYER_CAPTURE"
        outs.append((host(out).view(np.uint32), host(kc), host(vc)))
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    L.close()


def si_amd_buffer(L, name, count):
    from tests.gpu_helpers import device_view
    return device_view(L.buffer(name), count, _torch().float32)
