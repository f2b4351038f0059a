"""The host mirror's remaining drop-ins (libsi_host.so, include/si_host.h) on
the GPU, against the oracle and the golden fixtures written from the
reference's own build:
  * matvec_q4q8 (row-major Q4_0, block_q8_0), rmsnorm, rope: bit-exact;
  * fused_column_matvec on column-SoA tiles: bit-exact, fresh and
    accumulating;
  * fused_attention_pair / si_attention_group: within 2e-3 of the oracle;
  * attention_wo_fused, run_layer_legacy_fused and run_layer_fused against
    the reference's run_layer_fused outputs, with the chained checks (new
    K/V rows bit-exact, Q8 capture = quantize_q8 of the attention capture,
    output = the oracle's W_O of that Q8, bit for bit)."""
import ctypes
import os

import numpy as np
import pytest

import si_amd
from oracle.oracle_py import Q8_DTYPE, make_shape as or_shape
from tests.gpu_helpers import close, dev, empty, host, kv_history, make_layer, q4

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_golden.npz")
_P, _I, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float


class Model(ctypes.Structure):
    """si_model_t (include/si_host.h)."""
    _fields_ = [("shape", si_amd.Shape), ("layer", _P), ("stream", _P), ("max_tokens", _I),
                ("max_pos", _I), ("attn_ws", _P), ("attn_ws_bytes", ctypes.c_size_t),
                ("rope_cos", _P), ("rope_sin", _P), ("norm", _P), ("bq", _P), ("bk", _P),
                ("bv", _P)]


class FusedWeights(ctypes.Structure):
    """fused_weights_t (include/si_host.h)."""
    _fields_ = [("q", _P), ("kv", _P), ("o", _P), ("q_bytes", ctypes.c_size_t),
                ("kv_bytes", ctypes.c_size_t), ("o_bytes", ctypes.c_size_t), ("normed", _P),
                ("kvpair", _P), ("qpair", _P), ("opair", _P), ("inq8", _P), ("oq", _P)]


class Phase(ctypes.Structure):
    _fields_ = [(n, _F) for n in ("rms", "q8_input", "q_proj", "k_proj", "v_proj",
                                  "rope_cache", "attention", "q8_output", "out_proj")]


class Stats(ctypes.Structure):
    _fields_ = [("phase", Phase), ("tcm_stage", ctypes.c_double)]


def _host():
    H = ctypes.CDLL(si_amd.HOST_SO)
    MP = ctypes.POINTER(Model)
    FP = ctypes.POINTER(FusedWeights)
    for name, res, args in (
            ("si_model_from_host", MP, [ctypes.POINTER(si_amd.Shape),
                                        ctypes.POINTER(si_amd.LayerHost), _I, _I]),
            ("free_layer", None, [MP]),
            ("matvec_q4q8", None, [_P, _P, _I, _I, _P, _P]),
            ("rmsnorm", None, [MP, _P, _P, _P]),
            ("rope", None, [MP, _P, _I, _I]),
            ("fused_column_matvec", None, [_P, _P, _I, _P, _P, _P, _I]),
            ("fused_attention_pair", None, [MP, _P, _P, _P, _I, _I, _P]),
            ("si_fused_weights_from_host", FusedWeights, [MP, _P, _P, _P]),
            ("fused_weights_free", None, [FP]),
            ("si_colsoa_bytes", ctypes.c_size_t, [ctypes.POINTER(si_amd.Shape), _I]),
            ("si_colsoa_repack_host", None, [ctypes.POINTER(si_amd.Shape),
                                             ctypes.POINTER(si_amd.LayerHost), _P, _P, _P]),
            ("attention_wo_fused", None, [MP, FP, _P, _P, _P, _I, _I, _I, _P,
                                          ctypes.POINTER(Stats), _P, _P]),
            ("run_layer_legacy_fused", Stats, [MP, FP, _P, _P, _P, _I, _P, _P, _P]),
            ("run_layer_fused", Stats, [MP, FP, _P, _P, _P, _I, _P, _P, _P])):
        f = getattr(H, name)
        f.restype, f.argtypes = res, args
    return H


def _torch():
    import torch
    return torch


class _Mirror:
    """A loaded layer of the host mirror (si_model_t) and its tensors."""

    def __init__(self, shape_dict, lay, max_pos):
        self.H = _host()
        self.s = si_amd.make_shape(**shape_dict)
        self.keep = {k: np.ascontiguousarray(v) for k, v in lay.items() if v is not None}
        self.lh = si_amd.LayerHost(**{k: v.ctypes.data for k, v in self.keep.items()})
        self.m = self.H.si_model_from_host(ctypes.byref(self.s), ctypes.byref(self.lh), 1,
                                           max_pos)

    def fused_weights(self):
        """Column-SoA tiles from the product's host repacker, on the device."""
        s = self.s
        bufs = [np.zeros(self.H.si_colsoa_bytes(ctypes.byref(s), i), np.uint8) for i in range(3)]
        self.H.si_colsoa_repack_host(ctypes.byref(s), ctypes.byref(self.lh),
                                     *[b.ctypes.data for b in bufs])
        return self.H.si_fused_weights_from_host(self.m, *[b.ctypes.data for b in bufs]), bufs

    def close(self):
        self.H.free_layer(self.m)


def _golden():
    return np.load(GOLDEN, allow_pickle=False)


REF = dict(si_amd.SHAPES["1.5b_ref"])


@pytest.mark.parametrize("n,k,bias", [(64, 256, True), (1152, 896, True), (9728, 896, False),
                                      (3584, 18944, False)])
def test_matvec_q4q8_rowmajor_bit_exact(oracle, n, k, bias):
    torch = _torch()
    H = _host()
    rng = np.random.default_rng(n + k)
    w = q4(oracle, rng, n, k)
    xq = oracle.quantize_q8(rng.standard_normal(k).astype(np.float32))
    b = rng.normal(0, 0.02, n).astype(np.float32) if bias else None
    out = empty(n, torch.float32)
    H.matvec_q4q8(si_amd.ptr(dev(w)), si_amd.ptr(dev(xq.view(np.uint8))), k, n,
                  si_amd.ptr(None if b is None else dev(b)), si_amd.ptr(out))
    want = oracle.matvec(w, xq, k, n, b)
    assert np.array_equal(host(out).view(np.uint32), want.view(np.uint32))


def test_matvec_q4q8_golden():
    torch = _torch()
    g = _golden()
    out = empty(64, torch.float32)
    _host().matvec_q4q8(si_amd.ptr(dev(g["mv_w"])), si_amd.ptr(dev(g["mv_xq"])), 256, 64,
                        si_amd.ptr(dev(g["mv_b"])), si_amd.ptr(out))
    assert np.array_equal(host(out).view(np.uint32), g["mv_out"].view(np.uint32))


def test_rmsnorm_and_rope_golden(oracle):
    """rmsnorm and rope at the reference's shape against its own outputs
    (positions up to 32767, the table's last row)."""
    torch = _torch()
    g = _golden()
    lay = make_layer(oracle, or_shape(**REF), 3, ffn=False)
    M = _Mirror(REF, lay, 32768)
    out = empty(1536, torch.float32)
    M.H.rmsnorm(M.m, si_amd.ptr(dev(g["rms_in"])), si_amd.ptr(dev(g["rms_w"])), si_amd.ptr(out))
    assert np.array_equal(host(out).view(np.uint32), g["rms_out"].view(np.uint32))
    for pos, want in zip(g["rope_pos"], g["rope_out"]):
        h = dev(g["rope_in"])
        M.H.rope(M.m, si_amd.ptr(h), 12, int(pos))
        assert np.array_equal(host(h).view(np.uint32), want.view(np.uint32)), pos
    # and random rows against the oracle
    rng = np.random.default_rng(4)
    for scale in (1e-3, 1.0, 300.0):
        x = (rng.standard_normal(1536) * scale).astype(np.float32)
        w = rng.normal(1, 0.1, 1536).astype(np.float32)
        M.H.rmsnorm(M.m, si_amd.ptr(dev(x)), si_amd.ptr(dev(w)), si_amd.ptr(out))
        assert np.array_equal(host(out).view(np.uint32), oracle.rmsnorm(x, w).view(np.uint32)), \
            f"rmsnorm x{scale}"
    M.close()


def test_fused_column_matvec_golden_and_oracle(oracle):
    torch = _torch()
    g = _golden()
    H = _host()
    out = empty(256, torch.float32)
    bias = dev(g["fcm_bias"])
    tile, xq = dev(g["fcm_tile"]), dev(g["fcm_xq"])
    H.fused_column_matvec(si_amd.ptr(tile), si_amd.ptr(xq), 8, si_amd.ptr(bias),
                          ctypes.c_void_p(bias.data_ptr() + 512), si_amd.ptr(out), 0)
    assert np.array_equal(host(out).view(np.uint32), g["fcm_out"].view(np.uint32))
    H.fused_column_matvec(si_amd.ptr(tile), si_amd.ptr(xq), 8, None, None, si_amd.ptr(out), 1)
    assert np.array_equal(host(out).view(np.uint32), g["fcm_out_add"].view(np.uint32))
    # a 48-block tile of a real layer, without bias
    rng = np.random.default_rng(8)
    lay = make_layer(oracle, or_shape(**REF), 9, ffn=False)
    qt, _, _ = oracle.colsoa_repack(or_shape(**REF), lay)
    xq = oracle.quantize_q8(rng.standard_normal(1536).astype(np.float32))
    t1 = qt[5120 * 48:5120 * 96]
    H.fused_column_matvec(si_amd.ptr(dev(t1)), si_amd.ptr(dev(xq.view(np.uint8))), 48, None,
                          None, si_amd.ptr(out), 0)
    want = oracle.fused_column_matvec(t1, xq, 48)
    assert np.array_equal(host(out).view(np.uint32), want.view(np.uint32))


def test_product_colsoa_repacker_matches_oracle(oracle):
    """si_colsoa_repack_host (product, C) writes the oracle's bytes, which
    the reference build pins."""
    lay = make_layer(oracle, or_shape(**REF), 12, ffn=False)
    M = _Mirror(REF, lay, 64)
    fw, bufs = M.fused_weights()
    for got, want in zip(bufs, oracle.colsoa_repack(or_shape(**REF), lay)):
        assert np.array_equal(got, want)
    M.H.fused_weights_free(ctypes.byref(fw))
    M.close()


@pytest.mark.parametrize("ctx", [1, 17, 300, 4097])
def test_fused_attention_pair(oracle, ctx):
    torch = _torch()
    lay = make_layer(oracle, or_shape(**REF), 13, ffn=False)
    M = _Mirror(REF, lay, ctx)
    os_ = or_shape(**REF)
    rng = np.random.default_rng(ctx)
    kvd = 256
    kc, vc = kv_history(oracle, rng, ctx, kvd), kv_history(oracle, rng, ctx, kvd)
    kd, vd = dev(kc.view(np.int16)), dev(vc.view(np.int16))
    for group in range(2):
        qpair = rng.standard_normal(256).astype(np.float32)
        o = empty(256, torch.float32)
        M.H.fused_attention_pair(M.m, si_amd.ptr(dev(qpair)), si_amd.ptr(kd), si_amd.ptr(vd),
                                 ctx, group, si_amd.ptr(o))
        close(host(o), oracle.attention_pair(os_, qpair, kc, vc, ctx, group), 2e-3,
              f"pair attention group {group}")
    M.close()


@pytest.mark.parametrize("nheads", [1, 3, 7])
def test_attention_group_7b(oracle, nheads):
    """si_attention_group (C ABI): a KV group's query heads over the 7B cache
    layout against attention_flash's heads of that group."""
    torch = _torch()
    s = si_amd.make_shape(**si_amd.SHAPES["7b"])
    os_ = or_shape(**si_amd.SHAPES["7b"])
    ctx, group = 1000, 2
    rng = np.random.default_rng(nheads)
    kvd = 512
    kc, vc = kv_history(oracle, rng, ctx, kvd), kv_history(oracle, rng, ctx, kvd)
    q = rng.standard_normal(28 * 128).astype(np.float32)
    want = oracle.attention_flash(os_, q, kc, vc, ctx).reshape(28, 128)
    h0 = group * 7
    wsb = si_amd.lib().si_attention_group_workspace(ctypes.byref(s), nheads, ctx)
    ws = empty(wsb, torch.uint8)
    out = empty(nheads * 128, torch.float32)
    si_amd.call("si_attention_group", ctypes.byref(s), si_amd.ptr(dev(q[h0 * 128:(h0 + nheads) * 128])),
                nheads, group, si_amd.ptr(dev(kc.view(np.int16))), si_amd.ptr(dev(vc.view(np.int16))),
                ctx, si_amd.ptr(out), si_amd.ptr(ws), wsb, None)
    close(host(out), want[h0:h0 + nheads].reshape(-1), 2e-3, "group attention")


def _golden_layer(oracle):
    from tests.golden.make_golden import layer_weights
    g = _golden()
    return g, layer_weights(oracle, int(g["layer_seed"][0]), or_shape(**REF))


@pytest.mark.parametrize("ctx", [1, 17, 64])
def test_run_layer_legacy_fused_golden(oracle, ctx):
    torch = _torch()
    g, lay = _golden_layer(oracle)
    M = _Mirror(REF, lay, 64)
    fw, _ = M.fused_weights()
    kvd = 256
    kc, vc = dev(g[f"layer_kc_{ctx}"].view(np.int16)), dev(g[f"layer_vc_{ctx}"].view(np.int16))
    out = empty(1536, torch.float32)
    att = np.zeros(1536, np.float32)
    q8 = np.zeros(48, Q8_DTYPE)
    st = M.H.run_layer_legacy_fused(M.m, ctypes.byref(fw), si_amd.ptr(dev(g["layer_x"])),
                                    si_amd.ptr(kc), si_amd.ptr(vc), ctx, si_amd.ptr(out),
                                    att.ctypes.data, q8.ctypes.data)
    hk, hv = host(kc).view(np.uint16), host(vc).view(np.uint16)
    # the projections run in the reference's order and roundings: the new
    # fp16 K/V rows are the reference's bits
    assert np.array_equal(hk[(ctx - 1) * kvd:], g[f"fused_newk_{ctx}"])
    assert np.array_equal(hv[(ctx - 1) * kvd:], g[f"fused_newv_{ctx}"])
    close(att, g[f"fused_attn_{ctx}"], 2e-3, "attention capture vs reference")
    assert oracle.quantize_q8(att).tobytes() == q8.tobytes(), "Q8 capture"
    y = host(out)
    # W_O in head-pair order is matvec_q4q8's block order: bit-exact on the
    # GPU's own Q8
    want = oracle.matvec(lay["wo"], q8, 1536, 1536)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), "W_O on the Q8 capture"
    close(y, g[f"fused_out_{ctx}"], 1e-3, "Y vs the reference's run_layer_fused")
    ph = st.phase
    assert ph.q_proj > 0 and ph.k_proj > 0 and ph.attention > 0 and ph.out_proj > 0
    M.H.fused_weights_free(ctypes.byref(fw))
    M.close()


@pytest.mark.parametrize("ctx", [1, 17, 64])
def test_run_layer_fused_golden(oracle, ctx):
    """run_layer_fused (the fused decode kernels) against the reference's
    run_layer_fused outputs; its Q8 capture is the quantization of its
    attention capture and its output the oracle's W_O of that Q8."""
    torch = _torch()
    g, lay = _golden_layer(oracle)
    M = _Mirror(REF, lay, 64)
    fw, _ = M.fused_weights()
    kvd = 256
    for fwp in (ctypes.byref(fw), None):
        kc = dev(g[f"layer_kc_{ctx}"].view(np.int16))
        vc = dev(g[f"layer_vc_{ctx}"].view(np.int16))
        out = empty(1536, torch.float32)
        att = np.zeros(1536, np.float32)
        q8 = np.zeros(48, Q8_DTYPE)
        M.H.run_layer_fused(M.m, fwp, si_amd.ptr(dev(g["layer_x"])), si_amd.ptr(kc),
                            si_amd.ptr(vc), ctx, si_amd.ptr(out), att.ctypes.data,
                            q8.ctypes.data)
        hk, hv = host(kc).view(np.uint16), host(vc).view(np.uint16)
        close(oracle.f16_to_f32(hk[(ctx - 1) * kvd:]),
              oracle.f16_to_f32(g[f"fused_newk_{ctx}"]), 2e-3, "new K row")
        close(oracle.f16_to_f32(hv[(ctx - 1) * kvd:]),
              oracle.f16_to_f32(g[f"fused_newv_{ctx}"]), 2e-3, "new V row")
        close(att, g[f"fused_attn_{ctx}"], 2e-3, "attention capture")
        assert oracle.quantize_q8(att).tobytes() == q8.tobytes(), "Q8 capture"
        y = host(out)
        close(y, oracle.matvec(lay["wo"], q8, 1536, 1536), 1e-5, "W_O on the Q8 capture")
        close(y, g[f"fused_out_{ctx}"], 1e-3, "Y vs the reference's run_layer_fused")
    M.H.fused_weights_free(ctypes.byref(fw))
    M.close()


def test_attention_wo_fused_accumulates(oracle):
    """attention_wo_fused adds one pair's W_O partial into an existing
    output: the result is the start value plus the oracle's column-SoA W_O
    of the pair's Q8 capture, bit for bit."""
    torch = _torch()
    lay = make_layer(oracle, or_shape(**REF), 21, ffn=False)
    os_ = or_shape(**REF)
    M = _Mirror(REF, lay, 200)
    fw, (qt, kvt, ot) = M.fused_weights()
    rng = np.random.default_rng(22)
    ctx, kvd, group, pair = 150, 256, 1, 4
    kc, vc = kv_history(oracle, rng, ctx, kvd), kv_history(oracle, rng, ctx, kvd)
    qpair = rng.standard_normal(256).astype(np.float32)
    y0 = rng.standard_normal(1536).astype(np.float32)
    y = dev(y0)
    att = np.zeros(1536, np.float32)
    q8 = np.zeros(48, Q8_DTYPE)
    st = Stats()
    M.H.attention_wo_fused(M.m, ctypes.byref(fw), si_amd.ptr(dev(qpair)),
                           si_amd.ptr(dev(kc.view(np.int16))), si_amd.ptr(dev(vc.view(np.int16))),
                           ctx, group, pair, si_amd.ptr(y), ctypes.byref(st), att.ctypes.data,
                           q8.ctypes.data)
    a = att[pair * 256:(pair + 1) * 256]
    close(a, oracle.attention_pair(os_, qpair, kc, vc, ctx, group), 2e-3, "pair attention")
    oq = q8[pair * 8:(pair + 1) * 8]
    assert oracle.quantize_q8(a).tobytes() == oq.tobytes()
    want = y0.copy()
    sub = 8 * 5120
    for t in range(6):
        base = (pair * 6 + t) * sub
        want[t * 256:(t + 1) * 256] = oracle.fused_column_matvec(
            ot[base:base + sub], oq, 8, out=want[t * 256:(t + 1) * 256], add=True)
    assert np.array_equal(host(y).view(np.uint32), want.view(np.uint32))
    assert st.phase.attention > 0 and st.phase.out_proj > 0
    M.H.fused_weights_free(ctypes.byref(fw))
    M.close()
