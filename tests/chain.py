"""Chained parity check of one layer row against the oracle.

A quantized layer is ill-conditioned at its re-quantization points: a change
of a few 1e-6 in the attention output can move a 7B layer's output by 1e-2
(shown on the oracle alone in test_oracle_sensitivity.py).  So the layer is
checked as a chain, each link on identical inputs:

  1. input RMSNorm -> Q8 bit-exact in every mode; Q/K/V projections,
     RoPE, fp16 K/V rows: bit-exact in SI_LAYER_EXACT mode (fp32 rounding
     otherwise);
  2. attention on those inputs: within 2e-3 of attention_flash;
  3. the rest of the layer, recomputed by the oracle from the GPU's
     attention output: within 1e-3 of the GPU's layer output;
  4. every later stage on the GPU's own inputs: RMSNorm, quantizers and
     (EXACT) projections bit-exact, SwiGLU within 1e-6 (device expf vs
     libm).
"""
import numpy as np

from oracle.oracle_py import QK
from tests.gpu_helpers import close, device_view, host, planar_to_aos


def _torch():
    import torch
    return torch


class LayerBuffers:
    """Host copies of a layer's workspace buffers after a call."""

    def __init__(self, L, s, rows):
        torch = _torch()
        H, QD, KVD, F = s.hidden, s.qheads * s.hdim, s.kvheads * s.hdim, s.ffn
        NQKV = QD + 2 * KVD

        def f32(name, n):
            return host(device_view(L.buffer(name), rows * n, torch.float32).clone()).reshape(rows, n)

        def q8(prefix, n):
            qs = host(device_view(L.buffer(prefix + "_QS"), rows * n, torch.int8).clone())
            d = host(device_view(L.buffer(prefix + "_D"), rows * n // QK, torch.int16).clone())
            return planar_to_aos(qs, d.view(np.uint16)).reshape(rows, n // QK)

        self.normed, self.xq = f32("NORMED", H), q8("XQ", H)
        self.qkv, self.q = f32("QKV", NQKV), f32("Q", QD)
        self.attn, self.attq = f32("ATTN", QD), q8("ATTQ", QD)
        self.attn_out = f32("ATTN_OUT", H)
        if F:
            self.h, self.normed2, self.xq2 = f32("H", H), f32("NORMED2", H), q8("XQ2", H)
            self.gu, self.act, self.actq = f32("GU", 2 * F), f32("ACT", F), q8("ACTQ", F)


def _eq(a, b, what):
    assert np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8)), what


def check_row(oracle, os_, lay, x, t, B, kc_gpu, vc_gpu, base, pos, ctx, out_row, exact,
              full=True):
    """Chained check of row t (see module doc).  kc_gpu/vc_gpu: host copies of
    the device caches after the call; base: element offset of this row's
    cache; pos: its cache row; ctx: its attention context."""
    s = os_
    H, D = s.hidden, s.hdim
    QD, KVD, F = s.qheads * D, s.kvheads * D, s.ffn
    tag = f"row {t}"
    # 1. front half on identical input
    normed = oracle.rmsnorm(x, lay["norm"])
    _eq(B.normed[t], normed, tag + " rmsnorm")
    _eq(B.xq[t], oracle.quantize_q8(B.normed[t]), tag + " input Q8")
    xq = B.xq[t]
    q = oracle.matvec(lay["wq"], xq, H, QD, lay["bq"])
    k = oracle.matvec(lay["wk"], xq, H, KVD, lay["bk"])
    v = oracle.matvec(lay["wv"], xq, H, KVD, lay["bv"])
    q = oracle.rope(q, s.qheads, D, pos)
    k = oracle.rope(k, s.kvheads, D, pos)
    row = slice(base + pos * KVD, base + (pos + 1) * KVD)
    if exact:
        _eq(B.q[t], q, tag + " q")
        _eq(kc_gpu[row], oracle.f32_to_f16(k), tag + " new K row")
        _eq(vc_gpu[row], oracle.f32_to_f16(v), tag + " new V row")
    else:
        close(B.q[t], q, 1e-5, tag + " q")
        close(oracle.f16_to_f32(kc_gpu[row]), oracle.f16_to_f32(oracle.f32_to_f16(k)), 2e-3,
              tag + " new K row")
    # 2. attention on the same q and cache
    attn = oracle.attention_flash(s, B.q[t], kc_gpu[base:], vc_gpu[base:], ctx)
    close(B.attn[t], attn, 2e-3, tag + " attention")
    # 3. the oracle continued from the GPU's attention output
    attq = oracle.quantize_q8(B.attn[t])
    _eq(B.attq[t], attq, tag + " attention Q8")
    ao = oracle.matvec(lay["wo"], attq, QD, H)
    if not full:
        close(out_row, ao, 1e-3, tag + " W_O output (continued)")
        if exact:
            _eq(out_row, ao, tag + " W_O output")
        return
    h = x + ao
    n2 = oracle.rmsnorm(h, lay["post_norm"])
    xq2 = oracle.quantize_q8(n2)
    g = oracle.matvec(lay["wgate"], xq2, H, F)
    u = oracle.matvec(lay["wup"], xq2, H, F)
    y = h + oracle.matvec(lay["wdown"], oracle.quantize_q8(oracle.swiglu(g, u)), F, H)
    close(out_row, y, 1e-3, tag + " layer output (continued from GPU attention)")
    # 4. later stages on the GPU's own inputs
    if exact:
        _eq(B.attn_out[t], ao, tag + " W_O")
        _eq(B.h[t], x + B.attn_out[t], tag + " residual")
    _eq(B.normed2[t], oracle.rmsnorm(B.h[t], lay["post_norm"]), tag + " post-norm")
    _eq(B.xq2[t], oracle.quantize_q8(B.normed2[t]), tag + " post-norm Q8")
    gu = np.concatenate([oracle.matvec(lay["wgate"], B.xq2[t], H, F),
                         oracle.matvec(lay["wup"], B.xq2[t], H, F)])
    if exact:
        _eq(B.gu[t], gu, tag + " gate|up")
    else:
        close(B.gu[t], gu, 1e-5, tag + " gate|up")
    close(B.act[t], oracle.swiglu(B.gu[t, :F], B.gu[t, F:]), 1e-6, tag + " SwiGLU")
    _eq(B.actq[t], oracle.quantize_q8(B.act[t]), tag + " SwiGLU Q8")
    down = B.h[t] + oracle.matvec(lay["wdown"], B.actq[t], F, H)
    if exact:
        _eq(out_row, down, tag + " down + residual")
    else:
        close(out_row, down, 1e-5, tag + " down + residual")


# Asserted bound on the raw (unchained) end-to-end difference of a layer
# output from the oracle's, as max|got - want| / rms(want).  The chained
# check above is the parity bar; this loose bound catches a regression that
# moves every link while keeping each inside its own tolerance.  The 7B layer
# amplifies a 2e-5 change of its attention output to ~3e-3 at its outputs
# (test_oracle_sensitivity.py), so its bound is wider.
E2E_BOUND = {"0.5b": 2e-3, "1.5b_ref": 2e-3, "7b": 2e-2}


def end_to_end_report(got, want):
    """Statistics of the raw (unchained) difference, for reporting."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    return dict(max_over_rms=float(np.abs(got - want).max() / rms),
                norm_rel=float(np.linalg.norm(got - want) / np.linalg.norm(want)))
