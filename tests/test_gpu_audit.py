"""The reference's independent validation cases on the GPU layer
(audit_fusion_timing.c:133-206): five fresh tokens and K/V histories at
contexts {1, 2, 17, 64, max}, with adversarial tokens (alternating
+-(0.125+|r|); 0.8 spikes on every 13th element over 0.1-scaled noise) and K
history scales {0.25, 0.0125, 1, 0, 0.5}.  Each case runs through
si_layer_decode and passes the chained oracle check (tests/chain.py); the
attention outputs must change from case to case (the audit's dead-path check,
:201-206), the appended K/V rows are the oracle's bits, and the raw
end-to-end difference from the oracle's layer is bounded."""
import ctypes

import numpy as np
import pytest

import si_amd
from oracle.oracle_py import make_shape as or_shape
from tests.chain import E2E_BOUND, LayerBuffers, check_row, end_to_end_report
from tests.gpu_helpers import dev, empty, host, make_layer

pytestmark = pytest.mark.gpu

LENGTHS = (1, 2, 17, 64)           # then max_context (audit_fusion_timing.c:142)
KMUL = (0.25, 0.0125, 1.0, 0.0, 0.5)  # :152-156


class _Stream:
    """The reference's xorshift32 stream (qwen_one_layer.c:88-96), continued
    across cases as the audit's calls to random_float() are."""

    def __init__(self, oracle, seed=0x5217ac8b):
        self.lib = oracle.lib
        self.lib.or_rng_float.restype = ctypes.c_float
        self.lib.or_rng_seed(seed)

    def floats(self, n):
        out = np.empty(n, np.float32)
        self.lib.or_rng_fill(out.ctypes.data_as(ctypes.c_void_p), n, ctypes.c_float(1.0))
        return out


def _token(trial, r):
    """audit_fusion_timing.c:146-150."""
    i = np.arange(r.size)
    if trial == 1:
        return np.where(i & 1, np.float32(-0.125) - np.abs(r),
                        np.float32(0.125) + np.abs(r)).astype(np.float32)
    if trial == 3:
        return np.where(i % 13 == 0, np.float32(0.8), r * np.float32(0.1)).astype(np.float32)
    return r


@pytest.mark.parametrize("shape,max_ctx", [("0.5b", 1024), ("7b", 4096)])
@pytest.mark.parametrize("flags", [si_amd.SI_LAYER_FULL, si_amd.SI_LAYER_EXACT,
                                   si_amd.SI_LAYER_ATTN_ONLY])
def test_audit_validation_cases(oracle, shape, max_ctx, flags):
    import torch
    sd = si_amd.SHAPES[shape]
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    H, KVD = s.hidden, s.kvheads * s.hdim
    full = not (flags & si_amd.SI_LAYER_ATTN_ONLY)
    exact = bool(flags & si_amd.SI_LAYER_EXACT)
    lay = make_layer(oracle, os_, 900 + H, ffn=full)
    L = si_amd.Layer(s, lay, 1, max_ctx)
    rng = _Stream(oracle)
    previous, distinct = None, 0
    for trial, length in enumerate(LENGTHS + (max_ctx,)):
        ctx = min(length, max_ctx)
        x = _token(trial, rng.floats(H))
        # :158-162: K = f16(r * kmul), V = f16(r' * 0.25), interleaved draws
        hist = rng.floats(2 * (ctx - 1) * KVD).reshape(-1, 2) if ctx > 1 else np.zeros((0, 2),
                                                                                          np.float32)
        kc0 = np.zeros(ctx * KVD, np.uint16)
        vc0 = np.zeros(ctx * KVD, np.uint16)
        kc0[:(ctx - 1) * KVD] = oracle.f32_to_f16(hist[:, 0] * np.float32(KMUL[trial]))
        vc0[:(ctx - 1) * KVD] = oracle.f32_to_f16(hist[:, 1] * np.float32(0.25))
        kc, vc = dev(kc0.view(np.int16)), dev(vc0.view(np.int16))
        out = empty(H, torch.float32)
        L.decode(dev(x), kc, vc, ctx, out, flags)
        B = LayerBuffers(L, os_, 1)
        hk, hv = host(kc).view(np.uint16), host(vc).view(np.uint16)
        got = host(out)
        tag = f"case {trial + 1} (context {ctx}, K scale {KMUL[trial]})"
        assert np.array_equal(hk[:(ctx - 1) * KVD], kc0[:(ctx - 1) * KVD]), tag + " K history"
        check_row(oracle, os_, lay, x, 0, B, hk, hv, 0, ctx - 1, ctx, got, exact, full=full)
        if full:
            want = oracle.layer_decode(os_, lay, x, kc0.copy(), vc0.copy(), ctx)
        else:
            want = oracle.run_layer(os_, lay, x, kc0.copy(), vc0.copy(), ctx)
        e2e = end_to_end_report(got, want)
        assert e2e["max_over_rms"] <= E2E_BOUND[shape], f"{tag}: end-to-end {e2e}"
        attn = B.attn[0].copy()
        if trial and not np.array_equal(attn.view(np.uint32), previous.view(np.uint32)):
            distinct += 1
        previous = attn
    # :201-206: identical attention for every input means a dead path
    assert distinct == len(LENGTHS), f"only {distinct} of {len(LENGTHS)} cases changed the output"
    L.close()
