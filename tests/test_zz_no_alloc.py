"""si_attention_static, the allocation-free variant of si_attention (its
partial states in a fixed device buffer of the library), against
si_attention with a caller workspace, through the C ABI: bit-identical
outputs (attention, Q8 values, scales, block sums) on consecutive calls of
decreasing size over the two schedules (causal-prefill flash kernel,
split-context decode kernels), and a refused oversize call that launches
nothing."""
import ctypes

import numpy as np
import pytest

import si_amd
from tests.gpu_helpers import dev, empty, host, zeros

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    return torch


def _cache(rng, rows, kvd):
    return rng.standard_normal(rows * kvd).astype(np.float16).view(np.int16)


def _run_both(s, q, nq, kc, vc, stride, ctx_dev, ctx0, ctx_step, max_ctx):
    """(static outputs, workspace outputs) as host arrays."""
    torch = _torch()
    qd = s.qheads * s.hdim
    outs = []
    for static in (True, False):
        attn = zeros(nq * qd, torch.float32)
        qs, d = zeros(nq * qd, torch.int8), zeros(nq * qd // 32, torch.int16)
        bsum = zeros(nq * qd // 32, torch.int16)
        args = (ctypes.byref(s), si_amd.ptr(q), nq, si_amd.ptr(kc), si_amd.ptr(vc), stride,
                si_amd.ptr(ctx_dev), ctx0, ctx_step, max_ctx, si_amd.ptr(attn), si_amd.ptr(qs),
                si_amd.ptr(d), si_amd.ptr(bsum))
        if static:
            si_amd.call("si_attention_static", *args, None)
        else:
            wsb = si_amd.lib().si_attention_workspace(ctypes.byref(s), nq, max_ctx)
            ws = empty(wsb, torch.uint8)
            si_amd.call("si_attention", *args, si_amd.ptr(ws), wsb, None)
        outs.append([host(t) for t in (attn, qs, d, bsum)])
    return outs


def _same(a, b, what):
    for x, y, name in zip(a, b, ("attention", "Q8 values", "Q8 scales", "block sums")):
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), f"{what}: {name} differ"


def test_static_attention_matches_workspace_form():
    rng = np.random.default_rng(77)
    s7 = si_amd.make_shape(**si_amd.SHAPES["7b"])
    s05 = si_amd.make_shape(**si_amd.SHAPES["0.5b"])
    kvd7 = s7.kvheads * s7.hdim
    # 1. causal prefill of 256 tokens after 40 cached positions (flash kernel
    #    with split tiles; 7.5 MB of partial states)
    nq, prefix = 256, 40
    kc, vc = dev(_cache(rng, prefix + nq, kvd7)), dev(_cache(rng, prefix + nq, kvd7))
    q = dev(rng.standard_normal(nq * s7.qheads * s7.hdim).astype(np.float32))
    a, b = _run_both(s7, q, nq, kc, vc, 0, None, prefix + 1, 1, prefix + nq)
    _same(a, b, "7B prefill")
    assert np.abs(a[0]).max() > 0
    # 2. smaller: 16 decode queries over their own caches, ragged contexts
    #    up to 4096 (split-context kernels)
    nq, max_ctx = 16, 4096
    ctxs = np.array([1, 2, 63, 64, 65, 700, 4096, 4000, 17, 1000, 3, 128, 129, 2048, 5, 4095],
                    np.int32)
    kc, vc = dev(_cache(rng, nq * max_ctx, kvd7)), dev(_cache(rng, nq * max_ctx, kvd7))
    q = dev(rng.standard_normal(nq * s7.qheads * s7.hdim).astype(np.float32))
    a, b = _run_both(s7, q, nq, kc, vc, max_ctx * kvd7, dev(ctxs), 0, 0, max_ctx)
    _same(a, b, "7B batched decode")
    # 3. smaller still: one 0.5B query at context 100
    kvd = s05.kvheads * s05.hdim
    kc, vc = dev(_cache(rng, 100, kvd)), dev(_cache(rng, 100, kvd))
    q = dev(rng.standard_normal(s05.qheads * s05.hdim).astype(np.float32))
    a, b = _run_both(s05, q, 1, kc, vc, 0, None, 100, 0, 100)
    _same(a, b, "0.5B decode")


def test_static_attention_refuses_oversize():
    """A call whose partial states exceed the static buffer is refused before
    any launch (its output stays as it was)."""
    torch = _torch()
    s7 = si_amd.make_shape(**si_amd.SHAPES["7b"])
    nq = 2048
    need = si_amd.lib().si_attention_workspace(ctypes.byref(s7), nq, nq)
    assert need > 16 << 20
    qd = s7.qheads * s7.hdim
    attn = torch.full((nq * qd,), 7.0, dtype=torch.float32, device="cuda")
    rc = si_amd.lib().si_attention_static(ctypes.byref(s7), None, nq, None, None, 0, None, 1, 1,
                                          nq, si_amd.ptr(attn), None, None, None, None)
    assert rc == si_amd.SI_ERR_ARG
    assert b"static buffer" in si_amd.lib().si_last_error()
    torch.cuda.synchronize()
    assert bool((attn == 7.0).all())
