"""The textbook attention mode (attention_standard, attention_kernels.h:33-78)
on the GPU: the three-stage kernel against the oracle's restatement and the
reference's own function (oracle/_ref, 1.5B shape), the decode layer's
SI_LAYER_ATTN_STANDARD mode through the chained layer check, and the
one-layer command line (qwen_one_layer.c:596-713) with its standard, compare
and fused-compare reports on weight files and the reference's synthetic
input stream."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import si_amd
from oracle.oracle_py import make_shape as or_shape
from tests.chain import LayerBuffers, check_row
from tests.gpu_helpers import close, dev, empty, host, kv_history, make_layer

pytestmark = pytest.mark.gpu
STD = si_amd.SI_LAYER_ATTN_STANDARD
CLI = os.path.join(os.path.dirname(si_amd.AMD_SO), "si_qwen_layer")
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_golden.npz")
_SHAPES = {
    "g1_d32": dict(hidden=256, qheads=8, kvheads=1, hdim=32, ffn=0),
    "0.5b": si_amd.SHAPES["0.5b"],
    "g4_d96": dict(hidden=768, qheads=8, kvheads=4, hdim=96, ffn=0),
    "7b": si_amd.SHAPES["7b"],
}


def _torch():
    import torch
    return torch


def _run_standard(s, q, kc, vc, ctx):
    torch = _torch()
    QD = s.qheads * s.hdim
    out = empty(QD, torch.float32)
    scores = empty(max(s.qheads * ctx, 1), torch.float32)
    si_amd.call("si_attention_standard", ctypes.byref(s), si_amd.ptr(q), si_amd.ptr(kc),
                si_amd.ptr(vc), ctx, si_amd.ptr(out), si_amd.ptr(scores), None)
    torch.cuda.synchronize()
    return host(out), host(scores)[:s.qheads * ctx].reshape(s.qheads, ctx)


@pytest.mark.parametrize("name", list(_SHAPES))
@pytest.mark.parametrize("ctx", [1, 2, 255, 256, 257, 1000, 4999])
def test_standard_attention_vs_oracle(oracle, name, ctx):
    sd = _SHAPES[name]
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    kvd, QD = s.kvheads * s.hdim, s.qheads * s.hdim
    rng = np.random.default_rng(ctx * 7 + len(name))
    q = (rng.standard_normal(QD) * 1.5).astype(np.float32)
    kc, vc = kv_history(oracle, rng, ctx, kvd), kv_history(oracle, rng, ctx, kvd)
    print(f"standard attention {name} ctx {ctx}", flush=True)
    got, p = _run_standard(s, dev(q), dev(kc.view(np.int16)), dev(vc.view(np.int16)), ctx)
    want, pw = oracle.attention_standard(os_, q, kc, vc, ctx, with_scores=True)
    # probabilities: same scores (summed in the reference's order), device expf
    np.testing.assert_allclose(p, pw, rtol=2e-5, atol=1e-9)
    close(got, want, 2e-3, f"{name} ctx {ctx} standard")
    if ctx == 1:  # one position: the output is V exactly
        np.testing.assert_array_equal(
            got.reshape(s.qheads, s.hdim),
            oracle.f16_to_f32(vc).reshape(s.kvheads, s.hdim)[
                np.arange(s.qheads) // (s.qheads // s.kvheads)])


def test_standard_attention_edge_cases(oracle):
    torch = _torch()
    sd = _SHAPES["0.5b"]
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    kvd, QD, ctx = s.kvheads * s.hdim, s.qheads * s.hdim, 300
    rng = np.random.default_rng(5)
    vc = kv_history(oracle, rng, ctx, kvd)
    # zero K: uniform weights, the mean of V (the audit's kmul=0 case)
    kc = np.zeros(ctx * kvd, np.uint16)
    q = rng.standard_normal(QD).astype(np.float32)
    got, p = _run_standard(s, dev(q), dev(kc.view(np.int16)), dev(vc.view(np.int16)), ctx)
    assert np.all(p == np.float32(1.0) / np.float32(ctx))
    mean = oracle.f16_to_f32(vc).reshape(ctx, s.kvheads, s.hdim).astype(np.float64).mean(0)
    close(got, mean[np.arange(s.qheads) // (s.qheads // s.kvheads)], 1e-5, "mean of V")
    # one dominant position: its V row
    kc = kv_history(oracle, rng, ctx, kvd, 0.01)
    qn = np.zeros(QD, np.float32)
    kc2 = oracle.f16_to_f32(kc).reshape(ctx, kvd)
    kc2[123, :] = 4.0
    qn[:] = 4.0
    kc = oracle.f32_to_f16(kc2.reshape(-1))
    got, _ = _run_standard(s, dev(qn), dev(kc.view(np.int16)), dev(vc.view(np.int16)), ctx)
    v = oracle.f16_to_f32(vc).reshape(ctx, s.kvheads, s.hdim)[123]
    close(got, v[np.arange(s.qheads) // (s.qheads // s.kvheads)], 1e-5, "peaked")
    # context 0: zero output, nothing read
    out = dev(np.full(QD, 7.0, np.float32))
    si_amd.call("si_attention_standard", ctypes.byref(s), None, None, None, 0, si_amd.ptr(out),
                None, None)
    torch.cuda.synchronize()
    assert np.all(host(out) == 0)


@pytest.mark.parametrize("ctx", [1, 17, 64])
def test_standard_vs_reference_function(oracle, ref, ctx):
    """Against the reference's own attention_standard (1.5B shape)."""
    sd = si_amd.SHAPES["1.5b_ref"]
    s = si_amd.make_shape(**sd)
    kvd, QD = s.kvheads * s.hdim, s.qheads * s.hdim
    rng = np.random.default_rng(40 + ctx)
    q = rng.standard_normal(QD).astype(np.float32)
    kc, vc = kv_history(oracle, rng, ctx, kvd), kv_history(oracle, rng, ctx, kvd)
    got, p = _run_standard(s, dev(q), dev(kc.view(np.int16)), dev(vc.view(np.int16)), ctx)
    want, pw = ref.attention_standard(q, kc, vc, ctx, with_scores=True)
    np.testing.assert_allclose(p, pw, rtol=2e-5, atol=1e-9)
    close(got, want, 2e-3, "vs reference attention_standard")


def test_standard_vs_reference_fixture():
    """Against the reference's own attention_standard output recorded in the
    golden fixture (1.5B shape, context 64; tests/golden/make_golden.py), so
    the comparison also runs where the reference build is absent."""
    g = np.load(GOLDEN, allow_pickle=False)
    s = si_amd.make_shape(**si_amd.SHAPES["1.5b_ref"])
    ctx = 64
    got, p = _run_standard(s, dev(g["att_q"]), dev(g["att_kc"].view(np.int16)),
                           dev(g["att_vc"].view(np.int16)), ctx)
    close(got, g["att_standard"], 2e-3, "vs the reference's attention_standard (fixture)")
    # each head's normalised scores sum to one
    np.testing.assert_allclose(p.astype(np.float64).sum(1), 1.0, rtol=1e-5)


@pytest.mark.parametrize("name,ctx,flags", [
    ("0.5b", 1024, si_amd.SI_LAYER_ATTN_ONLY | si_amd.SI_LAYER_EXACT),
    ("0.5b", 1024, si_amd.SI_LAYER_FULL),
    ("0.5b", 5000, si_amd.SI_LAYER_EXACT),
    ("7b", 4096, si_amd.SI_LAYER_ATTN_ONLY),
    ("7b", 300, si_amd.SI_LAYER_EXACT),
])
def test_layer_decode_standard_mode(oracle, name, ctx, flags):
    torch = _torch()
    full = not flags & si_amd.SI_LAYER_ATTN_ONLY
    sd = dict(si_amd.SHAPES[name])
    if not full:
        sd["ffn"] = 0
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    lay = make_layer(oracle, os_, 31, ffn=full)
    kvd = s.kvheads * s.hdim
    rng = np.random.default_rng(32)
    kc0, vc0 = kv_history(oracle, rng, ctx, kvd), kv_history(oracle, rng, ctx, kvd)
    x = rng.standard_normal(s.hidden).astype(np.float32)
    L = si_amd.Layer(s, lay, 1, ctx)
    print(f"standard layer {name} ctx {ctx} flags {flags}", flush=True)
    outs = []
    for f in (flags | STD, flags):
        kc, vc = dev(kc0.view(np.int16)), dev(vc0.view(np.int16))
        out = empty(s.hidden, torch.float32)
        L.decode(dev(x), kc, vc, ctx, out, f)
        B = LayerBuffers(L, os_, 1)
        hk, hv = host(kc).view(np.uint16), host(vc).view(np.uint16)
        got = host(out)
        check_row(oracle, os_, lay, x, 0, B, hk, hv, 0, ctx - 1, ctx, got,
                  bool(f & si_amd.SI_LAYER_EXACT), full=full)
        outs.append((got, hk, hv, B.attn[0]))
    # both modes append the same K/V rows; attention agrees to 2e-3
    assert np.array_equal(outs[0][1], outs[1][1]) and np.array_equal(outs[0][2], outs[1][2])
    close(outs[0][3], outs[1][3], 2e-3, "standard vs flash attention")
    L.close()


def test_standard_flag_refused_outside_decode(oracle):
    sd = si_amd.SHAPES["0.5b"]
    s, os_ = si_amd.make_shape(**dict(sd, ffn=0)), or_shape(**dict(sd, ffn=0))
    L = si_amd.Layer(s, make_layer(oracle, os_, 1, ffn=False), 4, 64)
    torch = _torch()
    x = empty(4 * s.hidden, torch.float32)
    kc = empty(64 * s.kvheads * s.hdim, torch.int16)
    with pytest.raises(RuntimeError, match="single-token decode only"):
        L.prefill(x, 4, 0, kc, kc, x, si_amd.SI_LAYER_ATTN_ONLY | STD)
    with pytest.raises(RuntimeError, match="single-token decode only"):
        L.decode_batch(x, 4, kc, kc, 0, 8, 8, x, flags=si_amd.SI_LAYER_ATTN_ONLY | STD)
    with pytest.raises(RuntimeError, match="unknown flags"):
        L.decode(x, kc, kc, 8, x, 64)
    L.close()


# ---------------------------------------------------------------------------
# the command line


def _ref_stream(n, state):
    """qwen_one_layer.c:88-96: xorshift32, 16 low bits scaled to [-1, 1]."""
    out = np.empty(n, np.float32)
    v = state[0]
    scale, one = np.float32(1.0) / np.float32(32767.5), np.float32(1.0)
    raw = np.empty(n, np.uint32)
    for i in range(n):
        v ^= (v << 13) & 0xffffffff
        v ^= v >> 17
        v ^= (v << 5) & 0xffffffff
        raw[i] = v
    state[0] = v
    out[:] = (raw & 0xffff).astype(np.float32) * scale - one
    return out


def _ref_inputs(oracle, H, kvd, ctx):
    st = [0x5217ac8b]
    x = _ref_stream(H, st)
    kv = _ref_stream(2 * (ctx - 1) * kvd, st) * np.float32(0.25)
    kc = np.zeros(ctx * kvd, np.uint16)
    vc = np.zeros(ctx * kvd, np.uint16)
    kc[:(ctx - 1) * kvd] = oracle.f32_to_f16(np.ascontiguousarray(kv[0::2]))
    vc[:(ctx - 1) * kvd] = oracle.f32_to_f16(np.ascontiguousarray(kv[1::2]))
    return x, kc, vc


def _write_weights(d, lay):
    names = dict(wq="q.q4_0", wk="k.q4_0", wv="v.q4_0", wo="o.q4_0", norm="norm.f32",
                 bq="q_bias.f32", bk="k_bias.f32", bv="v_bias.f32")
    for k, f in names.items():
        if lay.get(k) is not None:
            (d / f).write_bytes(np.ascontiguousarray(lay[k]).tobytes())


def _cli(args, shape):
    assert os.path.exists(CLI), f"{CLI} missing: run __graft_entry__.build()"
    env = dict(os.environ, SI_SHAPE=shape)
    r = subprocess.run([CLI] + [str(a) for a in args], env=env, capture_output=True, text=True,
                       timeout=100)
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    return r


@pytest.fixture(scope="module")
def weights(tmp_path_factory, oracle):
    sd = dict(si_amd.SHAPES["0.5b"], ffn=0)
    os_ = or_shape(**sd)
    lay = make_layer(oracle, os_, 77, ffn=False)
    d = tmp_path_factory.mktemp("w05")
    _write_weights(d, lay)
    return d, os_, lay


@pytest.mark.parametrize("ctx", [1, 300])
def test_cli_compare_matches_oracle(oracle, weights, ctx):
    d, os_, lay = weights
    r = _cli([d, ctx, 3, "compare"], "0.5b")
    assert r.returncode == 0
    out = r.stdout
    assert "STANDARD vs FLASH" in out
    rows = re.findall(r"^\s+(\d)\s+(\S.*?)\s{2,}", out, re.M)
    assert [int(i) for i, _ in rows] == list(range(1, 10))
    for m in re.finditer(r"^\s+\d\s+.*?([\d.]+)\s+([\d.]+)\s+([\d.]+)x$", out, re.M):
        assert float(m.group(1)) >= 0 and float(m.group(2)) >= 0
    m = re.search(r"Attention O\[(\d+)\]: max_abs=(\S+), max_rel=(\S+)", out)
    assert int(m.group(1)) == 896 and float(m.group(2)) < 2e-3
    cs = re.search(r"Output checksums: standard=(\S+), flash=(\S+)", out)
    x, kc, vc = _ref_inputs(oracle, os_.hidden, os_.kvheads * os_.hdim, ctx)
    want = oracle.run_layer(os_, lay, x, kc, vc, ctx)
    tol = 2e-3 * float(np.abs(want).sum())
    for v in cs.groups():
        assert abs(float(v) - float(want.astype(np.float64).sum())) <= tol, (v, want.sum())


def test_cli_single_modes_and_fused_compare(weights):
    d, os_, lay = weights
    r = _cli([d, 257, 2, "standard"], "0.5b")
    assert r.returncode == 0 and "GQA score/softmax" in r.stdout
    assert "Attention: standard | Context: 257 tokens | Repeats: 2" in r.stdout
    c_std = float(re.search(r"Output checksum: (\S+)", r.stdout).group(1))
    r = _cli([d, 257, 2, "reference"], "0.5b")
    assert r.returncode == 0 and "GQA online (flash)" in r.stdout
    c_fl = float(re.search(r"Output checksum: (\S+)", r.stdout).group(1))
    assert abs(c_std - c_fl) <= 1e-2 * max(1.0, abs(c_fl))
    r = _cli([d, 257, 2, "fused-compare"], "0.5b")
    assert r.returncode == 0
    assert "Q8 blocks different=0/28" in r.stdout  # the same kernels on the GPU
    m = re.search(r"checksum baseline=(\S+) fused=(\S+)", r.stdout)
    assert m.group(1) == m.group(2)
    r = _cli([d, 257, 1, "fused"], "0.5b")
    assert r.returncode == 0 and "REGISTER FUSED one-token" in r.stdout


def test_cli_synthetic_7b_and_errors(tmp_path):
    r = _cli(["synthetic", 4096, 2, "compare"], "7b")
    assert r.returncode == 0
    m = re.search(r"Attention O\[(\d+)\]: max_abs=([^,\s]+)", r.stdout)
    assert int(m.group(1)) == 3584 and float(m.group(2)) < 2e-3
    assert _cli(["synthetic", 0], "7b").returncode == 1
    assert _cli(["synthetic", 16, 1, "bogus"], "7b").returncode == 1
    assert _cli(["synthetic"], "13b").returncode == 1
    assert _cli([tmp_path, 16], "0.5b").returncode == 1  # no weight files
    assert _cli([], "0.5b").returncode == 2


@pytest.fixture(scope="module")
def weights_colsoa(tmp_path_factory, oracle):
    """The reference's own 1.5B shape with its weight files and the
    column-SoA tiles repack_weights.py would write next to them
    (si_amd.repack, through the product's C repacker)."""
    from si_amd import repack
    sd = dict(si_amd.SHAPES["1.5b_ref"])
    os_ = or_shape(**sd)
    lay = make_layer(oracle, os_, 78, ffn=False)
    d = tmp_path_factory.mktemp("w15")
    _write_weights(d, lay)
    repack.repack(str(d), "1.5b_ref")
    return d, os_, lay


@pytest.mark.parametrize("ctx", [1, 300])
def test_cli_fused_compare_on_colsoa_files(oracle, weights_colsoa, ctx):
    """fused-compare with the column-SoA files present compares two different
    paths, as qwen_one_layer.c:650-686 does: the staged flash layer against
    run_layer_legacy_fused on the tiles.  Both outputs agree with the
    oracle's run_layer on the reference's input stream, the attention
    outputs within 2e-3 and the Q8 blocks with at most a rounding flip."""
    d, os_, lay = weights_colsoa
    r = _cli([d, ctx, 2, "fused-compare"], "1.5b")
    assert r.returncode == 0
    assert "COLUMN-SoA FUSED (run_layer_legacy_fused)" in r.stdout
    m = re.search(r"attention max_abs=(\S+), Q8 blocks different=(\d+)/(\d+)", r.stdout)
    assert float(m.group(1).rstrip(",")) < 2e-3 and int(m.group(3)) == 48
    assert int(m.group(2)) <= 2, r.stdout
    cs = re.search(r"checksum baseline=(\S+) fused=(\S+)", r.stdout)
    x, kc, vc = _ref_inputs(oracle, os_.hidden, os_.kvheads * os_.hdim, ctx)
    want = oracle.run_layer(os_, lay, x, kc, vc, ctx).astype(np.float64)
    tol = 2e-3 * float(np.abs(want).sum())
    for v in cs.groups():
        assert abs(float(v) - want.sum()) <= tol, (v, want.sum())
    # the single fused mode runs the same tiles
    r = _cli([d, ctx, 1, "soa-fused"], "1.5b")
    assert r.returncode == 0 and "column-SoA tiles (run_layer_legacy_fused)" in r.stdout
    c = float(re.search(r"Output checksum (\S+)", r.stdout).group(1))
    assert abs(c - want.sum()) <= tol


def test_cli_fused_synthetic_tiles_and_refusals(weights_colsoa):
    """Synthetic weights at a column-SoA shape build their tiles; a TCM
    request is refused (the GPU has no scratchpad to stage tiles in)."""
    r = _cli(["synthetic", 64, 1, "fused-compare"], "1.5b")
    assert r.returncode == 0 and "COLUMN-SoA FUSED" in r.stdout
    m = re.search(r"Q8 blocks different=(\d+)/48", r.stdout)
    assert int(m.group(1)) <= 2
    d, _, _ = weights_colsoa
    env_tcm = dict(os.environ, SI_SHAPE="1.5b", FUSED_TCM="1")
    rr = subprocess.run([CLI, str(d), "16", "1", "fused"], env=env_tcm, capture_output=True,
                        text=True, timeout=100)
    assert rr.returncode == 1 and "scratchpad" in rr.stderr
