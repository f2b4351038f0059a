"""Closed-form, brute-force and invariant checks of the oracle, independent of
the reference build.  They pin the build-defined parts (SwiGLU, the full
layer composition, the ggml Q4_0 quantizer) and re-check the reference-pinned
parts against the mathematics, chosen so a dropped term, wrong sign, wrong
index or transposed operand fails."""
import numpy as np
import pytest

from oracle.oracle_py import QK, Q4_BYTES, SHAPES, make_shape


def test_f16_against_numpy_ieee(oracle):
    h = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.isnan(got[nan]).all()
    x = np.arange(0, 1 << 32, 4099, dtype=np.uint64).astype(np.uint32).view(np.float32)
    fin = ~np.isnan(x)
    with np.errstate(over="ignore"):
        want16 = x[fin].astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(x[fin]), want16)
    assert set(np.unique(oracle.f32_to_f16(x[~fin]) & 0x7fff)) == {0x7e00}


def test_quantize_q8_invariants(oracle):
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(32 * 500) * np.repeat(10.0 ** rng.uniform(-3, 3, 500), 32)
         ).astype(np.float32)
    q = oracle.quantize_q8(x)
    xb = x.reshape(-1, 32).astype(np.float64)
    amax = np.abs(xb).max(1)
    d32 = (amax.astype(np.float32) / np.float32(127)).astype(np.float64)
    assert np.array_equal(q["d"], d32.astype(np.float32).astype(np.float16).view(np.uint16))
    qs = q["qs"].astype(np.int64)
    assert np.abs(qs).max() <= 127
    # the largest-magnitude element maps to +-127; every element is within d/2
    idx = np.abs(xb).argmax(1)
    assert np.array_equal(np.abs(qs[np.arange(len(idx)), idx]), np.full(len(idx), 127))
    assert (np.abs(xb - qs * d32[:, None]) <= d32[:, None] * (0.5 + 1e-5)).all()


def test_dot_32_brute_force(oracle):
    rng = np.random.default_rng(1)
    for _ in range(500):
        blk = rng.integers(0, 256, Q4_BYTES, dtype=np.uint8)
        a = rng.integers(-127, 128, QK).astype(np.int8)
        nib = np.concatenate([blk[2:] & 15, blk[2:] >> 4]).astype(np.int64) - 8
        assert oracle.dot_32(blk, a) == int((nib * a.astype(np.int64)).sum())


def test_matvec_against_float64(oracle):
    rng = np.random.default_rng(2)
    k, n = 896, 200
    w = oracle.quantize_q4_0(rng.normal(0, 0.02, (n, k)).astype(np.float32))
    xq = oracle.quantize_q8(rng.standard_normal(k).astype(np.float32))
    b = rng.normal(0, 0.02, n).astype(np.float32)
    got = oracle.matvec(w, xq, k, n, b)
    wf = oracle.dequantize_q4_0(w, n * k).reshape(n, k).astype(np.float64)
    xf = (xq["qs"].astype(np.float64) *
          xq["d"].view(np.float16).astype(np.float64)[:, None]).reshape(-1)
    want = wf @ xf + b
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_rmsnorm_against_float64(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(3584).astype(np.float32)
    w = rng.normal(1, 0.1, 3584).astype(np.float32)
    want = x / np.sqrt((x.astype(np.float64) ** 2).mean() + 1e-6) * w
    assert np.allclose(oracle.rmsnorm(x, w), want, rtol=2e-6, atol=1e-7)


def test_rope_rotation(oracle):
    rng = np.random.default_rng(4)
    d, nh = 64, 3
    v = rng.standard_normal(nh * d).astype(np.float32)
    assert np.array_equal(oracle.rope(v, nh, d, 0), v)  # theta = 0 is the identity
    for pos in (1, 5, 700):
        out = oracle.rope(v, nh, d, pos).reshape(nh, d).astype(np.float64)
        vin = v.reshape(nh, d).astype(np.float64)
        i = np.arange(d // 2)
        theta = pos / (1e6 ** (2 * i / d))
        z = (vin[:, :d // 2] + 1j * vin[:, d // 2:]) * np.exp(1j * theta)
        assert np.allclose(out[:, :d // 2], z.real, atol=2e-5)
        assert np.allclose(out[:, d // 2:], z.imag, atol=2e-5)


def _textbook_attention(q, kc, vc, s, ctx):
    D, per = s.hdim, s.qheads // s.kvheads
    K = kc.reshape(ctx, s.kvheads, D).astype(np.float64)
    V = vc.reshape(ctx, s.kvheads, D).astype(np.float64)
    out = np.zeros((s.qheads, D))
    for h in range(s.qheads):
        sc = K[:, h // per] @ q[h * D:(h + 1) * D].astype(np.float64) / np.sqrt(D)
        p = np.exp(sc - sc.max())
        out[h] = (p / p.sum()) @ V[:, h // per]
    return out.reshape(-1)


@pytest.mark.parametrize("shape", ["0.5b", "7b"])
def test_attention_against_textbook(oracle, shape):
    s = make_shape(**SHAPES[shape])
    rng = np.random.default_rng(5)
    ctx = 300
    kvd = s.kvheads * s.hdim
    q = rng.standard_normal(s.qheads * s.hdim).astype(np.float32)
    kc = oracle.f32_to_f16(rng.standard_normal(ctx * kvd))
    vc = oracle.f32_to_f16(rng.standard_normal(ctx * kvd))
    want = _textbook_attention(q, oracle.f16_to_f32(kc), oracle.f16_to_f32(vc), s, ctx)
    for fn in (oracle.attention_flash, oracle.attention_standard):
        assert np.allclose(fn(s, q, kc, vc, ctx), want, atol=2e-5, rtol=1e-4)
    # context 1 returns V exactly; zero keys give the plain mean of V
    one = oracle.attention_flash(s, q, kc, vc, 1)
    per = s.qheads // s.kvheads
    vf = oracle.f16_to_f32(vc).reshape(ctx, s.kvheads, s.hdim)
    assert np.array_equal(one.reshape(s.qheads, -1), vf[0][np.arange(s.qheads) // per])
    zero = np.zeros_like(kc)
    mean = oracle.attention_flash(s, q, zero, vc, ctx).reshape(s.qheads, -1)
    assert np.allclose(mean, vf.mean(0)[np.arange(s.qheads) // per], atol=1e-5)


def test_swiglu_closed_form(oracle):
    rng = np.random.default_rng(6)
    g = (rng.standard_normal(4096) * 4).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    gd = g.astype(np.float64)
    want = gd / (1 + np.exp(-gd)) * u
    assert np.allclose(oracle.swiglu(g, u), want, rtol=1e-6, atol=1e-7)


def test_q4_0_quantizer_invariants(oracle):
    rng = np.random.default_rng(7)
    w = rng.normal(0, 0.02, (16, 256)).astype(np.float32)
    w[0, :32] = 0.0
    q = oracle.quantize_q4_0(w).reshape(-1, Q4_BYTES)
    d = q[:, :2].copy().view(np.uint16).view(np.float16).astype(np.float64).reshape(-1)
    nib = np.concatenate([q[:, 2:] & 15, q[:, 2:] >> 4], axis=1).astype(np.int64)
    wb = w.reshape(-1, 32).astype(np.float64)
    m = wb[np.arange(len(wb)), np.abs(wb).argmax(1)]
    dm = (m / -8).astype(np.float32).astype(np.float16).astype(np.float64)
    assert np.array_equal(d, dm)
    assert ((nib >= 0) & (nib <= 15)).all()
    nz = d != 0
    assert (nib[nz, :][np.arange(nz.sum()), np.abs(wb[nz]).argmax(1)] == 0).all()
    err = np.abs(wb - (nib - 8) * d[:, None])
    # within half a step, except the clamp at nibble 15 (x/d in (7.5, 8]): one step
    clamped = (nib == 15) & (wb / np.where(d == 0, 1, d)[:, None] > 7.5)
    bound = np.abs(d[:, None]) * np.where(clamped, 1.0, 0.5) * (1 + 1e-3) + 1e-9
    assert (err[nz] <= bound[nz]).all()
    deq = oracle.dequantize_q4_0(q.reshape(-1), w.size).reshape(-1, 32)
    assert np.array_equal(deq, ((nib - 8) * d[:, None]).astype(np.float32))


def _layer(oracle, s, seed):
    rng = np.random.default_rng(seed)
    H, QD, KVD, F = s.hidden, s.qheads * s.hdim, s.kvheads * s.hdim, s.ffn
    q4 = lambda n, k: oracle.quantize_q4_0(rng.normal(0, 0.02, (n, k)).astype(np.float32))
    return dict(wq=q4(QD, H), wk=q4(KVD, H), wv=q4(KVD, H), wo=q4(H, QD),
                norm=rng.normal(1, 0.1, H).astype(np.float32),
                bq=rng.normal(0, 0.02, QD).astype(np.float32),
                bk=rng.normal(0, 0.02, KVD).astype(np.float32),
                bv=rng.normal(0, 0.02, KVD).astype(np.float32),
                post_norm=rng.normal(1, 0.1, H).astype(np.float32),
                wgate=q4(F, H), wup=q4(F, H), wdown=q4(H, F))


def test_full_layer_composition(oracle):
    """Full layer = attention sublayer, residual, post-norm, SwiGLU FFN, residual,
    re-assembled here from the oracle's primitives."""
    s = make_shape(**SHAPES["0.5b"])
    lay = _layer(oracle, s, 8)
    rng = np.random.default_rng(9)
    ctx = 33
    kvd = s.kvheads * s.hdim
    x = rng.standard_normal(s.hidden).astype(np.float32)
    kc = oracle.f32_to_f16(rng.standard_normal(ctx * kvd))
    vc = oracle.f32_to_f16(rng.standard_normal(ctx * kvd))
    kc2, vc2 = kc.copy(), vc.copy()
    out, cap = oracle.layer_decode(s, lay, x, kc, vc, ctx, capture=True)
    ao = oracle.run_layer(s, lay, x, kc2, vc2, ctx)
    assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2)
    h = x + ao
    n2 = oracle.rmsnorm(h, lay["post_norm"])
    xq2 = oracle.quantize_q8(n2)
    g = oracle.matvec(lay["wgate"], xq2, s.hidden, s.ffn)
    u = oracle.matvec(lay["wup"], xq2, s.hidden, s.ffn)
    aq = oracle.quantize_q8(oracle.swiglu(g, u))
    want = h + oracle.matvec(lay["wdown"], aq, s.ffn, s.hidden)
    assert np.array_equal(out, want)
    assert np.array_equal(cap["h"], h) and np.array_equal(cap["gate"], g)


def test_full_prefill_equals_sequential_decode(oracle):
    s = make_shape(**SHAPES["0.5b"])
    lay = _layer(oracle, s, 10)
    rng = np.random.default_rng(11)
    ntok, prefix = 5, 4
    kvd = s.kvheads * s.hdim
    x = rng.standard_normal((ntok, s.hidden)).astype(np.float32)
    kc = np.zeros((prefix + ntok) * kvd, np.uint16)
    vc = np.zeros_like(kc)
    kc[:prefix * kvd] = oracle.f32_to_f16(rng.standard_normal(prefix * kvd))
    vc[:prefix * kvd] = oracle.f32_to_f16(rng.standard_normal(prefix * kvd))
    kr, vr = kc.copy(), vc.copy()
    y = oracle.layer_prefill(s, lay, x, ntok, prefix, kc, vc)
    ysub = oracle.layer_prefill(s, lay, x, ntok, prefix, kc.copy(), vc.copy(), rows=[4, 1])
    for t in range(ntok):
        yt = oracle.layer_decode(s, lay, x[t], kr, vr, prefix + t + 1)
        assert np.array_equal(y[t], yt)
    assert np.array_equal(kc, kr) and np.array_equal(vc, vr)
    assert np.array_equal(ysub, y[[4, 1]])


# Column-SoA tiles (repack_weights.py) and the legacy fused path: the
# reference's portable build computes the same numbers in head-pair order as
# run_layer does in its staged order (same per-row block order, same softmax
# recurrence), so each fused piece must equal the staged function bit for bit
# on the matching rows.  A wrong index in the repacker or the fused path
# (a swapped nibble, pair or output tile) breaks these equalities.
_FUSED_SHAPES = {
    "1.5b": dict(hidden=1536, qheads=12, kvheads=2, hdim=128),
    "2k_g8": dict(hidden=2048, qheads=16, kvheads=2, hdim=128),   # 4 pairs per group
    "1k_g2": dict(hidden=1024, qheads=8, kvheads=4, hdim=128),    # 1 pair per group
}


def _fused_layer(oracle, s, seed):
    rng = np.random.default_rng(seed)
    H, QD, KVD = s.hidden, s.qheads * s.hdim, s.kvheads * s.hdim
    q4 = lambda n, k: oracle.quantize_q4_0(rng.normal(0, 0.02, (n, k)).astype(np.float32))
    return dict(wq=q4(QD, H), wk=q4(KVD, H), wv=q4(KVD, H), wo=q4(H, QD),
                norm=rng.normal(1, 0.1, H).astype(np.float32),
                bq=rng.normal(0, 0.02, QD).astype(np.float32),
                bk=rng.normal(0, 0.02, KVD).astype(np.float32),
                bv=rng.normal(0, 0.02, KVD).astype(np.float32))


@pytest.mark.parametrize("name", list(_FUSED_SHAPES))
def test_colsoa_tiles_equal_row_major_matvec(oracle, name):
    from oracle.oracle_py import make_shape
    s = make_shape(**_FUSED_SHAPES[name])
    lay = _fused_layer(oracle, s, 5)
    qt, kvt, ot = oracle.colsoa_repack(s, lay)
    H, D, QD = s.hidden, s.hdim, s.qheads * s.hdim
    nb, tile = H // 32, (H // 32) * 5120
    rng = np.random.default_rng(6)
    xq = oracle.quantize_q8(rng.standard_normal(H).astype(np.float32))
    q = oracle.matvec(lay["wq"], xq, H, QD, lay["bq"])
    for p in range(s.qheads // 2):
        bq = lay["bq"][p * 256:(p + 1) * 256]
        y = oracle.fused_column_matvec(qt[p * tile:(p + 1) * tile], xq, nb, bq[:128], bq[128:])
        assert np.array_equal(y.view(np.uint32), q[p * 256:(p + 1) * 256].view(np.uint32)), p
    k = oracle.matvec(lay["wk"], xq, H, s.kvheads * D, lay["bk"])
    v = oracle.matvec(lay["wv"], xq, H, s.kvheads * D, lay["bv"])
    for g in range(s.kvheads):
        y = oracle.fused_column_matvec(kvt[g * tile:(g + 1) * tile], xq, nb,
                                       lay["bk"][g * D:(g + 1) * D], lay["bv"][g * D:(g + 1) * D])
        want = np.concatenate([k[g * D:(g + 1) * D], v[g * D:(g + 1) * D]])
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), g
    # W_O: every pair's 8 input blocks added in pair order equals the staged
    # mat-vec, whose block order is the same
    aq = oracle.quantize_q8(rng.standard_normal(QD).astype(np.float32))
    want = oracle.matvec(lay["wo"], aq, QD, H)
    got = np.zeros(H, np.float32)
    sub, yt = 8 * 5120, H // 256
    for p in range(s.qheads // 2):
        for t in range(yt):
            base = (p * yt + t) * sub
            got[t * 256:(t + 1) * 256] = oracle.fused_column_matvec(
                ot[base:base + sub], aq[p * 8:(p + 1) * 8], 8, out=got[t * 256:(t + 1) * 256],
                add=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name", list(_FUSED_SHAPES))
@pytest.mark.parametrize("context", [1, 33])
def test_legacy_fused_layer_equals_run_layer(oracle, name, context):
    from oracle.oracle_py import make_shape
    s = make_shape(**_FUSED_SHAPES[name])
    lay = _fused_layer(oracle, s, 8)
    tiles = oracle.colsoa_repack(s, lay)
    rng = np.random.default_rng(context)
    kvd = s.kvheads * s.hdim
    x = rng.standard_normal(s.hidden).astype(np.float32)
    kc0 = oracle.f32_to_f16(rng.standard_normal(context * kvd).astype(np.float32))
    vc0 = oracle.f32_to_f16(rng.standard_normal(context * kvd).astype(np.float32))
    ka, va, kb, vb = kc0.copy(), vc0.copy(), kc0.copy(), vc0.copy()
    fo, fa, fq = oracle.run_layer_legacy_fused(s, lay, tiles, x, ka, va, context)
    so, sb = oracle.run_layer(s, lay, x, kb, vb, context, capture=True)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    assert np.array_equal(fa.view(np.uint32), sb["attn"].view(np.uint32))
    assert fq.tobytes() == sb["attq"].tobytes()
    assert np.array_equal(fo.view(np.uint32), so.view(np.uint32))
    # the pair attention is attention_flash's recurrence on the pair's heads
    per = s.qheads // s.kvheads
    for g in range(s.kvheads):
        for p in range(per // 2):
            h0 = g * per + 2 * p
            qpair = sb["q"][h0 * s.hdim:(h0 + 2) * s.hdim]
            got = oracle.attention_pair(s, qpair, kb, vb, context, g)
            assert np.array_equal(got.view(np.uint32),
                                  sb["attn"][h0 * s.hdim:(h0 + 2) * s.hdim].view(np.uint32))
