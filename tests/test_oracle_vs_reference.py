"""Pins the oracle bit-for-bit to the reference's own portable C path
(oracle/_ref: /root/reference compiled unchanged with its Makefile:7 flags).

Runs only where the reference sources were present at build time; the
committed golden fixtures (test_oracle_golden.py) carry the same checks to
hosts without them.
"""
import numpy as np
import pytest

from oracle.oracle_py import Q8_DTYPE, QK, Q4_BYTES


def _q4_weights(oracle, rng, rows, k, sigma=0.02):
    return oracle.quantize_q4_0(rng.normal(0, sigma, (rows, k)).astype(np.float32))


def test_f16_to_f32_exhaustive(oracle, ref):
    h = np.arange(65536, dtype=np.uint16)
    a = oracle.f16_to_f32(h).view(np.uint32)
    b = ref.f16_to_f32(h).view(np.uint32)
    assert np.array_equal(a, b)


def test_f32_to_f16_strided_sweep(oracle, ref):
    # every 251st bit pattern of all 2^32, plus the interesting neighbourhoods
    pats = np.arange(0, 1 << 32, 251, dtype=np.uint64).astype(np.uint32)
    edges = []
    for c in (0x477FE000, 0x477FF000, 0x38800000, 0x38000000, 0x33000000,
              0x33800000, 0x7F800000, 0x00000001, 0x3F800000):
        edges.append(np.arange(c - 4096, c + 4096, dtype=np.int64).astype(np.uint32))
    pats = np.concatenate([pats] + edges)
    pats = np.concatenate([pats, pats | np.uint32(0x80000000)])
    x = pats.view(np.float32)
    a = oracle.f32_to_f16(x)
    b = ref.f32_to_f16(x)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("case", ["normal", "tiny", "ties", "zeros", "huge", "mixed"])
def test_quantize_q8_bit_exact(oracle, ref, case):
    rng = np.random.default_rng(11)
    n = 32 * 96
    if case == "normal":
        x = rng.standard_normal(n).astype(np.float32)
    elif case == "tiny":  # f16-subnormal and fp32-subnormal scales
        x = (rng.standard_normal(n) * 10.0 ** rng.integers(-44, -3, n)).astype(np.float32)
    elif case == "ties":  # amax 127 -> d = 1, inv = 1: exact .5 ties
        x = (rng.integers(-254, 255, n) / 2.0).astype(np.float32)
        x[::32] = 127.0
    elif case == "zeros":
        x = np.zeros(n, np.float32)
        x[64:96] = rng.standard_normal(32)
    elif case == "huge":
        x = (rng.standard_normal(n) * 1e6).astype(np.float32)
        x[:32] *= np.float32(1e30)
    else:
        x = (rng.standard_normal(n) * np.repeat(10.0 ** rng.uniform(-6, 6, n // 32), 32)
             ).astype(np.float32)
    a = oracle.quantize_q8(x)
    b = ref.quantize_q8(x)
    assert a.tobytes() == b.tobytes()


def test_dot_32_bit_exact(oracle, ref):
    rng = np.random.default_rng(5)
    for trial in range(2000):
        w = rng.integers(0, 256, Q4_BYTES, dtype=np.uint8)
        a = rng.integers(-127, 128, QK, dtype=np.int8)
        if trial == 0:
            w[2:] = 0x00
            a[:] = 127
        elif trial == 1:
            w[2:] = 0xFF
            a[:] = -127
        assert oracle.dot_32(w, a) == ref.dot_32(w, a)


@pytest.mark.parametrize("k,n,bias", [(1536, 1536, True), (1536, 256, False),
                                      (896, 1152, True), (4864, 96, False)])
def test_matvec_bit_exact(oracle, ref, k, n, bias):
    rng = np.random.default_rng(k + n)
    w = _q4_weights(oracle, rng, n, k)
    xq = oracle.quantize_q8(rng.standard_normal(k).astype(np.float32))
    b = rng.normal(0, 0.02, n).astype(np.float32) if bias else None
    a = oracle.matvec(w, xq, k, n, b)
    r = ref.matvec(w, xq, k, n, b)
    assert a.view(np.uint32).tobytes() == r.view(np.uint32).tobytes()


@pytest.mark.parametrize("gain", [False, True])
def test_rmsnorm_bit_exact(oracle, ref, gain):
    rng = np.random.default_rng(2)
    for _ in range(20):
        x = (rng.standard_normal(ref.hidden) * rng.uniform(1e-3, 1e3)).astype(np.float32)
        w = rng.normal(1, 0.1, ref.hidden).astype(np.float32) if gain else None
        assert np.array_equal(oracle.rmsnorm(x, w).view(np.uint32),
                              ref.rmsnorm(x, w).view(np.uint32))


@pytest.mark.parametrize("pos", [0, 1, 17, 1023, 4095, 32767])
def test_rope_bit_exact(oracle, ref, pos):
    rng = np.random.default_rng(pos)
    for nh in (ref.qheads, ref.kvheads):
        v = rng.standard_normal(nh * ref.hdim).astype(np.float32)
        a = oracle.rope(v, nh, ref.hdim, pos)
        b = ref.rope(v, nh, pos)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# audit_fusion_timing.c:142-157: contexts {1,2,17,64,max}, K-history scales
AUDIT_CASES = [(1, 0.25), (2, 0.0125), (17, 1.0), (64, 0.0), (300, 0.5)]


@pytest.mark.parametrize("context,kmul", AUDIT_CASES)
def test_attention_bit_exact(oracle, ref, context, kmul):
    s = ref.shape()
    rng = np.random.default_rng(context)
    kvd = s.kvheads * s.hdim
    q = (rng.uniform(-1, 1, s.qheads * s.hdim) * 1.5).astype(np.float32)
    kc = oracle.f32_to_f16(rng.uniform(-1, 1, context * kvd) * kmul)
    vc = oracle.f32_to_f16(rng.uniform(-1, 1, context * kvd) * 0.25)
    for fn in ("attention_flash", "attention_standard"):
        a = getattr(oracle, fn)(s, q, kc, vc, context)
        b = getattr(ref, fn)(q, kc, vc, context)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), fn


def _ref_layer(oracle, rng, s, with_norm=True, with_bias=True):
    H, QD, KVD = s.hidden, s.qheads * s.hdim, s.kvheads * s.hdim
    return dict(
        wq=_q4_weights(oracle, rng, QD, H), wk=_q4_weights(oracle, rng, KVD, H),
        wv=_q4_weights(oracle, rng, KVD, H), wo=_q4_weights(oracle, rng, H, QD),
        norm=rng.normal(1, 0.1, H).astype(np.float32) if with_norm else None,
        bq=rng.normal(0, 0.02, QD).astype(np.float32) if with_bias else None,
        bk=rng.normal(0, 0.02, KVD).astype(np.float32) if with_bias else None,
        bv=rng.normal(0, 0.02, KVD).astype(np.float32) if with_bias else None)


@pytest.mark.parametrize("context,method,opt", [(1, 1, True), (2, 0, True), (17, 1, False),
                                               (64, 0, False), (129, 1, True)])
def test_run_layer_bit_exact(oracle, ref, context, method, opt):
    s = ref.shape()
    rng = np.random.default_rng(100 + context)
    layer = _ref_layer(oracle, rng, s, with_norm=opt, with_bias=opt)
    kvd = s.kvheads * s.hdim
    x = rng.uniform(-1, 1, s.hidden).astype(np.float32)
    kc0 = oracle.f32_to_f16(rng.uniform(-1, 1, context * kvd) * 0.25)
    vc0 = oracle.f32_to_f16(rng.uniform(-1, 1, context * kvd) * 0.25)
    kc1, vc1 = kc0.copy(), vc0.copy()
    out_o, cap = oracle.run_layer(s, layer, x, kc0, vc0, context, method, capture=True)
    out_r, attn_r, q8_r = ref.run_layer(layer, x, kc1, vc1, context, method)
    assert np.array_equal(out_o.view(np.uint32), out_r.view(np.uint32))
    assert np.array_equal(cap["attn"].view(np.uint32), attn_r.view(np.uint32))
    assert cap["attq"].tobytes() == q8_r.tobytes()
    # the appended fp16 K/V row must be bit-identical (audit_fusion_timing.c:192-196)
    assert np.array_equal(kc0, kc1) and np.array_equal(vc0, vc1)


def test_prefill_equals_sequential_reference_decode(oracle, ref):
    """prefill contract (bench_ai_dma_prefill.c:104-129): prefill == a loop of
    reference run_layer with context prefix+t+1, Y and every fp16 K/V bit-exact."""
    s = ref.shape()
    rng = np.random.default_rng(77)
    layer = _ref_layer(oracle, rng, s)
    ntok, prefix = 6, 3
    kvd = s.kvheads * s.hdim
    total = prefix + ntok
    x = rng.uniform(-1, 1, (ntok, s.hidden)).astype(np.float32)
    kc = np.zeros(total * kvd, np.uint16)
    vc = np.zeros(total * kvd, np.uint16)
    kc[:prefix * kvd] = oracle.f32_to_f16(rng.uniform(-1, 1, prefix * kvd) * 0.25)
    vc[:prefix * kvd] = oracle.f32_to_f16(rng.uniform(-1, 1, prefix * kvd) * 0.25)
    kr, vr = kc.copy(), vc.copy()
    y = oracle.layer_prefill(s, layer, x, ntok, prefix, kc, vc, full=False)
    for t in range(ntok):
        yr, _, _ = ref.run_layer(layer, x[t], kr, vr, prefix + t + 1, 1)
        assert np.array_equal(y[t].view(np.uint32), yr.view(np.uint32)), t
    assert np.array_equal(kc, kr) and np.array_equal(vc, vr)


def test_reference_rng_matches(oracle, ref):
    for seed in (0x5217ac8b, 0x8f53491a, 0x91be2145):
        assert np.array_equal(oracle.rng_floats(seed, 1000), ref.rng_floats(seed, 1000))


def _random_tile(rng, nblocks):
    """Arbitrary column-SoA groups: random nibble bytes, fp32 scales that are
    exact fp16 values (as repack_weights.py writes them)."""
    t = rng.integers(0, 256, (nblocks, 5120), dtype=np.uint8)
    sc = rng.normal(0, 0.01, (nblocks, 256)).astype(np.float16).astype(np.float32)
    t[:, 4096:] = sc.view(np.uint8).reshape(nblocks, 1024)
    return t.reshape(-1)


@pytest.mark.parametrize("add,bias", [(False, False), (False, True), (True, False)])
def test_fused_column_matvec_bit_exact(oracle, ref, add, bias):
    rng = np.random.default_rng(31)
    nb = 48
    tile = _random_tile(rng, nb)
    xq = ref.quantize_q8(rng.standard_normal(nb * QK).astype(np.float32))
    bl = rng.normal(0, 0.02, 128).astype(np.float32) if bias else None
    bh = rng.normal(0, 0.02, 128).astype(np.float32) if bias else None
    start = rng.standard_normal(256).astype(np.float32) if add else None
    a = oracle.fused_column_matvec(tile, xq, nb, bl, bh, start, add)
    b = ref.fused_column_matvec(tile, xq, nb, bl, bh, start, add)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("context,kmul", [(1, 1.0), (2, 0.0125), (17, 1.0), (64, 0.0),
                                          (300, 0.5)])
def test_attention_pair_bit_exact(oracle, ref, context, kmul):
    rng = np.random.default_rng(context)
    s = ref.shape()
    kvd = s.kvheads * s.hdim
    kc = oracle.f32_to_f16((rng.uniform(-1, 1, context * kvd) * kmul).astype(np.float32))
    vc = oracle.f32_to_f16((rng.uniform(-1, 1, context * kvd) * 0.25).astype(np.float32))
    for group in range(s.kvheads):
        qpair = rng.standard_normal(2 * s.hdim).astype(np.float32)
        a = oracle.attention_pair(s, qpair, kc, vc, context, group)
        b = ref.attention_pair(qpair, kc, vc, context, group)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("context", [1, 17, 64, 200])
def test_run_layer_fused_bit_exact(oracle, ref, context):
    """run_layer_fused of the portable build (= run_layer_legacy_fused over
    column-SoA tiles) against the oracle's restatement, on tiles built by the
    oracle's repacker: output, attention and Q8 captures, new K/V rows."""
    from tests.golden.make_golden import layer_weights
    s = ref.shape()
    lay = layer_weights(oracle, 77, s)
    tiles = oracle.colsoa_repack(s, lay)
    rng = np.random.default_rng(context)
    kvd = s.kvheads * s.hdim
    x = rng.standard_normal(s.hidden).astype(np.float32)
    kc0 = oracle.f32_to_f16(rng.uniform(-1, 1, context * kvd).astype(np.float32) * 0.25)
    vc0 = oracle.f32_to_f16(rng.uniform(-1, 1, context * kvd).astype(np.float32) * 0.25)
    ka, va, kb, vb = kc0.copy(), vc0.copy(), kc0.copy(), vc0.copy()
    oa, aa, qa = oracle.run_layer_legacy_fused(s, lay, tiles, x, ka, va, context)
    ob, ab, qb = ref.run_layer_fused(lay, tiles, x, kb, vb, context)
    assert np.array_equal(oa.view(np.uint32), ob.view(np.uint32))
    assert np.array_equal(aa.view(np.uint32), ab.view(np.uint32))
    assert qa.tobytes() == qb.tobytes()
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
