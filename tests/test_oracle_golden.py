"""Oracle vs the golden fixtures written from the reference's own build
(tests/golden/make_golden.py).  Runs everywhere, including hosts without
/root/reference; every comparison is bit-exact."""
import hashlib
import os

import numpy as np
import pytest

from oracle.oracle_py import Q8_DTYPE, make_shape

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_golden.npz")
REF_SHAPE = dict(hidden=1536, qheads=12, kvheads=2, hdim=128)


@pytest.fixture(scope="module")
def g():
    return np.load(GOLDEN, allow_pickle=False)


def test_f32_to_f16(oracle, g):
    assert np.array_equal(oracle.f32_to_f16(g["f32_in"]), g["f16_out"])


def test_quantize_q8(oracle, g):
    for x, want in zip(g["q8_in"], g["q8_out"]):
        assert oracle.quantize_q8(x).view(np.uint8).tobytes() == want.tobytes()


def test_matvec(oracle, g):
    xq = g["mv_xq"].view(Q8_DTYPE)
    out = oracle.matvec(g["mv_w"], xq, 256, 64, g["mv_b"])
    assert np.array_equal(out.view(np.uint32), g["mv_out"].view(np.uint32))


def test_rmsnorm_rope(oracle, g):
    assert np.array_equal(oracle.rmsnorm(g["rms_in"], g["rms_w"]).view(np.uint32),
                          g["rms_out"].view(np.uint32))
    for pos, want in zip(g["rope_pos"], g["rope_out"]):
        got = oracle.rope(g["rope_in"], 12, 128, int(pos))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), pos


def test_attention(oracle, g):
    s = make_shape(**REF_SHAPE)
    a = oracle.attention_flash(s, g["att_q"], g["att_kc"], g["att_vc"], 64)
    b = oracle.attention_standard(s, g["att_q"], g["att_kc"], g["att_vc"], 64)
    assert np.array_equal(a.view(np.uint32), g["att_flash"].view(np.uint32))
    assert np.array_equal(b.view(np.uint32), g["att_standard"].view(np.uint32))


def test_run_layer(oracle, g):
    from tests.golden.make_golden import layer_weights, weights_digest
    s = make_shape(**REF_SHAPE)
    lay = layer_weights(oracle, int(g["layer_seed"][0]), s)
    assert weights_digest(lay) == bytes(g["layer_sha256"]).decode()
    kvd = s.kvheads * s.hdim
    for ctx in (1, 17, 64):
        kc = g[f"layer_kc_{ctx}"].copy()
        vc = g[f"layer_vc_{ctx}"].copy()
        out, cap = oracle.run_layer(s, lay, g["layer_x"], kc, vc, ctx, 1, capture=True)
        assert np.array_equal(out.view(np.uint32), g[f"layer_out_{ctx}"].view(np.uint32))
        assert np.array_equal(cap["attn"].view(np.uint32),
                              g[f"layer_attn_{ctx}"].view(np.uint32))
        assert cap["attq"].view(np.uint8).tobytes() == g[f"layer_q8_{ctx}"].tobytes()
        assert np.array_equal(kc[(ctx - 1) * kvd:], g[f"layer_newk_{ctx}"])
        assert np.array_equal(vc[(ctx - 1) * kvd:], g[f"layer_newv_{ctx}"])


def test_fused_column_matvec(oracle, g):
    xq = g["fcm_xq"].view(Q8_DTYPE)
    y = oracle.fused_column_matvec(g["fcm_tile"], xq, 8, g["fcm_bias"][:128], g["fcm_bias"][128:])
    assert np.array_equal(y.view(np.uint32), g["fcm_out"].view(np.uint32))
    y2 = oracle.fused_column_matvec(g["fcm_tile"], xq, 8, out=y, add=True)
    assert np.array_equal(y2.view(np.uint32), g["fcm_out_add"].view(np.uint32))


def test_run_layer_fused(oracle, g):
    """The reference's run_layer_fused (portable build) on column-SoA tiles
    rebuilt here by the oracle's repacker (digest of the tiles recorded)."""
    from tests.golden.make_golden import layer_weights
    s = make_shape(**REF_SHAPE)
    lay = layer_weights(oracle, int(g["layer_seed"][0]), s)
    tiles = oracle.colsoa_repack(s, lay)
    digest = hashlib.sha256(b"".join(t.tobytes() for t in tiles)).hexdigest()
    assert digest == bytes(g["colsoa_sha256"]).decode()
    kvd = s.kvheads * s.hdim
    for ctx in (1, 17, 64):
        kc, vc = g[f"layer_kc_{ctx}"].copy(), g[f"layer_vc_{ctx}"].copy()
        out, attn, q8 = oracle.run_layer_legacy_fused(s, lay, tiles, g["layer_x"], kc, vc, ctx)
        assert np.array_equal(out.view(np.uint32), g[f"fused_out_{ctx}"].view(np.uint32))
        assert np.array_equal(attn.view(np.uint32), g[f"fused_attn_{ctx}"].view(np.uint32))
        assert q8.view(np.uint8).tobytes() == g[f"fused_q8_{ctx}"].tobytes()
        assert np.array_equal(kc[(ctx - 1) * kvd:], g[f"fused_newk_{ctx}"])
        assert np.array_equal(vc[(ctx - 1) * kvd:], g[f"fused_newv_{ctx}"])
