"""Writes tests/golden/ref_golden.npz from the reference's OWN portable C path
(oracle/_ref/libsi_ref.so, built from /root/reference by oracle/Makefile).

The reference ships no golden vectors; these fixtures carry its outputs to
hosts without its sources (the GPU box), where test_oracle_golden.py checks the
oracle against them.  Inputs use the reference's own xorshift32 generator and
seeds (qwen_one_layer.c:88-96, verify_fused_projections.c:76,:128) where the
reference tests do, and numpy PCG64 otherwise.  Large weight matrices are not
stored: they are regenerated from a seed and checked against a stored SHA-256.

Run:  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle.oracle_py import Q8_DTYPE, Oracle, Reference  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_golden.npz")


def layer_weights(oracle, seed, s):
    """Seeded 1.5B-shape attention-sublayer weights (quantized by the ggml
    Q4_0 rule in the oracle); regenerated identically by the tests."""
    rng = np.random.default_rng(seed)
    H, QD, KVD = s.hidden, s.qheads * s.hdim, s.kvheads * s.hdim
    q4 = lambda n, k: oracle.quantize_q4_0(rng.normal(0, 0.02, (n, k)).astype(np.float32))
    lay = dict(wq=q4(QD, H), wk=q4(KVD, H), wv=q4(KVD, H), wo=q4(H, QD),
               norm=rng.normal(1, 0.1, H).astype(np.float32),
               bq=rng.normal(0, 0.02, QD).astype(np.float32),
               bk=rng.normal(0, 0.02, KVD).astype(np.float32),
               bv=rng.normal(0, 0.02, KVD).astype(np.float32))
    return lay


def weights_digest(lay):
    h = hashlib.sha256()
    for k in sorted(lay):
        h.update(k.encode())
        h.update(np.ascontiguousarray(lay[k]).tobytes())
    return h.hexdigest()


def main():
    oracle, ref = Oracle(), Reference()
    s = ref.shape()
    g = {}
    # f16 <-> f32 round trip neighbourhoods
    pats = np.concatenate([np.arange(c - 512, c + 512, dtype=np.int64) for c in
                           (0x477FF000, 0x38800000, 0x33000000, 0x3F800000, 0x7F800000)])
    pats = np.concatenate([pats, pats + 0x80000000]).astype(np.uint32)
    g["f32_in"] = pats.view(np.float32)
    g["f16_out"] = ref.f32_to_f16(g["f32_in"])

    # quantize_q8: the reference's verify inputs (seed 0x8f53491a) plus ties/zeros/tiny
    x = ref.rng_floats(0x8f53491a, 1536)
    ties = (np.random.default_rng(1).integers(-254, 255, 1536) / 2.0).astype(np.float32)
    ties[::32] = 127.0
    tiny = (np.random.default_rng(2).standard_normal(1536) *
            10.0 ** np.random.default_rng(3).integers(-44, -3, 1536)).astype(np.float32)
    zeros = np.zeros(1536, np.float32)
    zeros[32:64] = x[:32]
    g["q8_in"] = np.stack([x, ties, tiny, zeros])
    g["q8_out"] = np.stack([ref.quantize_q8(r).view(np.uint8) for r in g["q8_in"]])

    # matvec on a small seeded matrix
    rng = np.random.default_rng(4)
    w = oracle.quantize_q4_0(rng.normal(0, 0.02, (64, 256)).astype(np.float32))
    xq = ref.quantize_q8(rng.standard_normal(256).astype(np.float32))
    b = rng.normal(0, 0.02, 64).astype(np.float32)
    g["mv_w"], g["mv_xq"], g["mv_b"] = w, xq.view(np.uint8), b
    g["mv_out"] = ref.matvec(w, xq, 256, 64, b)

    # rmsnorm / rope at the reference shape
    g["rms_in"] = ref.rng_floats(0x91be2145, 1536, 1.5)
    g["rms_w"] = np.random.default_rng(5).normal(1, 0.1, 1536).astype(np.float32)
    g["rms_out"] = ref.rmsnorm(g["rms_in"], g["rms_w"])
    g["rope_in"] = ref.rng_floats(0x5217ac8b, 1536)
    g["rope_pos"] = np.array([0, 1, 63, 4095, 32767], np.int32)
    g["rope_out"] = np.stack([ref.rope(g["rope_in"], s.qheads, int(p)) for p in g["rope_pos"]])

    # attention: verify_fused_projections.c:123-139 balanced control (ctx 64, x1.5)
    ctx = 64
    kvd = s.kvheads * s.hdim
    ref.lib.si_ref_rng_seed(0x91be2145)
    q = np.array([ref.lib.si_ref_random_float() * 1.5 for _ in range(s.qheads * s.hdim)],
                 np.float32)
    kv = np.array([ref.lib.si_ref_random_float() * 1.5 for _ in range(2 * ctx * kvd)],
                  np.float32).reshape(ctx * kvd, 2)
    g["att_q"] = q
    g["att_kc"] = ref.f32_to_f16(kv[:, 0])
    g["att_vc"] = ref.f32_to_f16(kv[:, 1])
    g["att_flash"] = ref.attention_flash(q, g["att_kc"], g["att_vc"], ctx)
    g["att_standard"] = ref.attention_standard(q, g["att_kc"], g["att_vc"], ctx)

    # run_layer, flash, audit-style contexts {1, 17, 64}
    lay = layer_weights(oracle, 1234, s)
    g["layer_seed"] = np.array([1234])
    g["layer_sha256"] = np.frombuffer(weights_digest(lay).encode(), np.uint8)
    g["layer_x"] = ref.rng_floats(0x5217ac8b, 1536)
    for ctx in (1, 17, 64):
        r = np.random.default_rng(ctx)
        kc = ref.f32_to_f16(r.uniform(-1, 1, ctx * kvd) * 0.25)
        vc = ref.f32_to_f16(r.uniform(-1, 1, ctx * kvd) * 0.25)
        g[f"layer_kc_{ctx}"], g[f"layer_vc_{ctx}"] = kc.copy(), vc.copy()
        out, attn, q8 = ref.run_layer(lay, g["layer_x"], kc, vc, ctx, 1)
        g[f"layer_out_{ctx}"], g[f"layer_attn_{ctx}"] = out, attn
        g[f"layer_q8_{ctx}"] = q8.view(np.uint8)
        g[f"layer_newk_{ctx}"] = kc[(ctx - 1) * kvd:]
        g[f"layer_newv_{ctx}"] = vc[(ctx - 1) * kvd:]
    # the column-SoA path: fused_column_matvec on an arbitrary 8-block tile
    # (fresh, then accumulating), and run_layer_fused (portable build =
    # run_layer_legacy_fused) on the tiles of the layer above; the tiles are
    # rebuilt on the test host by the oracle's repacker, whose layout the
    # reference build pins (test_oracle_vs_reference.py)
    rng = np.random.default_rng(6)
    tile = rng.integers(0, 256, (8, 5120), dtype=np.uint8)
    tile[:, 4096:] = rng.normal(0, 0.01, (8, 256)).astype(np.float16).astype(
        np.float32).view(np.uint8).reshape(8, 1024)
    g["fcm_tile"] = tile.reshape(-1)
    g["fcm_xq"] = ref.quantize_q8(rng.standard_normal(256).astype(np.float32)).view(np.uint8)
    g["fcm_bias"] = rng.normal(0, 0.02, 256).astype(np.float32)
    xq = g["fcm_xq"].view(Q8_DTYPE)
    g["fcm_out"] = ref.fused_column_matvec(g["fcm_tile"], xq, 8, g["fcm_bias"][:128],
                                           g["fcm_bias"][128:])
    g["fcm_out_add"] = ref.fused_column_matvec(g["fcm_tile"], xq, 8, out=g["fcm_out"], add=True)
    tiles = oracle.colsoa_repack(s, lay)
    g["colsoa_sha256"] = np.frombuffer(
        hashlib.sha256(b"".join(t.tobytes() for t in tiles)).hexdigest().encode(), np.uint8)
    for ctx in (1, 17, 64):
        kc, vc = g[f"layer_kc_{ctx}"].copy(), g[f"layer_vc_{ctx}"].copy()
        out, attn, q8 = ref.run_layer_fused(lay, tiles, g["layer_x"], kc, vc, ctx)
        g[f"fused_out_{ctx}"], g[f"fused_attn_{ctx}"] = out, attn
        g[f"fused_q8_{ctx}"] = q8.view(np.uint8)
        g[f"fused_newk_{ctx}"] = kc[(ctx - 1) * kvd:]
        g[f"fused_newv_{ctx}"] = vc[(ctx - 1) * kvd:]
    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
