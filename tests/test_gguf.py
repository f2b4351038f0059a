"""GGUF ingest (si_amd.gguf): the reader pinned against a byte image built
by hand from the published layout (independent of the module's writer),
writer/reader round trips, the reference extractor's refusals
(extract_weights.py:77-199), and on the GPU a layer loaded from a GGUF file
giving the same bits as the layer built from the same arrays."""
import os
import struct

import numpy as np
import pytest
import si_amd
from si_amd import gguf

from tests.gpu_helpers import dev, empty, host, kv_history


def _s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _hand_image():
    """A v3 file: 3 metadata keys (string, u32, array of strings that the
    reader skips), 2 tensors (Q4_0 matrix 32 x 2, F16 vector of 2)."""
    meta = (_s("general.architecture") + struct.pack("<I", 8) + _s("qwen2") +
            _s("qwen2.embedding_length") + struct.pack("<II", 4, 32) +
            _s("tokenizer.ggml.tokens") + struct.pack("<IIQ", 9, 8, 2) + _s("a") + _s("bc"))
    q4 = bytes(range(36))  # 2 rows x 1 block x 18 bytes
    f16 = np.array([1.5, -2.25], "<f2").tobytes()
    tens = (_s("w") + struct.pack("<I", 2) + struct.pack("<QQ", 32, 2) + struct.pack("<IQ", 2, 0) +
            _s("v") + struct.pack("<I", 1) + struct.pack("<Q", 2) + struct.pack("<IQ", 1, 64))
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, 3) + meta + tens
    pad = b"\0" * ((-len(head)) % 32)
    body = q4 + b"\0" * (64 - 36) + f16 + b"\0" * 28  # each tensor padded to 32
    return head + pad + body, len(head) + len(pad), q4, f16


def test_reader_on_hand_built_image(tmp_path):
    img, start, q4, f16 = _hand_image()
    meta, tens, data_start = gguf.read_index(img)
    assert data_start == start
    assert meta == {"general.architecture": "qwen2", "qwen2.embedding_length": 32}
    assert tens == {"w": ([32, 2], gguf.Q4_0, 0), "v": ([2], gguf.F16, 64)}
    p = tmp_path / "hand.gguf"
    p.write_bytes(img)
    with gguf.GGUFFile(str(p)) as gf:
        assert gf.raw("w").tobytes() == q4
        assert np.array_equal(gf.matrix_q4("w", 2, 32), np.frombuffer(q4, np.uint8).reshape(2, 18))
        assert np.array_equal(gf.vector_f32("v", 2), np.array([1.5, -2.25], np.float32))


def test_writer_matches_hand_image(tmp_path):
    img, _, q4, f16 = _hand_image()
    p = tmp_path / "w.gguf"
    gguf.write_gguf(str(p), {"general.architecture": "qwen2", "qwen2.embedding_length": 32,
                             "tokenizer.ggml.tokens": ["a", "bc"]},
                    {"w": (gguf.Q4_0, [32, 2], q4), "v": (gguf.F16, [2], f16)})
    assert p.read_bytes() == img


def _tiny_layer(seed=0, ffn=64):
    sd = dict(hidden=128, qheads=4, kvheads=2, hdim=32, ffn=ffn)
    rng = np.random.default_rng(seed)
    H, QD, KVD, F = sd["hidden"], sd["qheads"] * sd["hdim"], sd["kvheads"] * sd["hdim"], ffn
    q4 = lambda n, k: si_amd.quantize_q4_0(rng.normal(0, 0.02, (n, k)).astype(np.float32))
    t = dict(wq=q4(QD, H), wk=q4(KVD, H), wv=q4(KVD, H), wo=q4(H, QD),
             norm=rng.normal(1, 0.1, H).astype(np.float32),
             bq=rng.normal(0, 0.02, QD).astype(np.float32),
             bk=rng.normal(0, 0.02, KVD).astype(np.float32),
             bv=rng.normal(0, 0.02, KVD).astype(np.float32))
    if ffn:
        t.update(post_norm=rng.normal(1, 0.1, H).astype(np.float32),
                 wgate=q4(F, H), wup=q4(F, H), wdown=q4(H, F))
    return sd, t


@pytest.mark.parametrize("f16", [False, True])
def test_layer_round_trip(tmp_path, f16):
    sd, t = _tiny_layer(1)
    sd.update(rope_base=1e6, rms_eps=1e-6)
    meta = gguf.layer_meta(sd)
    meta["tokenizer.ggml.merges"] = ["x y"] * 50  # skipped by the reader
    meta["general.nested"] = [[1, 2], [3]]        # nested arrays parse
    path = str(tmp_path / "layer.gguf")
    gguf.write_gguf(path, meta, gguf.layer_tensors_gguf(sd, t, layer=3, f16_vectors=f16),
                    alignment=64)
    with gguf.GGUFFile(path) as gf:
        assert gf.meta["general.alignment"] == 64
        assert [list(x) for x in gf.meta["general.nested"]] == [[1, 2], [3]]
        assert not any(k.startswith("tokenizer.") for k in gf.meta)
        got_sd, got = gguf.load_layer(gf, 3)
        # tensors live in process memory, not in the file mapping
        assert all(v is None or v.base is None or not isinstance(v.base, type(gf._mm))
                   for v in got.values())
        assert all(v is None or v.flags.owndata for v in got.values())
        assert {k: got_sd[k] for k in ("hidden", "qheads", "kvheads", "hdim", "ffn")} == \
            {k: sd[k] for k in ("hidden", "qheads", "kvheads", "hdim", "ffn")}
        for k, v in t.items():
            want = v.astype(np.float16).astype(np.float32) if (f16 and v.dtype != np.uint8) else v
            assert np.array_equal(got[k], want), k
        _, attn = gguf.load_layer(gf, 3, ffn=False)
        assert "wgate" not in attn and attn["wq"].shape == t["wq"].shape


def test_optional_vectors_and_refusals(tmp_path):
    sd, t = _tiny_layer(2)
    names = gguf.layer_names(0)
    base = gguf.layer_tensors_gguf(sd, t)

    def write(tens, meta=None, **kw):
        p = str(tmp_path / f"f{len(os.listdir(tmp_path))}.gguf")
        gguf.write_gguf(p, meta if meta is not None else gguf.layer_meta(sd), tens, **kw)
        return p

    # missing norms / biases: identity norm and zero bias (None)
    tens = {k: v for k, v in base.items() if not k.endswith((".bias", "norm.weight"))}
    with gguf.GGUFFile(write(tens)) as gf:
        _, got = gguf.load_layer(gf, 0)
        assert all(got[k] is None for k in ("norm", "bq", "bk", "bv", "post_norm"))

    def refused(tens, what, meta=None):
        with pytest.raises(gguf.GGUFError, match=what):
            with gguf.GGUFFile(write(tens, meta)) as gf:
                gguf.load_layer(gf, 0)

    refused({k: v for k, v in base.items() if k != names["wq"]}, "required tensor not found")
    bad = dict(base)
    typ, dims, data = bad[names["wk"]]
    bad[names["wk"]] = (typ, [dims[1], dims[0]], data)  # transposed dims
    refused(bad, "expected")
    bad = dict(base)
    _, dims, _ = bad[names["wv"]]
    bad[names["wv"]] = (gguf.Q8_0, dims, np.zeros(dims[0] * dims[1] // 32 * 34, np.uint8))
    refused(bad, "not Q4_0")
    bad = dict(base)
    bad[names["norm"]] = (gguf.Q4_0, [sd["hidden"]], np.zeros(sd["hidden"] // 32 * 18, np.uint8))
    refused(bad, "must be F32/F16")
    meta = gguf.layer_meta(sd)
    meta["general.architecture"] = "llama"
    refused(base, "qwen2 architecture", meta)
    meta = gguf.layer_meta(sd)
    meta["qwen2.rope.dimension_count"] = sd["hdim"] // 2
    refused(base, "partial rotary", meta)


def test_malformed_files(tmp_path):
    img, *_ = _hand_image()
    cases = {
        "magic": b"GGUX" + img[4:],
        "version": img[:4] + struct.pack("<I", 1) + img[8:],
        "truncated": img[:40],
    }
    for what, data in cases.items():
        with pytest.raises(gguf.GGUFError):
            gguf.read_index(data)
    # duplicate tensor names
    dup = b"GGUF" + struct.pack("<IQQ", 3, 2, 0)
    for _ in range(2):
        dup += _s("t") + struct.pack("<I", 1) + struct.pack("<Q", 32) + struct.pack("<IQ", 0, 0)
    with pytest.raises(gguf.GGUFError, match="duplicate"):
        gguf.read_index(dup + b"\0" * 256)
    # a tensor whose data runs past the end of the file
    p = tmp_path / "short.gguf"
    short = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + _s("t") + struct.pack("<I", 1) + \
        struct.pack("<Q", 64) + struct.pack("<IQ", 0, 0)
    p.write_bytes(short + b"\0" * ((-len(short)) % 32) + b"\0" * 16)
    with gguf.GGUFFile(str(p)) as gf:
        with pytest.raises(gguf.GGUFError, match="exceeds"):
            gf.raw("t")
    # alignment must be a multiple of 8
    bad = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + _s("general.alignment") + \
        struct.pack("<II", 4, 12)
    with pytest.raises(gguf.GGUFError, match="alignment"):
        gguf.read_index(bad)


@pytest.mark.gpu
@pytest.mark.parametrize("name,ctx", [("0.5b", 300), ("7b", 1024)])
def test_layer_from_gguf_matches_direct(tmp_path, name, ctx):
    """A layer written to GGUF and loaded back (extract_weights.py:144-199
    feeding load_layer, qwen_one_layer.c:210-221): the tensors read equal
    the source arrays byte for byte, the decode passes the chained oracle
    check (tests/chain.py) on the source arrays, FULL and EXACT, and gives
    the same bits as the layer built from the arrays directly."""
    from oracle.oracle_py import Oracle
    from tests.chain import LayerBuffers, check_row
    from tests.gpu_helpers import make_layer, torch_cuda
    torch = torch_cuda()  # torch's device first, then the native layers
    from oracle.oracle_py import make_shape as or_shape
    oracle = Oracle()
    sd = dict(si_amd.SHAPES[name])
    s, os_ = si_amd.make_shape(**sd), or_shape(**sd)
    lay = make_layer(oracle, os_, 17)
    path = str(tmp_path / "l.gguf")
    gguf.write_gguf(path, gguf.layer_meta(sd), gguf.layer_tensors_gguf(sd, lay, layer=5))
    with gguf.GGUFFile(path) as gf:
        gsd, gt = gguf.load_layer(gf, 5)
        for key, shape_val in sd.items():
            assert gsd[key] == shape_val, key
        for key, arr in lay.items():
            if arr is None:
                assert gt[key] is None, key
            else:
                assert np.array_equal(np.asarray(gt[key]).view(np.uint8).reshape(-1),
                                      np.asarray(arr).view(np.uint8).reshape(-1)), key
        Lg = si_amd.Layer(si_amd.make_shape(**gsd), gt, 1, ctx)
    Ld = si_amd.Layer(s, lay, 1, ctx)
    kvd = s.kvheads * s.hdim
    rng = np.random.default_rng(18)
    kc0, vc0 = kv_history(oracle, rng, ctx, kvd), kv_history(oracle, rng, ctx, kvd)
    xh = rng.standard_normal(s.hidden).astype(np.float32)
    x = dev(xh)
    for flags in (si_amd.SI_LAYER_FULL, si_amd.SI_LAYER_EXACT):
        outs = []
        for L in (Lg, Ld):
            kc, vc = dev(kc0.view(np.int16)), dev(vc0.view(np.int16))
            out = empty(s.hidden, torch.float32)
            L.decode(x, kc, vc, ctx, out, flags)
            outs.append((host(out), host(kc), host(vc)))
            if L is Lg:
                B = LayerBuffers(Lg, os_, 1)
                hk, hv = outs[-1][1].view(np.uint16), outs[-1][2].view(np.uint16)
                check_row(oracle, os_, lay, xh, 0, B, hk, hv, 0, ctx - 1, ctx, outs[-1][0],
                          flags == si_amd.SI_LAYER_EXACT)
        assert all(np.array_equal(a, b) for a, b in zip(*outs)), flags
    Lg.close()
    Ld.close()


@pytest.mark.gpu
def test_device_manifest_round_trip(oracle):
    """The ingest manifest of a created layer: raw Q4_0 SHA-256 per matrix,
    the device arrays' digests, and the lossless unpack round trip."""
    import hashlib
    from oracle.oracle_py import make_shape as or_shape
    from si_amd import repack
    from tests.gpu_helpers import make_layer
    sd = si_amd.SHAPES["0.5b"]
    lay = make_layer(oracle, or_shape(**sd), 6)
    L = si_amd.Layer(si_amd.make_shape(**sd), lay, 1, 16)
    m = repack.device_manifest(L, lay)
    assert set(m["matrices"]) == {"qkv", "o", "gate_up", "down"}
    for name, parts in (("qkv", ("wq", "wk", "wv")), ("o", ("wo",)),
                        ("gate_up", ("wgate", "wup")), ("down", ("wdown",))):
        e = m["matrices"][name]
        assert e["round_trip"], name
        raw = b"".join(np.ascontiguousarray(lay[p]).tobytes() for p in parts)
        assert e["raw_q4_sha256"] == hashlib.sha256(raw).hexdigest()
    L.close()
