"""CPU-side checks of the native libraries (no GPU needed): they load, export
every function include/*.h declares, their host-side code (RoPE tables, the
Q4_0 weight quantizer) matches the oracle bit for bit, and argument errors
are reported without touching the device."""
import ctypes

import numpy as np
import pytest

import si_amd


def test_libraries_export_every_declared_symbol():
    amd = ctypes.CDLL(si_amd.AMD_SO)
    host = ctypes.CDLL(si_amd.HOST_SO)
    decl = si_amd.declared_functions()
    assert len(decl) > 30
    missing = [(h, n) for h, n in decl
               if not hasattr(amd if h == "si_abi.h" else host, n)]
    assert not missing, missing


@pytest.mark.parametrize("hdim,npos", [(64, 1100), (128, 4097)])
def test_rope_table_matches_oracle(oracle, hdim, npos):
    c = np.empty((npos, hdim // 2), np.float32)
    s = np.empty_like(c)
    si_amd.call("si_rope_table", npos, hdim, 1e6, si_amd.ptr(c), si_amd.ptr(s))
    oc, os_ = oracle.rope_table(0, npos, hdim)
    assert np.array_equal(c.view(np.uint32), oc.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), os_.view(np.uint32))


def test_product_q4_0_quantizer_matches_oracle(oracle):
    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.02, (64, 896)).astype(np.float32)
    w[3, :32] = 0.0
    w[5, 64:96] = 1e-9
    assert np.array_equal(si_amd.quantize_q4_0(w), oracle.quantize_q4_0(w))


def test_argument_errors_do_not_launch():
    L = si_amd.lib()
    assert L.si_quantize_q8(None, None, 33, None) == si_amd.SI_ERR_ARG
    assert b"multiple of 32" in L.si_last_error()
    assert L.si_gemm_q4q8(None, None, 8, 64, 30, None, None, 4, None, None, None, 64, 0,
                          None, 0, None) == si_amd.SI_ERR_ARG
    assert L.si_gemm_gateup_q8(None, None, 8, 48, 64, None, None, 4, None, None, None, None,
                               None, 0, None, 0, None) == si_amd.SI_ERR_ARG  # f % 32
    assert L.si_gemm_gateup_q8(None, None, 8, 64, 64, None, None, 4, None, None, None, None,
                               None, 0, None, 0, None) == si_amd.SI_ERR_ARG  # NULL
    assert b"NULL" in L.si_last_error()
    # a q output off 16-byte alignment (the epilogue stores 16 bytes); the
    # pointers are never dereferenced: the call is refused first
    a16, odd = 1 << 12, (1 << 12) + 4
    assert L.si_gemm_gateup_q8(a16, a16, 8, 64, 64, a16, a16, 4, a16, None, odd, a16, None, 0,
                               None, 0, None) == si_amd.SI_ERR_ARG
    assert b"16-byte aligned" in L.si_last_error()
    assert L.si_gemm_q4q8(None, None, 8, 1 << 20, 8192, None, None, 4, None, None, None,
                          1 << 20, 0, None, 0, None) == si_amd.SI_ERR_ARG
    assert b"2 GiB" in L.si_last_error()
    assert L.si_gemm_workspace(64, 3584, 18944) > 0  # small grid: K is split
    # operand-tiled activations: at most 512 rows, no exact mode
    assert L.si_gemm_q4q8(a16, a16, 8, 64, 64, a16, a16, 513, None, None, a16, 64,
                          si_amd.SI_GEMM_TILED_A, None, 0, None) == si_amd.SI_ERR_ARG
    assert b"at most 512 rows" in L.si_last_error()
    assert L.si_gemm_q4q8(a16, a16, 8, 64, 64, a16, a16, 4, None, None, a16, 64,
                          si_amd.SI_GEMM_TILED_A | si_amd.SI_GEMM_EXACT, None, 0,
                          None) == si_amd.SI_ERR_ARG
    assert L.si_q8_tile(a16, a16, 4, 48, a16, a16, None) == si_amd.SI_ERR_ARG  # k % 32
    assert L.si_q8_tile(odd, a16, 4, 64, a16, a16, None) == si_amd.SI_ERR_ARG
    assert b"16-byte aligned" in L.si_last_error()
    assert L.si_gemm_workspace(2048, 3584, 3584) == 0
    assert L.si_matvec_q4q8(None, None, 8, 64, 64, None, None, None, None, None, None, 0,
                            None) == si_amd.SI_ERR_ARG
    assert L.si_matvec_q4q8(None, None, 12, 64, 64, None, None, None, None, None, None, 0,
                            None) == si_amd.SI_ERR_ARG
    assert b"tile 12" in L.si_last_error()
    # the mat-vec kernels address weights with 32-bit buffer offsets
    assert L.si_matvec_q4q8(None, None, 8, 1 << 20, 8192, None, None, None, None, None, None,
                            0, None) == si_amd.SI_ERR_ARG
    assert b"4 GiB" in L.si_last_error()
    huge = si_amd.make_shape(8192, 64, 8, 128, ffn=1 << 20)
    assert L.si_layer_create(ctypes.byref(huge), ctypes.byref(si_amd.LayerHost()), 1, 16,
                             ctypes.byref(ctypes.c_void_p())) == si_amd.SI_ERR_ARG
    assert b"4 GiB" in L.si_last_error()
    assert L.si_q4_scale_count(300, 64, 16) == 304 * 2
    assert L.si_q4_tile(37888, 3584) == 32 and L.si_q4_tile(896, 896) == 8
    bad = si_amd.make_shape(896, 14, 3, 64)  # 14 % 3 != 0
    assert L.si_rope_kv_append(ctypes.byref(bad), None, 0, 0, 0, 0, 1, None, None, None, None,
                               None, None, 0, None) == si_amd.SI_ERR_ARG
    assert b"unsupported heads" in L.si_last_error()
    s = si_amd.make_shape(**si_amd.SHAPES["0.5b"])
    assert L.si_attention(ctypes.byref(s), None, 1, None, None, 0, None, 0, 0, 16, None, None,
                          None, None, None, 0, None) == si_amd.SI_ERR_ARG
    assert L.si_attention_standard(ctypes.byref(s), None, None, None, -1, None, None,
                                   None) == si_amd.SI_ERR_ARG
    assert b"negative context" in L.si_last_error()
    assert L.si_attention_standard(ctypes.byref(s), None, None, None, 4, ctypes.c_void_p(256),
                                   None, None) == si_amd.SI_ERR_ARG
    assert b"NULL" in L.si_last_error()
    assert L.si_attention_standard(ctypes.byref(bad), None, None, None, 0, None, None,
                                   None) == si_amd.SI_ERR_ARG
    h = ctypes.c_void_p()
    host = si_amd.LayerHost()
    assert L.si_layer_create(ctypes.byref(s), ctypes.byref(host), 1, 16,
                             ctypes.byref(h)) == si_amd.SI_ERR_ARG
    assert L.si_layer_decode(None, None, None, None, 1, None, 0, None) == si_amd.SI_ERR_ARG
    assert L.si_layer_create_in(None, ctypes.byref(host), ctypes.byref(h)) == si_amd.SI_ERR_ARG
    assert L.si_workspace_create(ctypes.byref(bad), 1, 16, ctypes.byref(h)) == si_amd.SI_ERR_ARG


def test_attention_workspace_sizing():
    s = si_amd.make_shape(**si_amd.SHAPES["7b"])
    ws = si_amd.lib().si_attention_workspace(ctypes.byref(s), 64, 4096)
    assert ws > 0 and ws % 4 == 0


def test_command_line_argument_errors():
    """lib/si_qwen_layer validates its arguments like qwen_one_layer.c:596-629
    before touching the device: usage -> 2, bad values -> 1 with the
    reference's messages."""
    import os
    import subprocess
    cli = os.path.join(os.path.dirname(si_amd.AMD_SO), "si_qwen_layer")
    assert os.path.exists(cli)

    def run(*args, shape="1.5b"):
        env = dict(os.environ, SI_SHAPE=shape)
        return subprocess.run([cli, *map(str, args)], env=env, capture_output=True, text=True,
                              timeout=60)

    r = run()
    assert r.returncode == 2 and "Usage:" in r.stderr
    assert run("w", 1, 1, "standard", "extra").returncode == 2
    for args, msg in (((0,), "Context must be 1..32768"), ((32769,), "Context must be 1..32768"),
                      ((16, 0), "repeat 1..100000"), (("12x",), "Invalid context argument"),
                      ((16, "3y"), "Invalid repeat argument"),
                      ((16, 1, "bogus"), "Attention mode must be")):
        r = run("synthetic", *args)
        assert r.returncode == 1 and msg in r.stderr, (args, r.stderr)
    r = run("synthetic", 16, 1, "flash", shape="13b")
    assert r.returncode == 1 and "SI_SHAPE" in r.stderr


def test_colsoa_repack_files_and_manifest(oracle, tmp_path):
    """si_amd.repack writes repack_weights.py's three column-SoA files (the
    product's C repacker, byte-equal to the oracle's layout, which the
    reference build pins) and a manifest whose SHA-256 values match the
    files and the raw Q4_0 tensors."""
    import hashlib
    import json
    from oracle.oracle_py import make_shape as or_shape
    from si_amd import repack
    from tests.gpu_helpers import make_layer
    sd = si_amd.SHAPES["1.5b_ref"]
    lay = make_layer(oracle, or_shape(**sd), 4, ffn=False)
    for stem, key in (("q", "wq"), ("k", "wk"), ("v", "wv"), ("o", "wo")):
        lay[key].tofile(tmp_path / f"{stem}.q4_0")
    m = repack.repack(str(tmp_path))
    want = oracle.colsoa_repack(or_shape(**sd), lay)
    for (name, t), w in zip((("q", 0), ("kv", 1), ("o", 2)), want):
        data = (tmp_path / f"{name}.colsoa").read_bytes()
        assert data == w.tobytes(), name
        assert m["files"][name]["sha256"] == hashlib.sha256(data).hexdigest()
    for stem, key in (("q", "wq"), ("k", "wk"), ("v", "wv"), ("o", "wo")):
        assert m["raw_q4_sha256"][stem] == hashlib.sha256(lay[key].tobytes()).hexdigest()
    on_disk = json.loads((tmp_path / "manifest_colsoa.json").read_text())
    assert on_disk == m
    # shapes without the layout are refused (hdim 64)
    with pytest.raises(ValueError):
        repack.repack(str(tmp_path), "0.5b")
