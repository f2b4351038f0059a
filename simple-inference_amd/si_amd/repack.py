"""Weight layouts on disk and their SHA-256 manifests.

* ``repack(directory)``: the column-SoA tiles of the legacy fused path
  (``q.colsoa``, ``kv.colsoa``, ``o.colsoa``) from a layer's ``*.q4_0`` files,
  written by the product's C repacker (``si_colsoa_repack_host``), plus
  ``manifest_colsoa.json`` with the SHA-256 of every tile file and of the raw
  Q4_0 tensors: the role of ``repack_weights.py`` (its layout, lines 1-20; its
  manifest, lines 126-137).
* ``device_manifest(layer, tensors)``: the same record for the device repack
  ``si_layer_create`` makes (``include/si_abi.h``): per matrix the SHA-256 of
  the raw row-major Q4_0 bytes, of the device nibble and scale arrays, and
  whether ``si_q4_unpack`` of the device arrays gives the raw bytes back
  (the repack is lossless).

    python -m si_amd.repack --weights DIR [--shape 1.5b|0.5b|7b]
"""
import argparse
import ctypes
import hashlib
import json
import os

import numpy as np

from . import SHAPES, LayerHost, call, host_lib, lib, make_shape, ptr

_QK, _Q4 = 32, 18


def _digest(data):
    return hashlib.sha256(memoryview(np.ascontiguousarray(data)).cast("B")).hexdigest()


def _read_q4(directory, stem, rows, cols):
    path = os.path.join(directory, stem + ".q4_0")
    data = np.fromfile(path, dtype=np.uint8)
    want = rows * cols // _QK * _Q4
    if data.size != want:
        raise ValueError(f"{path}: {data.size} bytes, the shape needs {want}")
    return data


class _DeviceArray:
    """__cuda_array_interface__ over a device buffer the library owns."""

    def __init__(self, addr, count, typestr):
        self.__cuda_array_interface__ = {"shape": (count,), "typestr": typestr,
                                         "data": (int(addr), False), "version": 2}


def repack(directory, shape_name="1.5b_ref"):
    """Writes the three .colsoa files and manifest_colsoa.json; returns the
    manifest."""
    sd = SHAPES[shape_name]
    s = make_shape(**sd)
    H, QD, KVD = s.hidden, s.qheads * s.hdim, s.kvheads * s.hdim
    raw = {"q": _read_q4(directory, "q", QD, H), "k": _read_q4(directory, "k", KVD, H),
           "v": _read_q4(directory, "v", KVD, H), "o": _read_q4(directory, "o", H, QD)}
    Hl = host_lib()
    Hl.si_colsoa_bytes.restype = ctypes.c_size_t
    Hl.si_colsoa_bytes.argtypes = [ctypes.c_void_p, ctypes.c_int]
    sizes = [Hl.si_colsoa_bytes(ctypes.byref(s), i) for i in range(3)]
    if not all(sizes):
        raise ValueError(f"shape {shape_name} has no column-SoA layout (needs hdim 128 and "
                         "paired query heads)")
    host = LayerHost(wq=raw["q"].ctypes.data, wk=raw["k"].ctypes.data,
                     wv=raw["v"].ctypes.data, wo=raw["o"].ctypes.data)
    tiles = [np.zeros(n, np.uint8) for n in sizes]
    Hl.si_colsoa_repack_host.restype = None
    Hl.si_colsoa_repack_host.argtypes = [ctypes.c_void_p] * 5
    Hl.si_colsoa_repack_host(ctypes.byref(s), ctypes.byref(host), *[t.ctypes.data for t in tiles])
    files = {}
    for name, t in zip(("q", "kv", "o"), tiles):
        path = os.path.join(directory, name + ".colsoa")
        t.tofile(path)
        files[name] = {"file": name + ".colsoa", "bytes": int(t.size), "sha256": _digest(t)}
    manifest = {
        "format": "Q4_0 column-SoA v1",
        "shape": shape_name,
        "tile_outputs": 256,
        "group_bytes": 5120,
        "packed_column_bytes": 128,
        "scales": "fp32, the exact value of each Q4_0 block's fp16 scale",
        "files": files,
        "raw_q4_sha256": {name: _digest(a) for name, a in raw.items()},
    }
    with open(os.path.join(directory, "manifest_colsoa.json"), "w") as f:
        json.dump(manifest, f, indent=2)
        f.write("\n")
    return manifest


def device_manifest(layer, tensors):
    """SHA-256 record of a created layer's device weights (si_amd.Layer) and
    of the host tensors it was made from, with the unpack round trip."""
    import torch
    groups = {0: ("qkv", ("wq", "wk", "wv")), 1: ("o", ("wo",)), 2: ("gate_up", ("wgate", "wup")),
              3: ("down", ("wdown",))}
    out = {"format": "si_q4_repack v1 (qs [K/32][N][16], d tile-major)", "matrices": {}}
    for which, (name, parts) in groups.items():
        if any(tensors.get(p) is None for p in parts):
            continue
        raw = np.concatenate([np.ascontiguousarray(tensors[p], np.uint8).reshape(-1)
                              for p in parts])
        qs, d, tile, n, k = layer.weights(which)
        nd = lib().si_q4_scale_count(n, k, tile)
        dqs = torch.as_tensor(_DeviceArray(qs, n * k // 2, "|u1"), device="cuda")
        dd = torch.as_tensor(_DeviceArray(d, nd, "<i2"), device="cuda")
        back = torch.empty(raw.size, dtype=torch.uint8, device="cuda")
        call("si_q4_unpack", ptr(dqs), ptr(dd), n, k, tile, ptr(back), None)
        torch.cuda.synchronize()
        out["matrices"][name] = {
            "rows": n, "cols": k, "scale_tile": tile,
            "raw_q4_sha256": _digest(raw),
            "device_qs_sha256": _digest(dqs.cpu().numpy()),
            "device_d_sha256": _digest(dd.cpu().numpy()),
            "round_trip": bool(np.array_equal(back.cpu().numpy(), raw)),
        }
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--weights", default="weights", help="directory holding the *.q4_0 files")
    ap.add_argument("--shape", default="1.5b", choices=["1.5b", "0.5b", "7b"])
    a = ap.parse_args()
    m = repack(a.weights, "1.5b_ref" if a.shape == "1.5b" else a.shape)
    for name, f in m["files"].items():
        print(f"  {name}: {f['file']} {f['bytes']:,} B sha256 {f['sha256'][:16]}...")
    print("  manifest:", os.path.join(a.weights, "manifest_colsoa.json"))


if __name__ == "__main__":
    main()
