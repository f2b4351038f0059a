"""GGUF v2/v3 ingest of one Qwen2 layer (and a minimal writer).

Reads the single-file little-endian checkpoint format the reference's
extractor consumes (extract_weights.py:77-128 `read_index`, :131-141
`tensor_size`, :144-199 `extract`): header, metadata key/values, the tensor
index, then the tensor data from the first aligned offset.  Q4_0 weight
tensors are taken byte for byte (`Layer` repacks them on the GPU, the job
`repack_weights.py` does for the RVV build); F32 and F16 norm and bias
vectors become fp32 (the reference widens F16 the same way, :188-193); a
weight of any other type is refused, never dequantized (:161-163).
Missing norms and biases mean identity norm and zero bias (:172-176).
The file is memory-mapped for the index; each tensor is copied once into
ordinary process memory, because the HIP runtime cannot copy to the device
from a file mapping (its page registration fails there, and the error
surfaces at a later HIP call).

Unlike the reference (fixed at the 1.5B attention sublayer), the layer
shape comes from the qwen2.* metadata and the FFN tensors are read too.
"""
import mmap
import os
import struct

import numpy as np

# metadata value types (GGUF spec): scalar struct formats; 8 string, 9 array
_SCALAR = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q",
           12: "d"}
F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
TYPE_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 8: "Q8_0", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K",
              13: "Q5_K", 14: "Q6_K"}
MAX_STRING = 1 << 33
MAX_ARRAY = 100_000_000
MAX_DEPTH = 8


class GGUFError(ValueError):
    pass


class _Reader:
    """Little-endian cursor over a bytes-like object (bounds-checked)."""

    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def take(self, n):
        if n < 0 or self.pos + n > len(self.buf):
            raise GGUFError("truncated GGUF file")
        out = self.buf[self.pos:self.pos + n]
        self.pos += n
        return out

    def num(self, fmt):
        return struct.unpack("<" + fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self, wanted=True):
        n = self.num("Q")
        if n > MAX_STRING:
            raise GGUFError("unreasonably long GGUF string")
        raw = self.take(n)
        return bytes(raw).decode("utf-8") if wanted else None

    def value(self, typ, wanted=True, depth=0):
        """A metadata value (skipped, None, when not wanted); arrays of
        scalars come back as numpy arrays."""
        if depth > MAX_DEPTH:
            raise GGUFError("GGUF metadata nesting too deep")
        if typ in _SCALAR:
            v = self.num(_SCALAR[typ])
            return v if wanted else None
        if typ == 8:
            return self.string(wanted)
        if typ == 9:
            inner = self.num("I")
            count = self.num("Q")
            if count > MAX_ARRAY:
                raise GGUFError("unreasonably long GGUF array")
            if inner in _SCALAR:
                fmt = "<" + _SCALAR[inner]
                raw = self.take(count * struct.calcsize(fmt))
                return np.frombuffer(raw, np.dtype(fmt)).copy() if wanted else None
            items = [self.value(inner, wanted, depth + 1) for _ in range(count)]
            return items if wanted else None
        raise GGUFError(f"unsupported GGUF metadata type {typ}")


def tensor_nbytes(dims, typ):
    """Bytes of a tensor's data (extract_weights.py:131-141)."""
    n = int(np.prod(dims, dtype=np.int64))
    if typ in (Q4_0, Q8_0):
        if n % 32:
            raise GGUFError(f"{TYPE_NAMES[typ]} element count {n} not divisible by 32")
        return n // 32 * (18 if typ == Q4_0 else 34)
    if typ == F32:
        return n * 4
    if typ == F16:
        return n * 2
    raise GGUFError(f"unsupported tensor type {TYPE_NAMES.get(typ, typ)}")


def read_index(buf):
    """(metadata dict, {name: (dims, type, offset)}, data start) of a GGUF
    image (extract_weights.py:77-128).  dims are in GGUF order: dims[0] is
    the row length (K) of a matrix, dims[1] the number of rows (N)."""
    r = _Reader(buf)
    if bytes(r.take(4)) != b"GGUF":
        raise GGUFError("expected a little-endian GGUF file (magic GGUF)")
    version = r.num("I")
    if version not in (2, 3):
        raise GGUFError(f"only GGUF v2/v3 are supported; found v{version}")
    ntensors, nmeta = r.num("Q"), r.num("Q")
    meta = {}
    for _ in range(nmeta):
        key = r.string()
        # the model's own keys; others (the tokenizer's large arrays) are
        # skipped without building them
        wanted = key.startswith(("general.", "qwen2."))
        v = r.value(r.num("I"), wanted)
        if wanted:
            meta[key] = v
    tensors = {}
    for _ in range(ntensors):
        name = r.string()
        rank = r.num("I")
        if not 1 <= rank <= 8:
            raise GGUFError(f"unexpected rank {rank} for {name}")
        dims = [r.num("Q") for _ in range(rank)]
        typ, off = r.num("I"), r.num("Q")
        if name in tensors:
            raise GGUFError(f"duplicate tensor {name}")
        tensors[name] = (dims, typ, off)
    align = int(meta.get("general.alignment", 32))
    if align < 8 or align % 8:
        raise GGUFError(f"unexpected GGUF alignment {align}")
    start = (r.pos + align - 1) // align * align
    return meta, tensors, start


class GGUFFile:
    """A memory-mapped GGUF file and its index."""

    def __init__(self, path):
        self.path = path
        with open(path, "rb") as f:
            size = os.fstat(f.fileno()).st_size
            if size == 0:
                raise GGUFError("empty GGUF file")
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        self.size = size
        self.meta, self.tensors, self.data_start = read_index(memoryview(self._mm))

    def close(self):
        """Unmaps the file, unless tensor views still use it (then the
        mapping goes when they do)."""
        if self._mm is not None:
            try:
                self._mm.close()
            except BufferError:
                pass
            self._mm = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def raw(self, name):
        """The tensor's bytes as a read-only uint8 view of the mapping."""
        dims, typ, off = self.tensors[name]
        n = tensor_nbytes(dims, typ)
        begin = self.data_start + off
        if off < 0 or begin + n > self.size:
            raise GGUFError(f"{name} data range exceeds the GGUF file")
        return np.frombuffer(self._mm, np.uint8, n, begin)

    def matrix_q4(self, name, n, k):
        """A Q4_0 weight of n rows by k inputs as row-major [n][k/32*18]
        (a copy in process memory)."""
        dims, typ, _ = self.tensors[name]
        if dims != [k, n]:
            raise GGUFError(f"{name} has dims {dims}, expected {[k, n]} (GGUF order)")
        if typ != Q4_0:
            raise GGUFError(f"{name} is {TYPE_NAMES.get(typ, typ)}, not Q4_0: a Q4_0 GGUF is "
                            "needed (weights are never dequantized)")
        return np.array(self.raw(name).reshape(n, k // 32 * 18))

    def vector_f32(self, name, n):
        """An F32 or F16 vector of n values as fp32 (F16 widened exactly)."""
        dims, typ, _ = self.tensors[name]
        if dims != [n]:
            raise GGUFError(f"{name} has dims {dims}, expected {[n]}")
        raw = self.raw(name)
        if typ == F32:
            return raw.view("<f4").astype(np.float32)
        if typ == F16:
            return raw.view("<f2").astype(np.float32)
        raise GGUFError(f"{name} must be F32/F16, got {TYPE_NAMES.get(typ, typ)}")


def shape_meta(meta):
    """The layer shape (si_amd.make_shape keywords) from qwen2.* metadata."""
    arch = meta.get("general.architecture", "qwen2")
    if arch != "qwen2":
        raise GGUFError(f"expected the qwen2 architecture, got {arch}")
    need = ["qwen2.embedding_length", "qwen2.attention.head_count",
            "qwen2.attention.head_count_kv"]
    for k in need:
        if k not in meta:
            raise GGUFError(f"metadata {k} missing")
    hidden = int(meta["qwen2.embedding_length"])
    qheads = int(meta["qwen2.attention.head_count"])
    kvheads = int(meta["qwen2.attention.head_count_kv"])
    hdim = int(meta.get("qwen2.attention.key_length", hidden // qheads))
    if int(meta.get("qwen2.attention.value_length", hdim)) != hdim:
        raise GGUFError("key and value head sizes differ")
    if int(meta.get("qwen2.rope.dimension_count", hdim)) != hdim:
        raise GGUFError("partial rotary embeddings are not supported")
    return dict(hidden=hidden, qheads=qheads, kvheads=kvheads, hdim=hdim,
                ffn=int(meta.get("qwen2.feed_forward_length", 0)),
                rope_base=float(meta.get("qwen2.rope.freq_base", 1e6)),
                rms_eps=float(meta.get("qwen2.attention.layer_norm_rms_epsilon", 1e-6)))


def layer_names(layer):
    """GGUF tensor names of one Qwen2 block, by si_layer_host_t field."""
    b = f"blk.{layer}."
    return dict(wq=b + "attn_q.weight", wk=b + "attn_k.weight", wv=b + "attn_v.weight",
                wo=b + "attn_output.weight", norm=b + "attn_norm.weight",
                bq=b + "attn_q.bias", bk=b + "attn_k.bias", bv=b + "attn_v.bias",
                post_norm=b + "ffn_norm.weight", wgate=b + "ffn_gate.weight",
                wup=b + "ffn_up.weight", wdown=b + "ffn_down.weight")


def load_layer(gf, layer, ffn=True):
    """(shape keywords, host tensors for si_amd.Layer) of block `layer`.

    Every required tensor is checked (presence, GGUF dims, type, data range)
    before any is returned.  ffn=False reads the attention sublayer only
    (the reference's extraction); the FFN weights are then absent."""
    sd = shape_meta(gf.meta)
    H, QD = sd["hidden"], sd["qheads"] * sd["hdim"]
    KVD, F = sd["kvheads"] * sd["hdim"], sd["ffn"]
    names = layer_names(layer)
    mats = dict(wq=(QD, H), wk=(KVD, H), wv=(KVD, H), wo=(H, QD))
    vecs = dict(norm=H, bq=QD, bk=KVD, bv=KVD)
    if ffn:
        if F <= 0:
            raise GGUFError("metadata qwen2.feed_forward_length missing")
        mats.update(wgate=(F, H), wup=(F, H), wdown=(H, F))
        vecs.update(post_norm=H)
    else:
        sd["ffn"] = 0
    for key in mats:
        if names[key] not in gf.tensors:
            raise GGUFError(f"required tensor not found: {names[key]}")
    out = {key: gf.matrix_q4(names[key], n, k) for key, (n, k) in mats.items()}
    for key, n in vecs.items():
        out[key] = gf.vector_f32(names[key], n) if names[key] in gf.tensors else None
    return sd, out


# ---------------------------------------------------------------------------
# writer (fixtures, tooling): the same layout, little-endian, version 3
# ---------------------------------------------------------------------------
def _pack_string(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(v):
    """(type, bytes) of a metadata value: str, bool, int (u32, or u64 when
    large), float (f32), or (type, value) to force a scalar type."""
    if isinstance(v, tuple):
        typ, x = v
        return typ, (_pack_string(x) if typ == 8 else struct.pack("<" + _SCALAR[typ], x))
    if isinstance(v, str):
        return 8, _pack_string(v)
    if isinstance(v, bool):
        return 7, struct.pack("<?", v)
    if isinstance(v, int):
        return (4, struct.pack("<I", v)) if 0 <= v < 1 << 32 else (11, struct.pack("<q", v))
    if isinstance(v, float):
        return 6, struct.pack("<f", v)
    if isinstance(v, list):
        items = [_pack_value(x) for x in v]
        inner = items[0][0] if items else 4
        if any(t != inner for t, _ in items):
            raise GGUFError("GGUF arrays hold one element type")
        return 9, struct.pack("<IQ", inner, len(items)) + b"".join(b for _, b in items)
    raise GGUFError(f"cannot encode metadata value {v!r}")


def write_gguf(path, meta, tensors, alignment=32, version=3):
    """meta: {key: value}; tensors: {name: (type, dims in GGUF order, data)}
    with data a bytes-like of exactly tensor_nbytes(dims, type) bytes."""
    meta = dict(meta)
    if alignment != 32:
        meta["general.alignment"] = (4, alignment)
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for k, v in meta.items():
        typ, body = _pack_value(v)
        head += _pack_string(k) + struct.pack("<I", typ) + body
    offs, off = [], 0
    for name, (typ, dims, data) in tensors.items():
        n = tensor_nbytes(dims, typ)
        if len(memoryview(data).cast("B")) != n:
            raise GGUFError(f"{name}: {len(data)} bytes for {n}")
        offs.append(off)
        off = (off + n + alignment - 1) // alignment * alignment
    for (name, (typ, dims, _)), o in zip(tensors.items(), offs):
        head += _pack_string(name) + struct.pack("<I", len(dims))
        head += struct.pack(f"<{len(dims)}Q", *dims) + struct.pack("<IQ", typ, o)
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * ((-len(head)) % alignment))
        for (name, (typ, dims, data)), o in zip(tensors.items(), offs):
            mv = memoryview(data).cast("B")
            f.write(mv)
            f.write(b"\0" * ((-len(mv)) % alignment))


def layer_tensors_gguf(sd, host, layer=0, f16_vectors=False):
    """The {name: (type, dims, data)} of one block from si_amd.Layer host
    tensors (row-major Q4_0 matrices, fp32 vectors); f16_vectors stores the
    norm and bias vectors as F16."""
    names = layer_names(layer)
    out = {}
    for key, arr in host.items():
        if arr is None:
            continue
        a = np.ascontiguousarray(arr)
        if a.dtype == np.uint8:
            n = a.shape[0]
            k = a.shape[1] // 18 * 32
            out[names[key]] = (Q4_0, [k, n], a)
        elif f16_vectors:
            out[names[key]] = (F16, [a.size], a.astype("<f2"))
        else:
            out[names[key]] = (F32, [a.size], a.astype("<f4"))
    return out


def layer_meta(sd):
    """qwen2.* metadata of a layer shape (si_amd.make_shape keywords)."""
    m = {"general.architecture": "qwen2",
         "qwen2.embedding_length": sd["hidden"],
         "qwen2.attention.head_count": sd["qheads"],
         "qwen2.attention.head_count_kv": sd["kvheads"],
         "qwen2.attention.key_length": sd["hdim"],
         "qwen2.attention.value_length": sd["hdim"],
         "qwen2.rope.dimension_count": sd["hdim"],
         "qwen2.rope.freq_base": float(sd.get("rope_base", 1e6)),
         "qwen2.attention.layer_norm_rms_epsilon": float(sd.get("rms_eps", 1e-6))}
    if sd.get("ffn", 0):
        m["qwen2.feed_forward_length"] = sd["ffn"]
    return m
