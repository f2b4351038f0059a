"""ctypes binding of the CPU parity oracle (oracle/libsi_oracle.so) and, when
built, of the reference's own portable path (oracle/_ref/libsi_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
the cpu_baseline leg of bench.py, always as the checker or the timed CPU
baseline, never on the product path.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libsi_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libsi_ref.so")

QK = 32
Q4_BYTES = 18
Q8_DTYPE = np.dtype([("d", "<u2"), ("qs", "i1", (QK,))])  # defines.h:27-28, 34 B
assert Q8_DTYPE.itemsize == 34

_P = ctypes.c_void_p


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class Shape(ctypes.Structure):
    """or_shape_t: defines.h:16-25 as runtime values."""
    _fields_ = [("hidden", ctypes.c_int), ("qheads", ctypes.c_int),
                ("kvheads", ctypes.c_int), ("hdim", ctypes.c_int),
                ("ffn", ctypes.c_int), ("rope_base", ctypes.c_float),
                ("rms_eps", ctypes.c_float)]


class _Layer(ctypes.Structure):
    _fields_ = [(n, _P) for n in ("wq", "wk", "wv", "wo", "norm", "bq", "bk", "bv",
                                  "post_norm", "wgate", "wup", "wdown")]


class _Capture(ctypes.Structure):
    _fields_ = [(n, _P) for n in ("normed", "xq", "q", "k", "v", "attn", "attq",
                                  "attn_out", "h", "normed2", "xq2", "gate", "up",
                                  "act", "actq", "ffn_out")]


SHAPES = {
    # Qwen2.5-0.5B / 7B shapes used by the benchmark configurations.
    "0.5b": dict(hidden=896, qheads=14, kvheads=2, hdim=64, ffn=4864),
    "7b": dict(hidden=3584, qheads=28, kvheads=4, hdim=128, ffn=18944),
    # The only shape the reference compiles for (defines.h:16-25).
    "1.5b_ref": dict(hidden=1536, qheads=12, kvheads=2, hdim=128, ffn=0),
}


def make_shape(hidden, qheads, kvheads, hdim, ffn=0, rope_base=1e6, rms_eps=1e-6):
    return Shape(hidden, qheads, kvheads, hdim, ffn, rope_base, rms_eps)


class Oracle:
    """Thin numpy wrapper; every method mirrors a reference function."""

    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = ctypes.CDLL(path)
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f32_to_f16_array.argtypes = [_P, _P, ctypes.c_size_t]
        L.or_f16_to_f32_array.argtypes = [_P, _P, ctypes.c_size_t]
        L.or_rng_seed.argtypes = [ctypes.c_uint32]
        L.or_rng_float.restype = ctypes.c_float
        L.or_rng_fill.argtypes = [_P, ctypes.c_size_t, ctypes.c_float]
        L.or_quantize_q8.argtypes = [_P, _P, ctypes.c_int]
        L.or_dot_32_q4q8.restype = ctypes.c_int32
        L.or_dot_32_q4q8.argtypes = [_P, _P]
        L.or_block_dots.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, _P]
        L.or_matvec_q4q8.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, _P, _P]
        L.or_rmsnorm.argtypes = [_P, _P, _P, ctypes.c_int, ctypes.c_float]
        L.or_rope.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        L.or_rope_table.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_float, _P, _P]
        L.or_attention_flash.argtypes = [ctypes.POINTER(Shape), _P, _P, _P, ctypes.c_int, _P]
        L.or_attention_standard.argtypes = [ctypes.POINTER(Shape), _P, _P, _P,
                                            ctypes.c_int, _P, _P]
        L.or_swiglu.argtypes = [_P, _P, _P, ctypes.c_int]
        L.or_run_layer.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(_Layer), _P, _P,
                                   _P, ctypes.c_int, _P, ctypes.c_int, _P,
                                   ctypes.POINTER(_Capture)]
        L.or_layer_decode.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(_Layer), _P,
                                      _P, _P, ctypes.c_int, _P, ctypes.POINTER(_Capture)]
        L.or_layer_prefill.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(_Layer), _P,
                                       ctypes.c_int, ctypes.c_int, _P, _P, _P,
                                       ctypes.c_int, ctypes.c_int, _P]
        L.or_colsoa_bytes.restype = ctypes.c_size_t
        L.or_colsoa_bytes.argtypes = [ctypes.POINTER(Shape), ctypes.c_int]
        L.or_colsoa_repack.argtypes = [ctypes.POINTER(Shape)] + [_P] * 7
        L.or_fused_column_matvec.argtypes = [_P, _P, ctypes.c_int, _P, _P, _P, ctypes.c_int]
        L.or_attention_pair.argtypes = [ctypes.POINTER(Shape), _P, _P, _P, ctypes.c_int,
                                        ctypes.c_int, _P]
        L.or_run_layer_legacy_fused.argtypes = [ctypes.POINTER(Shape), ctypes.POINTER(_Layer),
                                                _P, _P, _P, _P, _P, _P, ctypes.c_int, _P, _P,
                                                _P]
        L.or_quantize_q4_0.argtypes = [_P, _P, ctypes.c_int]
        L.or_dequantize_q4_0.argtypes = [_P, _P, ctypes.c_int]

    # ---- numerics ----
    def f32_to_f16(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, np.uint16)
        self.lib.or_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
        return out

    def f16_to_f32(self, h):
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.shape, np.float32)
        self.lib.or_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
        return out

    def rng_floats(self, seed, n, scale=1.0):
        self.lib.or_rng_seed(seed)
        out = np.empty(n, np.float32)
        self.lib.or_rng_fill(_ptr(out), n, scale)
        return out

    # ---- kernels ----
    def quantize_q8(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        out = np.zeros(x.size // QK, Q8_DTYPE)
        self.lib.or_quantize_q8(_ptr(x), _ptr(out), x.size)
        return out

    def dot_32(self, wblock, a):
        wblock = np.ascontiguousarray(wblock, np.uint8)
        a = np.ascontiguousarray(a, np.int8)
        return self.lib.or_dot_32_q4q8(_ptr(wblock), _ptr(a))

    def block_dots(self, w, xq, k, n):
        out = np.empty((n, k // QK), np.int32)
        self.lib.or_block_dots(_ptr(w), _ptr(xq), k, n, _ptr(out))
        return out

    def matvec(self, w, xq, k, n, bias=None):
        out = np.empty(n, np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.lib.or_matvec_q4q8(_ptr(w), _ptr(xq), k, n, _ptr(b), _ptr(out))
        return out

    def rmsnorm(self, x, w=None, eps=1e-6):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        wv = None if w is None else np.ascontiguousarray(w, np.float32)
        self.lib.or_rmsnorm(_ptr(x), _ptr(wv), _ptr(out), x.size, eps)
        return out

    def rope(self, heads, nheads, hdim, pos, base=1e6):
        h = np.array(heads, np.float32, copy=True).reshape(-1)
        self.lib.or_rope(_ptr(h), nheads, hdim, pos, base)
        return h

    def rope_table(self, pos0, npos, hdim, base=1e6):
        c = np.empty((npos, hdim // 2), np.float32)
        s = np.empty((npos, hdim // 2), np.float32)
        self.lib.or_rope_table(pos0, npos, hdim, base, _ptr(c), _ptr(s))
        return c, s

    def attention_flash(self, shape, q, kc, vc, context):
        out = np.empty(shape.qheads * shape.hdim, np.float32)
        self.lib.or_attention_flash(ctypes.byref(shape), _ptr(q), _ptr(kc), _ptr(vc),
                                    context, _ptr(out))
        return out

    def attention_standard(self, shape, q, kc, vc, context, with_scores=False):
        """out [qheads*hdim]; with_scores: also the normalised scores
        [qheads][context] the reference leaves in its workspace."""
        out = np.empty(shape.qheads * shape.hdim, np.float32)
        scores = np.empty(shape.qheads * max(context, 1), np.float32)
        self.lib.or_attention_standard(ctypes.byref(shape), _ptr(q), _ptr(kc), _ptr(vc),
                                       context, _ptr(out), _ptr(scores))
        if with_scores:
            return out, scores[:shape.qheads * context].reshape(shape.qheads, context)
        return out

    def swiglu(self, g, u):
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        out = np.empty_like(g)
        self.lib.or_swiglu(_ptr(g), _ptr(u), _ptr(out), g.size)
        return out

    def quantize_q4_0(self, w):
        w = np.ascontiguousarray(w, np.float32)
        rows = w.shape[0] if w.ndim == 2 else 1
        out = np.empty((rows, w.size // rows // QK * Q4_BYTES), np.uint8)
        self.lib.or_quantize_q4_0(_ptr(w), _ptr(out), w.size)
        return out

    def dequantize_q4_0(self, q, count):
        out = np.empty(count, np.float32)
        self.lib.or_dequantize_q4_0(_ptr(np.ascontiguousarray(q)), _ptr(out), count)
        return out

    # ---- column-SoA tiles and the legacy fused path (hdim 128) ----
    def colsoa_repack(self, shape, layer):
        """(q, kv, o) tile bytes of repack_weights.py's layout."""
        bufs = [np.zeros(self.lib.or_colsoa_bytes(ctypes.byref(shape), i), np.uint8)
                for i in range(3)]
        w = [np.ascontiguousarray(layer[k], np.uint8) for k in ("wq", "wk", "wv", "wo")]
        self.lib.or_colsoa_repack(ctypes.byref(shape), *[_ptr(a) for a in w],
                                  *[_ptr(b) for b in bufs])
        return tuple(bufs)

    def fused_column_matvec(self, tile, xq, nblocks, bias_lo=None, bias_hi=None, out=None,
                            add=False):
        y = np.zeros(256, np.float32) if out is None else np.array(out, np.float32, copy=True)
        bl = None if bias_lo is None else np.ascontiguousarray(bias_lo, np.float32)
        bh = None if bias_hi is None else np.ascontiguousarray(bias_hi, np.float32)
        self.lib.or_fused_column_matvec(_ptr(np.ascontiguousarray(tile, np.uint8)),
                                        _ptr(np.ascontiguousarray(xq)), nblocks, _ptr(bl),
                                        _ptr(bh), _ptr(y), int(add))
        return y

    def attention_pair(self, shape, qpair, kc, vc, context, group):
        out = np.empty(2 * shape.hdim, np.float32)
        self.lib.or_attention_pair(ctypes.byref(shape),
                                   _ptr(np.ascontiguousarray(qpair, np.float32)), _ptr(kc),
                                   _ptr(vc), context, group, _ptr(out))
        return out

    def run_layer_legacy_fused(self, shape, layer, tiles, x, kc, vc, context):
        """(out, attention capture, Q8 capture); kc/vc get the new row."""
        lay, keep = self._layer(layer)
        out = np.empty(shape.hidden, np.float32)
        att = np.empty(shape.qheads * shape.hdim, np.float32)
        q8 = np.zeros(shape.qheads * shape.hdim // QK, Q8_DTYPE)
        self.lib.or_run_layer_legacy_fused(ctypes.byref(shape), ctypes.byref(lay),
                                           *[_ptr(t) for t in tiles], _ptr(x), _ptr(kc),
                                           _ptr(vc), context, _ptr(out), _ptr(att), _ptr(q8))
        del keep
        return out, att, q8

    # ---- layers ----
    @staticmethod
    def _layer(layer):
        keep = []
        vals = {}
        for name, _ in _Layer._fields_:
            arr = layer.get(name)
            if arr is not None:
                arr = np.ascontiguousarray(arr)
                keep.append(arr)
                vals[name] = arr.ctypes.data
        return _Layer(**vals), keep

    @staticmethod
    def capture_buffers(shape):
        H, QD = shape.hidden, shape.qheads * shape.hdim
        KVD, F = shape.kvheads * shape.hdim, shape.ffn
        bufs = dict(normed=np.zeros(H, np.float32), xq=np.zeros(H // QK, Q8_DTYPE),
                    q=np.zeros(QD, np.float32), k=np.zeros(KVD, np.float32),
                    v=np.zeros(KVD, np.float32), attn=np.zeros(QD, np.float32),
                    attq=np.zeros(QD // QK, Q8_DTYPE), attn_out=np.zeros(H, np.float32))
        if F:
            bufs.update(h=np.zeros(H, np.float32), normed2=np.zeros(H, np.float32),
                        xq2=np.zeros(H // QK, Q8_DTYPE), gate=np.zeros(F, np.float32),
                        up=np.zeros(F, np.float32), act=np.zeros(F, np.float32),
                        actq=np.zeros(F // QK, Q8_DTYPE), ffn_out=np.zeros(H, np.float32))
        cap = _Capture(**{k: v.ctypes.data for k, v in bufs.items()})
        return cap, bufs

    def run_layer(self, shape, layer, x, kc, vc, context, method=1, capture=False):
        lay, keep = self._layer(layer)
        out = np.empty(shape.hidden, np.float32)
        cap, bufs = self.capture_buffers(shape) if capture else (None, None)
        self.lib.or_run_layer(ctypes.byref(shape), ctypes.byref(lay), _ptr(x), _ptr(kc),
                              _ptr(vc), context, _ptr(out), method, None,
                              ctypes.byref(cap) if cap else None)
        del keep
        return (out, bufs) if capture else out

    def layer_decode(self, shape, layer, x, kc, vc, context, capture=False):
        lay, keep = self._layer(layer)
        out = np.empty(shape.hidden, np.float32)
        cap, bufs = self.capture_buffers(shape) if capture else (None, None)
        self.lib.or_layer_decode(ctypes.byref(shape), ctypes.byref(lay), _ptr(x), _ptr(kc),
                                 _ptr(vc), context, _ptr(out),
                                 ctypes.byref(cap) if cap else None)
        del keep
        return (out, bufs) if capture else out

    def layer_prefill(self, shape, layer, x, ntok, prefix, kc, vc, rows=None, full=True):
        lay, keep = self._layer(layer)
        r = None if rows is None else np.ascontiguousarray(rows, np.int32)
        n = ntok if r is None else r.size
        out = np.empty((n, shape.hidden), np.float32)
        self.lib.or_layer_prefill(ctypes.byref(shape), ctypes.byref(lay), _ptr(x), ntok,
                                  prefix, _ptr(kc), _ptr(vc), _ptr(r),
                                  0 if r is None else r.size, int(full), _ptr(out))
        del keep
        return out


class Reference:
    """The reference's own portable path compiled from /root/reference
    (oracle/_ref); fixed at its compile-time 1.5B shape."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = ctypes.CDLL(path)
        for n in ("si_ref_hidden", "si_ref_qheads", "si_ref_kvheads", "si_ref_hdim"):
            getattr(L, n).restype = ctypes.c_int
        L.si_ref_f32_to_f16_array.argtypes = [_P, _P, ctypes.c_size_t]
        L.si_ref_f16_to_f32_array.argtypes = [_P, _P, ctypes.c_size_t]
        L.si_ref_rng_seed.argtypes = [ctypes.c_uint32]
        L.si_ref_random_float.restype = ctypes.c_float
        L.si_ref_fill_kv_history.argtypes = [_P, _P, ctypes.c_int]
        L.si_ref_quantize_q8.argtypes = [_P, _P, ctypes.c_int]
        L.si_ref_dot_32_q4q8.restype = ctypes.c_int32
        L.si_ref_dot_32_q4q8.argtypes = [_P, _P]
        L.si_ref_matvec_q4q8.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, _P, _P]
        L.si_ref_rmsnorm.argtypes = [_P, _P, _P]
        L.si_ref_rope.argtypes = [_P, ctypes.c_int, ctypes.c_int]
        L.si_ref_attention_flash.argtypes = [_P, _P, _P, ctypes.c_int, _P]
        L.si_ref_attention_standard.argtypes = [_P, _P, _P, ctypes.c_int, _P, _P]
        L.si_ref_run_layer.argtypes = [_P] * 11 + [ctypes.c_int, _P, ctypes.c_int, _P, _P, _P]
        L.si_ref_fused_column_matvec.argtypes = [_P, _P, ctypes.c_int, _P, _P, _P,
                                                 ctypes.c_int]
        L.si_ref_fused_attention_pair.argtypes = [_P, _P, _P, ctypes.c_int, ctypes.c_int, _P]
        L.si_ref_run_layer_fused.argtypes = [_P] * 14 + [ctypes.c_int, _P, _P, _P]
        self.hidden = L.si_ref_hidden()
        self.qheads = L.si_ref_qheads()
        self.kvheads = L.si_ref_kvheads()
        self.hdim = L.si_ref_hdim()

    def shape(self):
        return make_shape(self.hidden, self.qheads, self.kvheads, self.hdim)

    def f32_to_f16(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, np.uint16)
        self.lib.si_ref_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
        return out

    def f16_to_f32(self, h):
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty(h.shape, np.float32)
        self.lib.si_ref_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
        return out

    def rng_floats(self, seed, n, scale=1.0):
        self.lib.si_ref_rng_seed(seed)
        return np.array([self.lib.si_ref_random_float() * scale for _ in range(n)],
                        np.float32)

    def quantize_q8(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.zeros(x.size // QK, Q8_DTYPE)
        self.lib.si_ref_quantize_q8(_ptr(x), _ptr(out), x.size)
        return out

    def dot_32(self, wblock, a):
        return self.lib.si_ref_dot_32_q4q8(_ptr(np.ascontiguousarray(wblock, np.uint8)),
                                           _ptr(np.ascontiguousarray(a, np.int8)))

    def matvec(self, w, xq, k, n, bias=None):
        out = np.empty(n, np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, np.float32)
        self.lib.si_ref_matvec_q4q8(_ptr(w), _ptr(xq), k, n, _ptr(b), _ptr(out))
        return out

    def rmsnorm(self, x, w=None):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        wv = None if w is None else np.ascontiguousarray(w, np.float32)
        self.lib.si_ref_rmsnorm(_ptr(x), _ptr(wv), _ptr(out))
        return out

    def rope(self, heads, nheads, pos):
        h = np.array(heads, np.float32, copy=True).reshape(-1)
        self.lib.si_ref_rope(_ptr(h), nheads, pos)
        return h

    def attention_flash(self, q, kc, vc, context):
        out = np.empty(self.qheads * self.hdim, np.float32)
        self.lib.si_ref_attention_flash(_ptr(q), _ptr(kc), _ptr(vc), context, _ptr(out))
        return out

    def attention_standard(self, q, kc, vc, context, with_scores=False):
        out = np.empty(self.qheads * self.hdim, np.float32)
        scores = np.empty(self.qheads * max(context, 1), np.float32)
        self.lib.si_ref_attention_standard(_ptr(q), _ptr(kc), _ptr(vc), context,
                                           _ptr(out), _ptr(scores))
        if with_scores:
            return out, scores[:self.qheads * context].reshape(self.qheads, context)
        return out

    def run_layer(self, layer, x, kc, vc, context, method=1):
        out = np.empty(self.hidden, np.float32)
        attn = np.empty(self.qheads * self.hdim, np.float32)
        q8 = np.zeros(self.qheads * self.hdim // QK, Q8_DTYPE)
        scores = np.empty(self.qheads * max(context, 1), np.float32)
        g = layer.get
        self.lib.si_ref_run_layer(_ptr(g("wq")), _ptr(g("wk")), _ptr(g("wv")), _ptr(g("wo")),
                                  _ptr(g("norm")), _ptr(g("bq")), _ptr(g("bk")),
                                  _ptr(g("bv")), _ptr(x), _ptr(kc), _ptr(vc), context,
                                  _ptr(out), method, _ptr(scores), _ptr(attn), _ptr(q8))
        return out, attn, q8


    def fused_column_matvec(self, tile, xq, nblocks, bias_lo=None, bias_hi=None, out=None,
                            add=False):
        y = np.zeros(256, np.float32) if out is None else np.array(out, np.float32, copy=True)
        bl = None if bias_lo is None else np.ascontiguousarray(bias_lo, np.float32)
        bh = None if bias_hi is None else np.ascontiguousarray(bias_hi, np.float32)
        self.lib.si_ref_fused_column_matvec(_ptr(np.ascontiguousarray(tile, np.uint8)),
                                            _ptr(np.ascontiguousarray(xq)), nblocks, _ptr(bl),
                                            _ptr(bh), _ptr(y), int(add))
        return y

    def attention_pair(self, qpair, kc, vc, context, group):
        out = np.empty(2 * self.hdim, np.float32)
        self.lib.si_ref_fused_attention_pair(_ptr(np.ascontiguousarray(qpair, np.float32)),
                                             _ptr(kc), _ptr(vc), context, group, _ptr(out))
        return out

    def run_layer_fused(self, layer, tiles, x, kc, vc, context):
        out = np.empty(self.hidden, np.float32)
        attn = np.empty(self.qheads * self.hdim, np.float32)
        q8 = np.zeros(self.qheads * self.hdim // QK, Q8_DTYPE)
        g = layer.get
        self.lib.si_ref_run_layer_fused(_ptr(g("wq")), _ptr(g("wk")), _ptr(g("wv")),
                                        _ptr(g("wo")), _ptr(g("norm")), _ptr(g("bq")),
                                        _ptr(g("bk")), _ptr(g("bv")), *[_ptr(t) for t in tiles],
                                        _ptr(x), _ptr(kc), _ptr(vc), context, _ptr(out),
                                        _ptr(attn), _ptr(q8))
        return out, attn, q8


def have_reference():
    return os.path.exists(REF_SO)
