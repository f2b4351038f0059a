"""Python plumbing over the MI355X hot-path libraries (ctypes).

The product is the C ABI in lib/libsi_amd.so (include/si_abi.h) and the C11
host mirror in lib/libsi_host.so (include/si_host.h).  This module only binds
them for tests and the benchmark; torch supplies device memory and streams.
It fails loudly when the native libraries are missing: there is no fallback.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
LIB_DIR = os.path.join(PKG, "lib")
AMD_SO = os.path.join(LIB_DIR, "libsi_amd.so")
HOST_SO = os.path.join(LIB_DIR, "libsi_host.so")
ROOT = os.path.dirname(PKG)
INCLUDE_DIR = os.path.join(ROOT, "include")

QK = 32
Q8_DTYPE = np.dtype([("d", "<u2"), ("qs", "i1", (QK,))])  # defines.h:27-28

SI_OK, SI_ERR_ARG, SI_ERR_HIP, SI_ERR_STATE, SI_ERR_NOMEM = range(5)
SI_LAYER_FULL, SI_LAYER_ATTN_ONLY, SI_LAYER_EXACT, SI_LAYER_ATTN_STANDARD = 0, 1, 2, 4
SI_LAYER_CAPTURE = 8
SI_GEMM_EXACT = 1
SI_GEMM_F16 = 2
SI_GEMM_TILED_A = 4
SI_GEMM_F6 = 8
BUFFERS = ["NORMED", "XQ_QS", "XQ_D", "XQ_S", "QKV", "Q", "ATTN", "ATTQ_QS", "ATTQ_D",
           "ATTQ_S", "ATTN_OUT", "H", "NORMED2", "XQ2_QS", "XQ2_D", "XQ2_S", "GU", "ACT",
           "ACTQ_QS", "ACTQ_D", "ACTQ_S", "ACTQ_TQ", "ACTQ_TD"]
BUF = {n: i for i, n in enumerate(BUFFERS)}
PHASES = ["rms_q8", "qkv_proj", "rope_kv", "attention_q8", "out_proj", "post_norm_q8",
          "gate_up", "swiglu_q8", "down_proj"]

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t


class SiError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"si error {code}: {msg}")
        self.code = code


class Shape(ctypes.Structure):
    """si_shape_t (include/si_abi.h)."""
    _fields_ = [("hidden", _I), ("qheads", _I), ("kvheads", _I), ("hdim", _I), ("ffn", _I),
                ("rope_base", _F), ("rms_eps", _F)]


def make_shape(hidden, qheads, kvheads, hdim, ffn=0, rope_base=1e6, rms_eps=1e-6):
    return Shape(hidden, qheads, kvheads, hdim, ffn, rope_base, rms_eps)


SHAPES = {
    "0.5b": dict(hidden=896, qheads=14, kvheads=2, hdim=64, ffn=4864),
    "7b": dict(hidden=3584, qheads=28, kvheads=4, hdim=128, ffn=18944),
    "1.5b_ref": dict(hidden=1536, qheads=12, kvheads=2, hdim=128, ffn=0),
}


class LayerHost(ctypes.Structure):
    """si_layer_host_t: host pointers to row-major Q4_0 / fp32 tensors."""
    _fields_ = [(n, _P) for n in ("wq", "wk", "wv", "wo", "norm", "bq", "bk", "bv",
                                  "post_norm", "wgate", "wup", "wdown")]


_SIGS = {
    "si_last_error": (ctypes.c_char_p, []),
    "si_kernel_timing_start": (_I, [ctypes.c_char_p, _I]),
    "si_kernel_timing_stop": (_I, [_P, _I, ctypes.POINTER(_I)]),
    "si_kernel_timing_name": (ctypes.c_char_p, [_I]),
    "si_stream_read": (_I, [_P, ctypes.c_size_t, _P, _I, _I, _P]),
    "si_q8_tile": (_I, [_P, _P, _I, _I, _P, _P, _P]),
    "si_q4_repack": (_I, [_P, _I, _I, _I, _P, _P, _P]),
    "si_q4_unpack": (_I, [_P, _P, _I, _I, _I, _P, _P]),
    "si_q4_tile": (_I, [_I, _I]),
    "si_q4_scale_count": (_Z, [_I, _I, _I]),
    "si_quantize_q8": (_I, [_P, _P, _I, _P]),
    "si_quantize_q8_rows": (_I, [_P, _I, _I, _P, _P, _P, _P]),
    "si_rmsnorm_q8": (_I, [_P, _P, _I, _I, _F, _P, _P, _P, _P, _P]),
    "si_residual_rmsnorm_q8": (_I, [_P, _P, _P, _I, _I, _F, _P, _P, _P, _P, _P, _P]),
    "si_q4q8_block_dots": (_I, [_P, _P, _I, _I, _P, _P, _P, _P]),
    "si_matvec_q4q8": (_I, [_P, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _I, _P]),
    "si_ffn_gateup_q8": (_I, [_P, _P, _I, _F, _P, _P, _I, _I, _P, _P, _P, _P, _I, _P]),
    "si_gemm_q4q8": (_I, [_P, _P, _I, _I, _I, _P, _P, _I, _P, _P, _P, _I, _I, _P, _Z, _P]),
    "si_gemm_workspace": (_Z, [_I, _I, _I]),
    "si_gemm_f6_workspace": (_Z, [_I, _I, _I]),
    "si_gemm_gateup_q8": (_I, [_P, _P, _I, _I, _I, _P, _P, _I, _P, _P, _P, _P, _P, _I, _P, _Z,
                               _P]),
    "si_rope_kv_append": (_I, [ctypes.POINTER(Shape), _P, _I, _I, _I, _I, _I, _P, _P, _P, _P,
                               _P, _P, _Z, _P]),
    "si_rope_table": (_I, [_I, _I, _F, _P, _P]),
    "si_attention": (_I, [ctypes.POINTER(Shape), _P, _I, _P, _P, _Z, _P, _I, _I, _I, _P, _P,
                          _P, _P, _P, _Z, _P]),
    "si_attention_workspace": (_Z, [ctypes.POINTER(Shape), _I, _I]),
    "si_attention_static": (_I, [ctypes.POINTER(Shape), _P, _I, _P, _P, _Z, _P, _I, _I, _I, _P,
                                 _P, _P, _P, _P]),
    "si_attention_standard": (_I, [ctypes.POINTER(Shape), _P, _P, _P, _I, _P, _P, _P]),
    "si_f32_to_f16": (_I, [_P, _P, _Z, _P]),
    "si_f16_to_f32": (_I, [_P, _P, _Z, _P]),
    "si_matvec_q4q8_rowmajor": (_I, [_P, _P, _I, _I, _P, _P, _P]),
    "si_colsoa_matvec": (_I, [_P, _I, _P, _I, _P, _P, _P, _I, _P]),
    "si_rmsnorm": (_I, [_P, _P, _I, _I, _F, _P, _P]),
    "si_rope": (_I, [ctypes.POINTER(Shape), _P, _I, _I, _P, _P, _I, _P]),
    "si_attention_group": (_I, [ctypes.POINTER(Shape), _P, _I, _I, _P, _P, _I, _P, _P, _Z, _P]),
    "si_attention_group_workspace": (_Z, [ctypes.POINTER(Shape), _I, _I]),
    "si_swiglu_q8": (_I, [_P, _I, _I, _P, _P, _P, _P, _P]),
    "si_layer_create": (_I, [ctypes.POINTER(Shape), ctypes.POINTER(LayerHost), _I, _I,
                             ctypes.POINTER(_P)]),
    "si_layer_destroy": (_I, [_P]),
    "si_workspace_create": (_I, [ctypes.POINTER(Shape), _I, _I, ctypes.POINTER(_P)]),
    "si_workspace_destroy": (_I, [_P]),
    "si_layer_create_in": (_I, [_P, ctypes.POINTER(LayerHost), ctypes.POINTER(_P)]),
    "si_layer_decode": (_I, [_P, _P, _P, _P, _I, _P, _I, _P]),
    "si_layer_decode_batch": (_I, [_P, _P, _I, _P, _P, _Z, _P, _I, _I, _P, _I, _P]),
    "si_layer_prefill": (_I, [_P, _P, _I, _I, _P, _P, _P, _I, _P]),
    "si_layer_decode_paged": (_I, [_P, _P, _I, _P, _P, _I, _I, _P, _I, _P, _I, _I, _P, _I, _P]),
    "si_attention_paged": (_I, [ctypes.POINTER(Shape), _P, _I, _P, _P, _I, _I, _P, _I, _P, _I,
                                _P, _P, _P, _P, _P, _Z, _P]),
    "si_layer_buffer": (_P, [_P, _I]),
    "si_layer_set_timing": (_I, [_P, _I]),
    "si_layer_phase_ms": (_I, [_P, _P]),
    "si_layer_weights": (_I, [_P, _I, ctypes.POINTER(_P), ctypes.POINTER(_P),
                              ctypes.POINTER(_I), ctypes.POINTER(_I), ctypes.POINTER(_I)]),
}

_lib = None
_host = None


def lib():
    """The ABI library; raises if it was not built (no fallback exists)."""
    global _lib
    if _lib is None:
        try:  # bind to the HIP runtime torch already carries (same SONAME)
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(AMD_SO):
            raise RuntimeError(f"{AMD_SO} missing: run __graft_entry__.build() "
                               "(make -C simple-inference_amd)")
        L = ctypes.CDLL(AMD_SO)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def host_lib():
    global _host
    if _host is None:
        if not os.path.exists(HOST_SO):
            raise RuntimeError(f"{HOST_SO} missing: run __graft_entry__.build()")
        H = ctypes.CDLL(HOST_SO)
        H.si_quantize_q4_0_host.argtypes = [_P, _P, _I]
        H.si_quantize_q4_0_host.restype = None
        for name, res, args in (
                ("si_kv_pages_create", _P, [_I, _I, _I, _I]),
                ("si_kv_pages_destroy", None, [_P]),
                ("si_kv_seq_add", _I, [_P]),
                ("si_kv_seq_grow", _I, [_P, _I, _I]),
                ("si_kv_seq_free", None, [_P, _I]),
                ("si_kv_seq_len", _I, [_P, _I]),
                ("si_kv_pages_free", _I, [_P]),
                ("si_kv_page_table", ctypes.POINTER(_I), [_P]),
                ("si_stack_create", _P, [ctypes.POINTER(Shape), _P, _I, _I, _I, _I, _I]),
                ("si_stack_destroy", None, [_P]),
                ("si_stack_pages", _P, [_P]),
                ("si_stack_k_pool", _P, [_P, _I]),
                ("si_stack_v_pool", _P, [_P, _I]),
                ("si_stack_layer", _P, [_P, _I]),
                ("si_stack_dev_table", _P, [_P]),
                ("si_stack_dev_ctx", _P, [_P]),
                ("si_stack_nseq", _I, [_P]),
                ("si_stack_prepare", _I, [_P, _P, _I]),
                ("si_stack_decode", None, [_P, _P, _P, _I, _P])):
            f = getattr(H, name)
            f.restype = res
            f.argtypes = args
        _host = H
    return _host


def call(name, *args):
    rc = getattr(lib(), name)(*args)
    if rc != SI_OK:
        raise SiError(rc, lib().si_last_error().decode())
    return rc


def kernel_times_ms(kernel_filter, fn, capacity=4096):
    """Runs fn() with per-dispatch timing on (si_kernel_timing_start) and
    returns [(kernel, ms)] for the launches whose kernel name contains one of
    the '|'-separated alternatives of kernel_filter, in launch order (none
    under stream capture); kernel is the demangled name without namespace
    and parameters, e.g. "k_dec_attn<64, 8, false, false, 1>"."""
    call("si_kernel_timing_start", kernel_filter.encode(), capacity)
    try:
        fn()
    finally:
        ms = np.zeros(capacity, np.float32)
        n = ctypes.c_int(0)
        call("si_kernel_timing_stop", ms.ctypes.data_as(ctypes.c_void_p), capacity,
             ctypes.byref(n))
    names = [lib().si_kernel_timing_name(i).decode() for i in range(n.value)]
    return list(zip(names, ms[:n.value].tolist()))


def ptr(t):
    """Device (torch) or host (numpy) buffer address; None stays NULL."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return ctypes.c_void_p(t.data_ptr())
    return t.ctypes.data_as(ctypes.c_void_p)


def stream_handle(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def quantize_q4_0(w):
    """Product-side ggml Q4_0 quantizer (host C): fp32 [rows][k] -> uint8 rows."""
    w = np.ascontiguousarray(w, np.float32)
    rows = w.shape[0] if w.ndim == 2 else 1
    out = np.empty((rows, w.size // rows // QK * 18), np.uint8)
    host_lib().si_quantize_q4_0_host(ptr(w), ptr(out), w.size)
    return out


def declared_functions():
    """Function names declared in include/*.h (for the export check)."""
    import re
    names = []
    for fn in sorted(os.listdir(INCLUDE_DIR)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE_DIR, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(\w+)\s*\([^;{]*\)\s*;", text, flags=re.M):
            if not m.group(0).lstrip().startswith("typedef"):
                names.append((fn, m.group(1)))
    return names


class Workspace:
    """si_workspace_t owner: activation buffers shared by the layers of a model."""

    def __init__(self, shape, max_tokens, max_pos):
        self.shape, self.max_tokens, self.max_pos = shape, max_tokens, max_pos
        h = _P()
        call("si_workspace_create", ctypes.byref(shape), max_tokens, max_pos, ctypes.byref(h))
        self.h = h

    def close(self):
        if self.h:
            lib().si_workspace_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Layer:
    """si_layer_t owner built from host tensors (dict of numpy arrays), on a
    private workspace or on a shared Workspace."""

    def __init__(self, shape, tensors, max_tokens=None, max_pos=None, workspace=None):
        self.shape = shape
        self._keep = {k: np.ascontiguousarray(v) for k, v in tensors.items() if v is not None}
        host = LayerHost(**{k: v.ctypes.data for k, v in self._keep.items()})
        h = _P()
        if workspace is not None:
            call("si_layer_create_in", workspace.h, ctypes.byref(host), ctypes.byref(h))
            max_tokens, max_pos = workspace.max_tokens, workspace.max_pos
        else:
            call("si_layer_create", ctypes.byref(shape), ctypes.byref(host), max_tokens, max_pos,
                 ctypes.byref(h))
        self.h = h
        self.max_tokens, self.max_pos = max_tokens, max_pos

    def close(self):
        if self.h:
            lib().si_layer_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def buffer(self, name):
        return lib().si_layer_buffer(self.h, BUF[name])

    def weights(self, which):
        """(qs, d, tile, n, k) device pointers and shape of matrix `which`."""
        qs, d, tile, n, k = _P(), _P(), _I(), _I(), _I()
        call("si_layer_weights", self.h, which, ctypes.byref(qs), ctypes.byref(d),
             ctypes.byref(tile), ctypes.byref(n), ctypes.byref(k))
        return qs.value, d.value, tile.value, n.value, k.value

    # The layer calls below keep the intermediates in the layer's buffers
    # (SI_LAYER_CAPTURE) unless capture=False, for the stagewise checks.
    def decode(self, x, kc, vc, context, out, flags=SI_LAYER_FULL, stream=None, capture=True):
        call("si_layer_decode", self.h, ptr(x), ptr(kc), ptr(vc), context, ptr(out),
             flags | (SI_LAYER_CAPTURE if capture else 0), stream_handle(stream))

    def decode_batch(self, x, nseq, kc, vc, kv_seq_stride, context, max_ctx, out,
                     ctx_dev=None, flags=SI_LAYER_FULL, stream=None, capture=True):
        call("si_layer_decode_batch", self.h, ptr(x), nseq, ptr(kc), ptr(vc), kv_seq_stride,
             ptr(ctx_dev), context, max_ctx, ptr(out),
             flags | (SI_LAYER_CAPTURE if capture else 0), stream_handle(stream))

    def decode_paged(self, x, nseq, k_pool, v_pool, npages, page_size, pages, max_pages,
                     ctx_dev, max_ctx, out, flags=SI_LAYER_FULL, stream=None, capture=True):
        call("si_layer_decode_paged", self.h, ptr(x), nseq, ptr(k_pool), ptr(v_pool), npages,
             page_size, ptr(pages), max_pages, ptr(ctx_dev), max_ctx, max_ctx, ptr(out),
             flags | (SI_LAYER_CAPTURE if capture else 0), stream_handle(stream))

    def prefill(self, x, ntok, prefix, kc, vc, out, flags=SI_LAYER_FULL, stream=None,
                capture=True):
        call("si_layer_prefill", self.h, ptr(x), ntok, prefix, ptr(kc), ptr(vc), ptr(out),
             flags | (SI_LAYER_CAPTURE if capture else 0), stream_handle(stream))

    def set_timing(self, on=True):
        call("si_layer_set_timing", self.h, int(on))

    def phase_ms(self):
        ms = np.zeros(len(PHASES), np.float32)
        call("si_layer_phase_ms", self.h, ptr(ms))
        return dict(zip(PHASES, ms.tolist()))
