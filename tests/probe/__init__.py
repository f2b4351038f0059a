"""Loader of the test-only device probe library (tests/probe/libsi_probe.so)."""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PROBE_SO = os.path.join(HERE, "libsi_probe.so")
_P, _I, _Z, _U = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_uint32
_lib = None


def probe():
    global _lib
    if _lib is None:
        import torch  # noqa: F401  (bind to the HIP runtime torch carries)
        if not os.path.exists(PROBE_SO):
            raise RuntimeError(f"{PROBE_SO} missing: run __graft_entry__.build()")
        L = ctypes.CDLL(PROBE_SO)
        for name, args in (("si_probe_lane_ops", [_P, _P]),
                           ("si_probe_mfma_f16", [_P, _P, _P, _P, _P]),
                           ("si_probe_h2f", [_P, _P, _P, _Z, _P]),
                           ("si_probe_f2h_sweep", [_U, _U, _Z, _P, _P])):
            f = getattr(L, name)
            f.restype, f.argtypes = _I, args
        _lib = L
    return _lib


def call(name, *args):
    rc = getattr(probe(), name)(*args)
    assert rc == 0, f"{name} returned {rc}"
