"""Build/load helper for the C restatement (test infrastructure only)."""
import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libmxfp4_oracle.so")
SRC = os.path.join(HERE, "mxfp4_oracle.c")


def build(force=False):
    if force or not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(SRC):
        subprocess.run(["make", "-C", HERE, "-B" if force else "all"], check=True,
                       stdout=subprocess.DEVNULL)
    return LIB


_lib = None


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(LIB)
        L.mxo_e8m0_code.argtypes = [ctypes.c_float]
        L.mxo_e8m0_code.restype = ctypes.c_uint8
        L.mxo_e8m0_code_frexp.argtypes = [ctypes.c_float]
        L.mxo_e8m0_code_frexp.restype = ctypes.c_uint8
        L.mxo_e2m1_code.argtypes = [ctypes.c_float]
        L.mxo_e2m1_code.restype = ctypes.c_uint8
        L.mxo_quantize_rows.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                        ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
        L.mxo_quantize_rows.restype = None
        L.mxo_sweep_scale.argtypes = [ctypes.c_uint32, ctypes.c_uint32,
                                      ctypes.POINTER(ctypes.c_uint32)]
        L.mxo_sweep_scale.restype = ctypes.c_int64
        _lib = L
    return _lib


def quantize_rows_c(w, kp=None):
    import numpy as np
    w = np.ascontiguousarray(np.asarray(w, np.float32))
    if w.ndim == 1:
        w = w[None]
    n, k = w.shape
    kp = (k + 31) // 32 * 32 if kp is None else kp
    packed = np.zeros((n, kp // 2), np.uint8)
    scales = np.zeros((n, kp // 32), np.uint8)
    lib().mxo_quantize_rows(w.ctypes.data, n, k, kp, packed.ctypes.data, scales.ctypes.data)
    return packed, scales
