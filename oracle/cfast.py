"""ctypes loader for oracle/law_c.c -- TEST INFRASTRUCTURE (expected
results in tests and the multi-threaded CPU baseline; never a product
fallback)."""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle_w4a8.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        L = ctypes.CDLL(path)
        L.orc_matvec_y32_img.argtypes = [ctypes.c_void_p, ctypes.c_int64,
                                         ctypes.c_int32, ctypes.c_int32,
                                         ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_int32]
        L.orc_matvec_y32_img.restype = ctypes.c_int
        L.orc_dynq8.argtypes = [ctypes.c_void_p, ctypes.c_int32,
                                ctypes.c_void_p, ctypes.c_void_p]
        L.orc_num_threads.restype = ctypes.c_int
        _LIB = L
    return _LIB


def num_threads():
    return int(lib().orc_num_threads())


def matvec_y32_img(img, nrows, K, sh, x8, nthreads=0):
    """img: bytes / uint8 array of a row image."""
    a = np.frombuffer(img, dtype=np.uint8) if isinstance(img, (bytes, bytearray)) \
        else np.ascontiguousarray(img, dtype=np.uint8)
    x = np.ascontiguousarray(x8, dtype=np.int8)
    y = np.empty(nrows, dtype=np.int32)
    rc = lib().orc_matvec_y32_img(a.ctypes.data, nrows, K, sh, x.ctypes.data,
                                  y.ctypes.data, nthreads)
    if rc == -4:
        raise AssertionError("y32 overflow — sh miscomputed")
    if rc:
        raise AssertionError(f"orc_matvec_y32_img rc={rc}")
    return y


def dyn_quant_i8(x16):
    x = np.ascontiguousarray(x16, dtype=np.int16)
    out = np.empty(x.size, dtype=np.int8)
    e = ctypes.c_int32()
    lib().orc_dynq8(x.ctypes.data, x.size, out.ctypes.data, ctypes.byref(e))
    return out, int(e.value)
