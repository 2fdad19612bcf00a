"""Drop-in for the matvec-path entry points of ref/fixedpoint.py, computed
on the MI355X engine.

  dyn_quant_i8(x16) -> (x8, e)   fixedpoint.py:24-33 (HIP; n <= 12288)
  rsqrt_lut() / sigmoid_table()  the device's tables, read back from the
                                 engine (fixedpoint.py:42-53, 128-142)
"""
import numpy as np

from .engine import default_context


def dyn_quant_i8(x16):
    """int16 vector -> (int8 vector, right shift e >= 0): the least e with
    max|rshift_round(x, e)| <= 127, values clipped to +-127."""
    x = np.asarray(x16)
    assert x.ndim == 1 and x.size >= 1, "dyn_quant_i8 takes a non-empty vector"
    assert x.size <= 12288, "DYNQ8 vector longer than the engine's 12288 limit"
    return default_context().dynq8(x.astype(np.int16))


def rsqrt_lut():
    return default_context().tables()[0].astype(np.int64)


def sigmoid_table():
    return default_context().tables()[1].astype(np.int64)
