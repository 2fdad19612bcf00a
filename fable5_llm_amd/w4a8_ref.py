"""Drop-in for the W4A8 entry points of ref/w4a8_ref.py, computed on the
MI355X engine.

Same names, argument meaning and error behaviour (AssertionError with the
reference's messages):
  rshift_round(v, s)                  w4a8_ref.py:90-99     (HIP kernel)
  row_beats(K, g) / row_stride(K, g)  w4a8_ref.py:102-114   (wire arithmetic)
  group_size_of(w4, m, g)             w4a8_ref.py:143-151
  pack_w4 / unpack_w4                 w4a8_ref.py:331-346   (host wire format)
  pack_ddr_rows / unpack_ddr_rows     w4a8_ref.py:349-370, 429-446
  matvec_y32(w4, m, sh, x8, g=None)   w4a8_ref.py:254-289   (HIP GEMV)

Only the g = 128 wire format is executable (the engine format of the 9B
build, rtl/matvec_engine.sv:17-34); g = 64 images can be packed but a g = 64
matvec raises AssertionError, as the 9B RTL refuses it.
"""
import numpy as np

from .engine import default_context

G = 128
G_WIRE = (128, 64)
K_PER_WBEAT = 128
SCALES_PER_BEAT = 32


def rshift_round(v, s):
    """Round-half-away-from-zero shift of an int64 array (negative s =
    exact left shift), on the device."""
    scalar = np.ndim(v) == 0
    out = default_context().rshift_round(np.asarray(v, dtype=np.int64), int(s))
    return out.reshape(()) if scalar else out


def row_beats(K, g=G):
    assert g in G_WIRE, f"group size {g} has no defined wire format"
    assert K % K_PER_WBEAT == 0, f"K={K} must be a multiple of {K_PER_WBEAT}"
    return K // K_PER_WBEAT, (K // g + SCALES_PER_BEAT - 1) // SCALES_PER_BEAT


def row_stride(K, g=G):
    wb, sb = row_beats(K, g)
    return (wb + sb) * 64


def group_size_of(w4, m, g=None):
    K = np.shape(w4)[1]
    ng = np.shape(m)[1]
    assert ng > 0 and K % ng == 0, f"m has {ng} groups, incompatible with K={K}"
    gi = K // ng
    if g is not None:
        assert int(g) == gi, f"declared g={g} but w4/m imply {gi}"
    return gi


def pack_w4(w4):
    """(N,K) int4 values -> (N, K//2) uint8, low nibble = even k."""
    u = (np.asarray(w4).astype(np.int16) & 0xF).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def unpack_w4(packed, K):
    p = np.asarray(packed, dtype=np.uint8)
    lo = (p & 0xF).astype(np.int8)
    hi = (p >> 4).astype(np.int8)
    out = np.empty((p.shape[0], K), dtype=np.int8)
    out[:, 0::2] = np.where(lo > 7, lo - 16, lo)
    out[:, 1::2] = np.where(hi > 7, hi - 16, hi)
    return out


def pack_ddr_rows(w4, m, g=None):
    """Row image [weight beats | uint16-LE scales | zero tail], rows back to
    back.  Returns (image_bytes, row_stride)."""
    w4 = np.asarray(w4)
    N, K = w4.shape
    g = group_size_of(w4, m, g)
    wb, sb = row_beats(K, g)
    stride = (wb + sb) * 64
    img = np.zeros((N, stride), dtype=np.uint8)
    img[:, :K // 2] = pack_w4(w4)
    mb = np.asarray(m).astype('<u2').view(np.uint8).reshape(N, -1)
    assert mb.shape[1] <= sb * 64, "scale bytes overflow the scale beats"
    img[:, K // 2:K // 2 + mb.shape[1]] = mb
    return img.tobytes(), stride


def unpack_ddr_rows(img, nrows, K, g=G):
    wb, sb = row_beats(K, g)
    stride = (wb + sb) * 64
    a = np.frombuffer(img, dtype=np.uint8)
    assert a.size == nrows * stride, \
        f"image is {a.size}B, expected {nrows}*{stride}={nrows * stride}"
    a = a.reshape(nrows, stride)
    w4 = unpack_w4(a[:, :wb * 64], K)
    ng = K // g
    m = a[:, wb * 64:wb * 64 + 2 * ng].copy().view('<u2').reshape(nrows, ng)
    return w4, m


def sh_for_k(K, g=G):
    """The final shift quantize_weights picks (w4a8_ref.py:177-179)."""
    bound = (K // g) * 65535 * (g * 8 * 127)
    return max(0, bound.bit_length() - 31)


def matvec_y32(w4, m, sh, x8, g=None):
    """int32 y = rshift_round(sum_g m[g] * sum_k w4*x8, sh) per row, on the
    MI355X engine (AssertionError on the reference's overflow conditions)."""
    w4 = np.asarray(w4)
    N, K = w4.shape
    g = group_size_of(w4, m, g)
    assert g == G, "g=64 images are not executable by the 9B engine (g=128 only)"
    x8 = np.asarray(x8)
    assert x8.shape == (K,), f"x8 has shape {x8.shape}, expected ({K},)"
    img, _ = pack_ddr_rows(w4, m, g)
    ctx = default_context()
    w = ctx.upload(img, N, K, int(sh))
    try:
        return ctx.matvec_y32(w, x8.astype(np.int8))
    finally:
        w.free()
