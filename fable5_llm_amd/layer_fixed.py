"""Drop-in for the matvec-path entry points of ref/layer_fixed.py and the
MOVY / ALU / AMAX32 movers, computed on the MI355X engine.

  matvec_fx(qw, x16, out_f)            layer_fixed.py:1201-1221
  matvec_to(qw, x16, in_f, out_f)      layer_fixed.py:1224-1236 (one fused launch)
  rmsnorm_fx(x16, w_q14, in_f, one_plus) layer_fixed.py:1242-1278
  mlp_fx(xn16, qm, rs_f)               layer_fixed.py:1597-1604
  movy(y32, shift, mode)               seq_model.py:1027-1050
  alu_shift32/shift32w/silu32/emul32   gen_layer_script.py:1397-1423
  Amax32 / head_argmax                 gen_layer_script.py:1424-1433,
                                       gen_model_script.py:627-643
  head_topk32 / topk32                 the layer_topk32 block, docs/SEQ_ISA.md B8

A quantised matrix `qw` is the reference's dict {"w4", "m", "e", "sh"} (or
an already-uploaded engine.Weights via qw["dev"]).
"""
import numpy as np

from . import _native as N
from .engine import default_context
from .w4a8_ref import G, pack_ddr_rows

RS_F_9B = 7      # layer_fixed.py:103 (9B operating point)
MOVY_PAIRS32 = N.MOVY_PAIRS32
MOVY_INT16 = N.MOVY_INT16


def clip16(x):
    return np.clip(np.asarray(x, dtype=np.int64), -32768, 32767)


def _weights(qw):
    """Upload (once per dict) the matrix of a quantised dict."""
    w = qw.get("dev") if isinstance(qw, dict) else None
    if w is not None and w.h is not None:
        return w
    g = int(qw.get("g", G))
    assert g == G, "g=64 images are not executable by the 9B engine (g=128 only)"
    w4 = np.asarray(qw["w4"])
    img, _ = pack_ddr_rows(w4, qw["m"])
    w = default_context().upload(img, w4.shape[0], w4.shape[1], int(qw["sh"]))
    qw["dev"] = w
    return w


def shift_for(qw, e_x, in_f, out_f):
    """MOVY shift (gen_layer_script.py:1753-1754)."""
    return (15 - qw["e"] - qw["sh"]) - e_x + in_f - out_f


def matvec_fx(qw, x16, out_f=None):
    """DYNQ8 then matvec: returns (y32, e_x)."""
    w = _weights(qw)
    y, _x8, e_x, _ = default_context().matvec_fused(
        w, np.asarray(x16, dtype=np.int16), prologue=N.PRO_DYNQ8,
        epilogue=N.EPI_Y32)
    return y, e_x


def matvec_to(qw, x16, in_f, out_f):
    """x16 (in_f frac) -> int64 y with out_f frac bits:
    rshift_round(y32, (15-e-sh) - e_x + in_f - out_f), one device launch."""
    w = _weights(qw)
    p0 = (15 - int(qw["e"]) - int(qw["sh"])) + int(in_f) - int(out_f)
    y, _x8, _e, _ = default_context().matvec_fused(
        w, np.asarray(x16, dtype=np.int16), prologue=N.PRO_DYNQ8,
        epilogue=N.EPI_SHIFT_I64, p0=p0)
    return y


def rmsnorm_fx(x16, w_q14, in_f, one_plus):
    x = np.asarray(x16)
    n = x.size
    nbits = n.bit_length() - 1
    assert n > 0 and (1 << nbits) == n, f"rmsnorm_fx: n={n} not a power of 2"
    return default_context().rmsnorm(x, w_q14, in_f, one_plus).astype(np.int64)


def movy(y32, shift, mode):
    return default_context().movy(y32, shift, mode).astype(np.int64)


def alu_shift32(y32, p0):
    return default_context().alu(N.ALU_SHIFT32, y32, p0).astype(np.int64)


def alu_shift32w(y32, p0):
    return default_context().alu(N.ALU_SHIFT32W, y32, p0).astype(np.int64)


def alu_silu32(y32, p0):
    return default_context().alu(N.ALU_SILU32, y32, p0).astype(np.int64)


def alu_emul32(y32, b16, p0):
    return default_context().alu(N.ALU_EMUL32, y32, p0, b=b16).astype(np.int64)


def mlp_fx(xn16, qm, rs_f=RS_F_9B):
    """SwiGLU block (layer_fixed.py:1597-1604): gate -> SILU32 (out_f 12),
    up -> SHIFT32W (out_f rs_f), EMUL32 product at p0 12, DYNQ8 -> down ->
    int16, as one device-resident chain (w4a8_mlp_async: gate and up in one
    launch, then EMUL32, then down).

    layer_fixed.py:1602 multiplies the unclipped int64 up value u; the
    engine keeps it clipped to int32, as SHIFT32W does
    (gen_layer_script.py:2176-2186).  The product is the same either way:
    where |u| >= 2^31 and the SILU32 factor sg is nonzero, |sg * u| and
    |sg * clip32(u)| are both >= 2^31 - 1, so rshift_round by 12 is
    >= 2^19 and clip16 saturates both to the same rail (the sign of
    sg * u); where sg = 0 both are 0.  Left shifts of the y32s (shift =
    p0 - e_x < 0) are therefore matched as long as the reference's own int64
    arithmetic is exact: sg * u needs |u| < 2^48, i.e. a left shift of the
    up projection's y32 (|y32| < 2^31) of at most 17, and the gate and down
    projections' y32 << s needs s <= 32.  Beyond that numpy's int64 wraps
    and the reference has no defined result; with e_x <= 9 (DYNQ8 of int16),
    such p0s are refused with AssertionError."""
    import torch
    ctx = default_context()
    p0s = [(15 - qm[k]["e"] - qm[k]["sh"]) + rs_f - out_f
           for k, out_f in (("gate", 12), ("up", rs_f), ("down", rs_f))]
    for name, p0, most in zip(("gate", "up", "down"), p0s, (32, 17, 32)):
        assert 9 - p0 <= most, (
            f"mlp_fx: the {name} projection's shift p0 - e_x = {p0} - e_x could shift its "
            f"y32 left by more than {most} bits, where layer_fixed.py:1597-1604's int64 "
            f"arithmetic wraps")
    wg, wu, wd = _weights(qm["gate"]), _weights(qm["up"]), _weights(qm["down"])
    dev = torch.device("cuda", ctx.device)
    x = torch.from_numpy(np.ascontiguousarray(xn16, dtype=np.int16)).to(dev)
    y = torch.empty(wd.nrows, dtype=torch.int16, device=dev)
    torch.cuda.synchronize(dev)          # the input copy ran on torch's stream
    ctx.mlp_async(wg, wu, wd, p0s, x, mlp_out=y)
    ctx.sync()
    return y.cpu().numpy().astype(np.int64)


class Amax32:
    """AMAX32 running argmax over int32 chunks, fed on the host the way
    the head loop feeds 2048-row chunks; the fused device path is
    head_argmax()."""

    def __init__(self):
        self.val, self.idx, self.g, self.first = 0, 0, 0, True

    def feed(self, y32, fresh=False):
        if fresh:
            self.g, self.first = 0, True
        y = np.asarray(y32, dtype=np.int64)
        if y.size:
            i = int(np.argmax(y))          # first max inside the chunk
            if self.first or int(y[i]) > self.val:
                self.val, self.idx = int(y[i]), self.g + i
            self.first = False
            self.g += y.size
        return self


def head_argmax(qw, x, prologue=N.PRO_X8, norm_w=None, in_f=0, one_plus=False):
    """LM head in one pass: (argmax row, its int32 y32), lowest index on ties."""
    return default_context().head_argmax(_weights(qw), x, prologue=prologue,
                                         norm_w=norm_w, in_f=in_f, one_plus=one_plus)


def topk32(y32):
    """TOPK-32 of an int32 vector scanned after one fresh (docs/SEQ_ISA.md
    B8): (vals, rows, count, overflow), the block's TK_VAL / TK_IDX entries
    below count and TK_STATUS's count and overflow bit."""
    return default_context().topk32(y32)


def head_topk32(qw, x, prologue=N.PRO_X8, norm_w=None, in_f=0, one_plus=False):
    """The LM head's matvec then TOPK-32 of its raw y32 (the AMAX32 head
    loop feeding the block, gen_model_script.py:627-643)."""
    return default_context().head_topk32(_weights(qw), x, prologue, norm_w, in_f, one_plus)
