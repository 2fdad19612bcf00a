"""numpy restatement of the reference's W4A8 integer law -- TEST INFRASTRUCTURE.

Used only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
Every function cites the reference file:line it restates (paths relative to
the coreyhahn/fable5_llm checkout).  All arithmetic is exact integer
arithmetic in int64 (or Python int where a product could exceed 63 bits).

How each function is pinned (the checks live in tests/test_oracle_*.py):

  rshift_round      KATs (w4a8_ref.py:471-472), brute force against exact
                    rational rounding, tb/vectors/s*/alu_shift32* files
  row_beats/stride  contract table w4a8_ref.py:549-556, engine table
                    matvec_engine.sv:252-258, tb/vec_s*/params.txt, manifests
  sh_for_k          manifests (K 1024/2048/3584 -> 5/6/7), closed form
  pack/unpack       tb/vec_s*/beats.hex byte images and the committed
                    tb/scripts/*_w*.bin images (row subsets); at K = 4096 /
                    8192 / 12288 (2-3 scale beats) the bytes the reference's
                    pack_ddr_rows wrote (tests/golden/q9_vectors.npz)
  matvec_y32        tb/vec_s1..s4 golden y32; every V record of
                    tb/scripts/{layer,token}_s*.txt (row subsets); y32 the
                    reference's matvec_y32 wrote at K = 4096 / 8192 / 12288;
                    brute force with Python ints; dequantised-float bound
  dyn_quant_i8      tb/vectors/s*/alu_dynq8_{x,y,e}; R+E records before each
                    V record; brute-force exponent search
  rsqrt_lut/rsqrt_q roms/rsqrt_rom.hex; tb/rsqrt_cases_s*.txt (2000 cases)
  rmsnorm_fx        tb/vectors/s*/rmsnorm_{x16,w14,y16}
  sigmoid_table,
  silu_q            roms/sigmoid_rom.hex; tb/silu_cases_s*.txt;
                    alu_silu32_y
  alu_emul32        alu_emul32_y
  alu_shift32w      alu_shift32w_y (left-shift path)
  movy              closed form == alu_shift32/shift32w on the fixture
                    values; RTL caps checked on the boundary shifts
  amax32            A records of tb/scripts/token_s*.txt against the V
                    record of the head; planted ties (== numpy argmax)
  matvec_to         closed form over pinned parts; the shift identity of
                    a V record: C-record ALU p0 == shift_for (layer_s1)
  mlp_fx            composition of pinned parts; the SwiGLU chain between
                    the matvecs by the scripts' gate / up V records and the
                    down record's R + E records (first MLP block of each)
  Topk32 / topk32   no committed fixture (the generator's cases are written
                    to a gitignored directory): entry 0 == amax32 (A
                    records); the list == the first 32 of (value desc,
                    index asc) by numpy lexsort; the overflow bit == its
                    prefix-count form (an element i >= 32 with fewer than
                    32 earlier elements above it and at least 32 at or
                    above it) by brute force; the generator's named cases
                    (rails, tie storms, tie at entry 31, displaced tie)
"""
import numpy as np

I64 = np.int64
G = 128                 # group size of the 9B engine (quant_spec.md:15-16)
SCALES_PER_BEAT = 32    # w4a8_ref.py:85
INT32_MAX = (1 << 31) - 1


# ---------------------------------------------------------------------------
# a1: rounding shift
# ---------------------------------------------------------------------------
def rshift_round(v, s):
    """Round-half-away-from-zero right shift; s < 0 is an exact left shift.

    Restates ref/w4a8_ref.py:90-99 (and rtl/fx_pkg.sv:9-20): the magnitude is
    rounded and the sign re-applied, so -5 >> 1 rounds to -3, not -2.
    """
    v = np.asarray(v, dtype=I64)
    s = int(s)
    if s == 0:
        return v.copy()
    if s < 0:
        return v << I64(-s)
    half = I64(1) << I64(s - 1)
    pos = (v + half) >> I64(s)
    neg = -((-v + half) >> I64(s))
    return np.where(v >= 0, pos, neg)


def rs_s(v, p):
    """seq_model.rs_s / gen_layer_script.rs_s (seq_model.py:89-92,
    gen_layer_script.py:498-501): rshift_round for p >= 0, exact left shift
    for p < 0."""
    return rshift_round(v, p)


def clip16(x):
    """layer_fixed.clip16 / seq_model.clip16 (seq_model.py:85-86)."""
    return np.clip(np.asarray(x, dtype=I64), -32768, 32767)


def clip32(x):
    return np.clip(np.asarray(x, dtype=I64), -(1 << 31), (1 << 31) - 1)


# ---------------------------------------------------------------------------
# a2/a6: wire arithmetic and the final shift
# ---------------------------------------------------------------------------
def row_beats(K, g=G):
    """(weight beats, scale beats) of one row: ref/w4a8_ref.py:102-108."""
    assert g in (128, 64), f"group size {g} has no defined wire format"
    assert K % 128 == 0, f"K={K} must be a multiple of 128"
    return K // 128, (K // g + SCALES_PER_BEAT - 1) // SCALES_PER_BEAT


def row_stride(K, g=G):
    """Bytes per wire row: ref/w4a8_ref.py:111-114."""
    wb, sb = row_beats(K, g)
    return (wb + sb) * 64


def sh_for_k(K, g=G):
    """Final shift of quantize_weights: ref/w4a8_ref.py:177-179
    (the worst-case |p| bound NG*65535*(g*8*127) brought under 2^31)."""
    ng = K // g
    bound = ng * 65535 * (g * 8 * 127)
    return max(0, bound.bit_length() - 31)


# ---------------------------------------------------------------------------
# a3/a4: nibble packing and the row image
# ---------------------------------------------------------------------------
def pack_w4(w4):
    """(N,K) int4 values -> (N,K/2) bytes, even k in the low nibble.
    ref/w4a8_ref.py:331-334."""
    u = (np.asarray(w4).astype(np.int16) & 0xF).astype(np.uint8)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def unpack_w4(packed, K):
    """Inverse of pack_w4 (ref/w4a8_ref.py:337-346): sign-extend nibbles."""
    p = np.asarray(packed, dtype=np.uint8)
    lo = (p & 0xF).astype(np.int8)
    hi = (p >> 4).astype(np.int8)
    lo = np.where(lo > 7, lo - 16, lo).astype(np.int8)
    hi = np.where(hi > 7, hi - 16, hi).astype(np.int8)
    out = np.empty((p.shape[0], K), dtype=np.int8)
    out[:, 0::2] = lo
    out[:, 1::2] = hi
    return out


def pack_ddr_rows(w4, m):
    """Row image [weight beats | uint16-LE scales | zero tail] per row,
    rows back to back (ref/w4a8_ref.py:349-370).  Returns (bytes, stride)."""
    w4 = np.asarray(w4)
    m = np.asarray(m)
    N, K = w4.shape
    assert m.shape == (N, K // G), f"m shape {m.shape} != {(N, K // G)}"
    stride = row_stride(K)
    img = np.zeros((N, stride), dtype=np.uint8)
    img[:, :K // 2] = pack_w4(w4)
    img[:, K // 2:K // 2 + 2 * (K // G)] = (
        m.astype('<u2').view(np.uint8).reshape(N, -1))
    return img.tobytes(), stride


def unpack_ddr_rows(img, nrows, K):
    """The engine's view of a row image (ref/w4a8_ref.py:429-446):
    returns (w4 (N,K) int8, m (N,NG) uint16)."""
    stride = row_stride(K)
    a = np.frombuffer(img, dtype=np.uint8)
    assert a.size == nrows * stride, \
        f"image is {a.size}B, expected {nrows}*{stride}={nrows * stride}"
    a = a.reshape(nrows, stride)
    w4 = unpack_w4(a[:, :K // 2], K)
    ng = K // G
    m = a[:, K // 2:K // 2 + 2 * ng].copy().view('<u2').reshape(nrows, ng)
    return w4, m


# ---------------------------------------------------------------------------
# a5: the matvec law
# ---------------------------------------------------------------------------
def matvec_y32(w4, m, sh, x8, rowchunk=8192):
    """acc[r,g] = sum_k w4*x8 over each 128-group; p = sum_g m*acc (int64);
    y = rshift_round(p, sh); |acc|, |y| < 2^31 asserted.
    Restates ref/w4a8_ref.py:254-289 (g = 128); rows are evaluated in blocks
    of `rowchunk`, which is exact because the law is row-separable
    (gen_layer_script.py:1513-1515 does the same for the LM head)."""
    w4 = np.asarray(w4)
    m = np.asarray(m)
    x8 = np.asarray(x8)
    N, K = w4.shape
    assert K % G == 0 and m.shape == (N, K // G), "shape"
    ng = K // G
    xg = x8.astype(I64).reshape(1, ng, G)
    out = np.empty(N, dtype=np.int32)
    for r0 in range(0, N, rowchunk):
        r1 = min(N, r0 + rowchunk)
        acc = (w4[r0:r1].reshape(r1 - r0, ng, G).astype(I64) * xg).sum(axis=2)
        assert np.abs(acc).max(initial=0) < (1 << 31)
        p = (m[r0:r1].astype(I64) * acc).sum(axis=1)
        y = rshift_round(p, sh)
        assert np.abs(y).max(initial=0) < (1 << 31), \
            "y32 overflow — sh miscomputed"
        out[r0:r1] = y.astype(np.int32)
    return out


def matvec_y32_image(img, nrows, K, sh, x8, rowchunk=8192):
    """matvec_y32 read straight from a row image, block by block (the
    seq_model.DDRWeights.matvec view, seq_model.py:431-452)."""
    stride = row_stride(K)
    a = np.frombuffer(img, dtype=np.uint8).reshape(nrows, stride)
    out = np.empty(nrows, dtype=np.int32)
    for r0 in range(0, nrows, rowchunk):
        r1 = min(nrows, r0 + rowchunk)
        w4, m = unpack_ddr_rows(a[r0:r1].tobytes(), r1 - r0, K)
        out[r0:r1] = matvec_y32(w4, m, sh, x8, rowchunk=rowchunk)
    return out


# ---------------------------------------------------------------------------
# a8: DYNQ8
# ---------------------------------------------------------------------------
def dyn_quant_i8(x16):
    """Least e >= 0 with round(max|x| / 2^e) <= 127 (half away from zero),
    then x8 = clip(rshift_round(x, e), -127, 127).  Restates
    ref/fixedpoint.py:24-33 (RTL: vec_alu.sv op 0, clamp at +-127)."""
    x = np.asarray(x16, dtype=I64)
    mx = int(np.abs(x).max()) if x.size else 0
    e = 0
    while (mx + ((1 << e) >> 1)) >> e > 127:
        e += 1
    q = rshift_round(x, e) if e else x
    return np.clip(q, -127, 127).astype(np.int8), e


# ---------------------------------------------------------------------------
# a9: RMSNorm (rsqrt LUT + 2 Newton steps)
# ---------------------------------------------------------------------------
_RSQRT_LUT = None


def rsqrt_lut():
    """512 Q1.15 seeds of 1/sqrt(m): 256 midpoints over [1,2) then 256 over
    [2,4) (ref/fixedpoint.py:42-53); pinned by roms/rsqrt_rom.hex."""
    global _RSQRT_LUT
    if _RSQRT_LUT is None:
        mid = np.concatenate([1.0 + (np.arange(256) + 0.5) / 256.0,
                              2.0 + (np.arange(256) + 0.5) / 128.0])
        _RSQRT_LUT = np.round(32768.0 / np.sqrt(mid)).astype(I64)
    return _RSQRT_LUT


def rsqrt_q(v, P):
    """(r, e) with 1/sqrt(v * 2^-P) ~= r * 2^(e-30).  Restates
    ref/fixedpoint.py:56-75: normalise v to m in [2^30, 2^32) with an even
    exponent, seed from the LUT by bit slice, two Newton steps in Q30."""
    v = int(v)
    assert v > 0
    s = v.bit_length() - 32
    if (s - P) & 1:
        s += 1
    m = (v >> s) if s >= 0 else (v << -s)
    E = s - P + 30
    if m < (1 << 31):
        idx = (m >> 22) & 0xFF
    else:
        idx = 256 | ((m >> 23) & 0xFF)
    r = int(rsqrt_lut()[idx]) << 15
    for _ in range(2):
        r2 = (r * r) >> 30
        mr2 = (m * r2) >> 30
        r = (r * ((3 << 30) - mr2)) >> 31
    return r, -E // 2


def rmsnorm_fx(x16, w_q14, in_f, one_plus):
    """Integer RMSNorm, ref/layer_fixed.py:1242-1278 (vecnorm modes 0/1):
    ss = sum x^2 (0 -> 1); (r, e) = rsqrt_q(ss, 2*in_f + log2 n);
    y = clip(rshift_round(x*r, 30-e), -2^32, 2^32-1);
    out = clip16(rshift_round(y * (w + one_plus*2^14), 14)).  n must be a
    power of two (layer_fixed.py:1270-1272)."""
    x = np.asarray(x16, dtype=I64)
    n = x.size
    nbits = n.bit_length() - 1
    assert n > 0 and (1 << nbits) == n, f"rmsnorm_fx: n={n} not a power of 2"
    ss = int((x * x).sum())
    if ss == 0:
        ss = 1
    r, e = rsqrt_q(ss, 2 * in_f + nbits)
    y = rshift_round(x * I64(r), 30 - e)
    y = np.clip(y, -(1 << 32), (1 << 32) - 1)
    w = np.asarray(w_q14, dtype=I64)
    scale = w + (1 << 14) if one_plus else w
    return clip16(rshift_round(y * scale, 14))


# ---------------------------------------------------------------------------
# a11: sigmoid / silu PWL and the FFN ALU ops
# ---------------------------------------------------------------------------
_SIG = None


def sigmoid_table():
    """257 Q15 knots of sigmoid over [-16, 16] in steps of 1/8, saturated at
    32767 (ref/fixedpoint.py:128-142); pinned by roms/sigmoid_rom.hex."""
    global _SIG
    if _SIG is None:
        xs = -16.0 + 32.0 * np.arange(257) / 256.0
        _SIG = np.minimum(np.round(32768.0 / (1.0 + np.exp(-xs))),
                          32767).astype(I64)
    return _SIG


def sigmoid_q(x_q12):
    """PWL sigmoid, Q12 in -> Q15 out (ref/fixedpoint.py:135-147)."""
    t = sigmoid_table()
    x = min(max(int(x_q12), -16 << 12), (16 << 12) - 1)
    u = x + (16 << 12)
    i, lo = u >> 9, u & 0x1FF
    a, b = int(t[i]), int(t[i + 1])
    return a + (((b - a) * lo + 256) >> 9)


def silu_q(x_q12):
    """x * sigmoid(x), Q12 in/out (ref/fixedpoint.py:168-171)."""
    return int(rshift_round(I64(int(x_q12) * sigmoid_q(x_q12)), 15))


def alu_shift32(y32, p0):
    """ALU op 1 SHIFT32: clip16(rs_s(y, p0)) (gen_layer_script.py:1399-1400)."""
    return clip16(rs_s(y32, p0))


def alu_shift32w(y32, p0):
    """ALU op 9 SHIFT32W: clip32(rs_s(y, p0)) (gen_layer_script.py:1418-1421)."""
    return clip32(rs_s(y32, p0))


def alu_silu32(y32, p0):
    """ALU op 6 SILU32: clip16(silu_q(clip(rs_s(y, p0), +-2^20)))
    (gen_layer_script.py:1409-1413)."""
    x = np.clip(rs_s(y32, p0), -(1 << 20), (1 << 20) - 1)
    return clip16(np.array([silu_q(int(v)) for v in x], dtype=I64))


def alu_emul32(y32, b16, p0):
    """ALU op 8 EMUL32: clip16(rshift_round(y * b, p0))
    (gen_layer_script.py:1416-1417)."""
    return clip16(rshift_round(np.asarray(y32, dtype=I64)
                               * np.asarray(b16, dtype=I64), p0))


# ---------------------------------------------------------------------------
# a10: MOVY epilogue
# ---------------------------------------------------------------------------
MOVY_PAIRS32 = 0
MOVY_INT16 = 1


def movy(y32, shift, mode):
    """MOVY dequant: v = rs_s(y, shift) then clip16 (int16 mode) or clip32
    (pairs mode).  seq_model.py:1027-1050 with the RTL's shift caps
    (right by at most 63, left by at most 40: seq_movers.sv:770-777), which
    agree with rs_s for every shift in [-40, 63]."""
    y = np.asarray(y32, dtype=I64)
    shift = int(shift)
    if shift >= 0:
        mm = min(shift, 63)
        half = I64(0) if mm == 0 else (I64(1) << I64(mm - 1))
        mag = np.where(y < 0, -y, y)
        r = (mag + half) >> I64(mm)
        v = np.where(y < 0, -r, r)
    else:
        v = y << I64(min(-shift, 40))
    return clip16(v) if mode == MOVY_INT16 else clip32(v)


def shift_for(e, sh, e_x, in_f, out_f):
    """MOVY shift of a matvec result: (15 - e - sh) - e_x + in_f - out_f
    (gen_layer_script.py:1753-1754; layer_fixed.py:1233)."""
    return (15 - e - sh) - e_x + in_f - out_f


# ---------------------------------------------------------------------------
# a12: AMAX32 running argmax
# ---------------------------------------------------------------------------
class Amax32:
    """ALU op 10 state machine (gen_layer_script.py:1424-1433): a value
    replaces the running maximum only if strictly greater, so the lowest
    index wins ties; `fresh` restarts the scan and the global index."""

    def __init__(self):
        self.val, self.idx, self.g, self.first = 0, 0, 0, True

    def feed(self, y32, fresh=False):
        if fresh:
            self.g, self.first = 0, True
        for v in np.asarray(y32, dtype=I64):
            if self.first or int(v) > self.val:
                self.val, self.idx = int(v), self.g
            self.first = False
            self.g += 1
        return self


def amax32(y32, chunk=2048):
    """Whole-vector AMAX32 fed in 2048-row chunks as the head loop does
    (gen_model_script.py:633-638).  Returns (idx, val)."""
    st = Amax32()
    y = np.asarray(y32)
    for c in range(0, y.size, chunk):
        st.feed(y[c:c + chunk], fresh=(c == 0))
    return st.idx, st.val


IDX_BITS = 18          # am_g, the AMAX32 / TOPK element counter (vec_alu.sv)


class Topk32:
    """TOPK-32 running list (docs/SEQ_ISA.md B8; the model of
    tb/scripts/gen_topk_cases.py:60-104): 32 entries sorted by value
    descending, stable after equals (ties keep arrival order = the lower
    index); once full, an arrival not greater than entry[31] is rejected,
    and a rejection that equals entry[31] sets the sticky overflow bit
    (`ovf_lit`, the bit the hardware exports).  `ovf_disp` also sets when an
    insertion displaces an element equal to the new entry[31].  The element
    index is the 18-bit AMAX32 counter; `fresh` clears everything."""

    def __init__(self):
        self.fresh()

    def fresh(self):
        self.g = 0
        self.lst = []          # [(val, idx)]
        self.ovf_lit = False
        self.ovf_disp = False

    def feed(self, y32, fresh=False):
        if fresh:
            self.fresh()
        mask = (1 << IDX_BITS) - 1
        for v in np.asarray(y32, dtype=I64).tolist():
            idx = self.g & mask
            self.g += 1
            lst = self.lst
            if len(lst) < 32:
                pos = 0
                while pos < len(lst) and lst[pos][0] >= v:
                    pos += 1
                lst.insert(pos, (v, idx))
                continue
            last = lst[31][0]
            if v > last:
                pos = 0
                while pos < 32 and lst[pos][0] >= v:
                    pos += 1
                lst.insert(pos, (v, idx))
                dropped = lst.pop()
                if dropped[0] == lst[31][0]:
                    self.ovf_disp = True
            elif v == last:
                self.ovf_lit = True
                self.ovf_disp = True
        return self

    @property
    def count(self):
        return len(self.lst)


def topk32(y32, chunk=2048):
    """TOPK-32 over a whole head fed in 2048-row chunks after one fresh
    (the list accumulates across chained AMAX32 chunks, SEQ_ISA.md B8).
    Returns (vals, idx, count, overflow) with vals / idx int64[count]."""
    st = Topk32()
    y = np.asarray(y32)
    for c in range(0, y.size, chunk):
        st.feed(y[c:c + chunk], fresh=(c == 0))
    vals = np.array([v for v, _ in st.lst], dtype=I64)
    idx = np.array([i for _, i in st.lst], dtype=I64)
    return vals, idx, st.count, st.ovf_lit


# ---------------------------------------------------------------------------
# composites
# ---------------------------------------------------------------------------
def matvec_to(w4, m, e, sh, x16, in_f, out_f):
    """DYNQ8 -> matvec_y32 -> shift to out_f, int64 result, no clip.
    ref/layer_fixed.py:1201-1236."""
    x8, e_x = dyn_quant_i8(x16)
    y32 = matvec_y32(w4, m, sh, x8)
    s = shift_for(e, sh, e_x, in_f, out_f)
    if s >= 0:
        return rshift_round(y32.astype(I64), s)
    return y32.astype(I64) << I64(-s)


def mlp_fx(xn16, gate, up, down, rs_f=7):
    """SwiGLU block, ref/layer_fixed.py:1597-1604.  gate/up/down are
    (w4, m, e, sh) tuples."""
    g = matvec_to(*gate, xn16, rs_f, 12)
    u = matvec_to(*up, xn16, rs_f, rs_f)
    sg = clip16(np.array([silu_q(int(np.clip(v, -(1 << 20), (1 << 20) - 1)))
                          for v in g], dtype=I64))
    prod = clip16(rshift_round(sg * u, 12))
    return clip16(matvec_to(*down, prod, rs_f, rs_f))
