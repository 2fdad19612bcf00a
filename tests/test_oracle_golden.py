"""Pin the CPU oracle (oracle/law.py) against the reference's own golden
vectors, known-answer tests and brute force.  No GPU needed."""
from fractions import Fraction

import numpy as np
import pytest

from oracle import law
from oracle.fixtures import script_argmax, script_records, script_tags, vec_case


# --------------------------------------------------------------- a1 rounding
def test_rshift_round_kats():
    # ref/w4a8_ref.py:471-472
    assert law.rshift_round(5, 1) == 3 and law.rshift_round(-5, 1) == -3
    assert law.rshift_round(4, 2) == 1 and law.rshift_round(-4, 2) == -1
    assert law.rshift_round(7, -3) == 56 and law.rshift_round(-7, -3) == -56
    assert law.rshift_round(-9, 0) == -9


def _round_half_away(fr):
    q = abs(fr)
    n = int(q)
    if q - n >= Fraction(1, 2):
        n += 1
    return n if fr >= 0 else -n


def test_rshift_round_brute_force():
    rng = np.random.default_rng(11)
    v = np.concatenate([rng.integers(-(1 << 40), 1 << 40, 3000),
                        np.arange(-70, 71)])
    for s in range(0, 34):
        got = law.rshift_round(v, s)
        want = [_round_half_away(Fraction(int(x), 1 << s)) for x in v[::37]]
        assert list(got[::37]) == want, s


def test_shift32_vectors(vectors):
    # gen_layer_vectors.py:183-184, 197-198: rshr 5 + clip16; left 8 + clip32
    for s in range(1, 5):
        v = vectors[f"s{s}_alu_shift32_v"]
        assert np.array_equal(law.alu_shift32(v, 5), vectors[f"s{s}_alu_shift32_y"])
        assert np.array_equal(law.alu_shift32w(v, -8), vectors[f"s{s}_alu_shift32w_y"])
        # the MOVY epilogue is the same law in int16 / pairs32 mode
        assert np.array_equal(law.movy(v, 5, law.MOVY_INT16),
                              vectors[f"s{s}_alu_shift32_y"])
        assert np.array_equal(law.movy(v, -8, law.MOVY_PAIRS32),
                              vectors[f"s{s}_alu_shift32w_y"])


def test_movy_rtl_caps():
    # seq_movers.sv:770-777: right shifts cap at 63, left shifts at 40
    y = np.array([-(2**31) + 1, -3, -1, 0, 1, 3, 2**31 - 1], dtype=np.int64)
    assert np.array_equal(law.movy(y, 63, law.MOVY_PAIRS32), np.zeros(7))
    assert np.array_equal(law.movy(y, 200, law.MOVY_PAIRS32), np.zeros(7))
    assert np.array_equal(law.movy(y, -40, law.MOVY_INT16),
                          law.movy(y, -55, law.MOVY_INT16))
    assert np.array_equal(law.movy(y, -2, law.MOVY_PAIRS32),
                          np.clip(y * 4, -(2**31), 2**31 - 1))


# ---------------------------------------------------- a2/a6 wire arithmetic
def test_row_beats_contract(vectors):
    # w4a8_ref.py:549-556 and matvec_engine.sv:252-258
    want = {1024: (8, 1), 2048: (16, 1), 3584: (28, 1), 4096: (32, 1),
            8192: (64, 2), 12288: (96, 3)}
    for K, wb in want.items():
        assert law.row_beats(K) == wb
    assert law.row_stride(4096) == 2112 and law.row_stride(12288) == 6336
    for s in range(1, 5):
        c = vec_case(vectors, s)
        assert c["BPR"] == sum(law.row_beats(c["K"]))
        assert c["NG"] == c["K"] // 128
        assert c["SH"] == law.sh_for_k(c["K"])
    with pytest.raises(AssertionError):
        law.row_beats(1000)


def test_sh_rule():
    assert [law.sh_for_k(k) for k in (1024, 2048, 3584, 4096, 12288)] == \
        [5, 6, 7, 7, 9]


def test_manifest_sh_and_stride(scripts):
    for tag in script_tags():
        for rec in script_records(scripts, tag):
            assert rec["sh"] == law.sh_for_k(rec["K"])
            assert rec["NG"] == rec["K"] // 128


# ------------------------------------------------------- a3/a4 wire format
def test_pack_roundtrip_vec_images(vectors):
    for s in range(1, 5):
        c = vec_case(vectors, s)
        w4, m = law.unpack_ddr_rows(c["img"], c["N"], c["K"])
        assert w4.min() >= -8 and w4.max() <= 7
        img, stride = law.pack_ddr_rows(w4, m)
        assert stride == c["BPR"] * 64
        assert img == c["img"]        # identical bytes, zero tail included


def test_pack_roundtrip_script_images(scripts):
    seen = set()
    for tag in script_tags():
        for rec in script_records(scripts, tag):
            key = (tag, rec["wid"])
            if key in seen:
                continue
            seen.add(key)
            n = rec["rows"].size
            w4, m = law.unpack_ddr_rows(rec["img"], n, rec["K"])
            assert law.pack_ddr_rows(w4, m)[0] == rec["img"]


def test_q9_images_and_y32(q9):
    """The 9B row geometry (2 and 3 scale beats per row): the reference's
    own pack_ddr_rows bytes and matvec_y32 outputs, incl. all-(-8) x all-(-128)
    products at full-range mantissas."""
    from tests.conftest import q9_cases
    n = 0
    for c in q9_cases(q9):
        assert c["sh"] == law.sh_for_k(c["K"])
        assert c["stride"] == law.row_stride(c["K"])
        img, stride = law.pack_ddr_rows(c["w4"], c["m"])
        assert stride == c["stride"] and img == c["img"], c["tag"]
        w4, m = law.unpack_ddr_rows(c["img"], c["N"], c["K"])
        assert np.array_equal(w4, c["w4"]) and np.array_equal(m, c["m"])
        y = law.matvec_y32(c["w4"], c["m"], c["sh"], c["x8"])
        assert np.array_equal(y, c["y32"]), c["tag"]
        ext = np.full(c["K"], -128, dtype=np.int8)
        y = law.matvec_y32_image(c["img"], c["N"], c["K"], c["sh"], ext)
        assert np.array_equal(y, c["y32_ext"]), c["tag"]
        n += 1
    assert n == 9


def test_pack_w4_nibble_order():
    # low nibble = even k (w4a8_ref.py:331-334)
    w = np.array([[1, -2, 7, -8]], dtype=np.int8)
    assert list(law.pack_w4(w)[0]) == [0xE1, 0x87]


# ------------------------------------------------------------- a5 matvec
def test_matvec_vec_goldens(vectors):
    for s in range(1, 5):
        c = vec_case(vectors, s)
        y = law.matvec_y32_image(c["img"], c["N"], c["K"], c["SH"], c["x8"])
        assert np.array_equal(y, c["y32"]), s


def test_matvec_script_v_records(scripts):
    n = 0
    for tag in script_tags():
        for rec in script_records(scripts, tag):
            y = law.matvec_y32_image(rec["img"], rec["rows"].size, rec["K"],
                                     rec["sh"], rec["x8"])
            assert np.array_equal(y, rec["y32"]), (tag, rec["v"])
            n += 1
    assert n == 4 * 45 + 4 * 48


def test_matvec_brute_force_python_ints():
    rng = np.random.default_rng(5)
    for N, K in [(3, 128), (5, 256), (2, 1024)]:
        w4 = rng.integers(-8, 8, (N, K)).astype(np.int8)
        m = rng.integers(0, 65536, (N, K // 128)).astype(np.uint16)
        x8 = rng.integers(-128, 128, K).astype(np.int8)
        x8[:3] = -128
        sh = law.sh_for_k(K)
        y = law.matvec_y32(w4, m, sh, x8)
        for r in range(N):
            p = 0
            for g in range(K // 128):
                acc = sum(int(w4[r, k]) * int(x8[k])
                          for k in range(128 * g, 128 * g + 128))
                p += int(m[r, g]) * acc
            q = abs(p)
            q = (q + (1 << (sh - 1))) >> sh
            assert int(y[r]) == (q if p >= 0 else -q)


def test_matvec_overflow_asserts():
    w4 = np.full((1, 128), -8, dtype=np.int8)
    m = np.full((1, 1), 65535, dtype=np.uint16)
    x8 = np.full(128, -128, dtype=np.int8)
    with pytest.raises(AssertionError, match="y32 overflow"):
        law.matvec_y32(w4, m, 0, x8)


# --------------------------------------------------------------- a8 DYNQ8
def test_dynq8_vectors(vectors):
    for s in range(1, 5):
        x8, e = law.dyn_quant_i8(vectors[f"s{s}_alu_dynq8_x"])
        assert np.array_equal(x8.astype(np.int64), vectors[f"s{s}_alu_dynq8_y"])
        assert e == int(vectors[f"s{s}_alu_dynq8_e"][0])


def test_dynq8_brute_force():
    rng = np.random.default_rng(9)
    for _ in range(200):
        scale = int(rng.integers(1, 32768))
        x = rng.integers(-scale, scale + 1, 64)
        x[0] = int(rng.choice([-1, 1])) * int(rng.integers(0, 32769))
        x = np.clip(x, -32768, 32767)
        x8, e = law.dyn_quant_i8(x)
        # least e with every rounded magnitude <= 127
        e_bf = next(k for k in range(17)
                    if np.abs(law.rshift_round(x, k)).max() <= 127)
        assert e == e_bf
        assert np.array_equal(x8.astype(np.int64), law.rshift_round(x, e))
    x8, e = law.dyn_quant_i8(np.array([-32768, 5]))
    assert e == 9 and int(x8[0]) == -64


# ------------------------------------------------------------ a9 RMSNorm
def test_rsqrt_lut_rom(vectors):
    assert np.array_equal(law.rsqrt_lut(), vectors["rom_rsqrt"])


def test_rsqrt_cases(vectors):
    for s in range(1, 5):
        for v, P, r, e in vectors[f"rsqrt_cases{s}"]:
            got = law.rsqrt_q(int(v), int(P))
            assert got == (int(r), int(e)), (v, P)


def test_rmsnorm_vectors(vectors):
    for s in range(1, 5):
        y = law.rmsnorm_fx(vectors[f"s{s}_rmsnorm_x16"],
                           vectors[f"s{s}_rmsnorm_w14"], 8, True)
        assert np.array_equal(y, vectors[f"s{s}_rmsnorm_y16"])
    # mode 1 with folded weights == mode 0 (the C1 equivalence)
    x = vectors["s1_rmsnorm_x16"]
    w = vectors["s1_rmsnorm_w14"]
    assert np.array_equal(law.rmsnorm_fx(x, w + (1 << 14), 8, False),
                          law.rmsnorm_fx(x, w, 8, True))


# ----------------------------------------------------- a11 FFN epilogues
def test_sigmoid_rom(vectors):
    assert np.array_equal(law.sigmoid_table(), vectors["rom_sigmoid"])


def test_silu_cases(vectors):
    for s in range(1, 5):
        for x, y in vectors[f"silu_cases{s}"]:
            assert int(law.clip16(law.silu_q(int(x)))) == int(y), x


def test_alu_silu32_emul32_vectors(vectors):
    for s in range(1, 5):
        v = vectors[f"s{s}_alu_shift32_v"]
        assert np.array_equal(law.alu_silu32(v, 0), vectors[f"s{s}_alu_silu32_y"])
        assert np.array_equal(law.alu_emul32(v, vectors[f"s{s}_alu_emul_b"], 15),
                              vectors[f"s{s}_alu_emul32_y"])


# -------------------------------------------------------- a10 MOVY shift
# in_f - out_f of each matrix of the 0.8B-geometry layer scripts (RS_F 8):
# the ->12 projections are in_b/in_a (wid 2, 3) and the two MLP gates.
_IN_MINUS_OUT = {2: -4, 3: -4, 5: -4, 12: -4}
_ALU_OP = {5: 6, 6: 9, 12: 6, 13: 9}       # SILU32 / SHIFT32W; others SHIFT32


def test_movy_shift_identity_from_commands(scripts):
    n = 0
    for tag in script_tags():
        for rec in script_records(scripts, tag):
            cmd = rec["cmd"]
            if cmd is None or int(cmd[0]) != 11 or (int(cmd[1]) & 0xF) == 10:
                continue
            a0, a2 = int(cmd[1]), int(cmd[3])
            op = a0 & 0xF
            p0 = (a2 & 0xFFFF) | (((a0 >> 18) & 1) << 16)
            p0 = p0 - (1 << 17) if p0 >= (1 << 16) else p0
            d = _IN_MINUS_OUT.get(rec["wid"], 0)
            assert p0 == law.shift_for(rec["e"], rec["sh"], rec["e_x"], d, 0), \
                (tag, rec["v"])
            assert op == _ALU_OP.get(rec["wid"], 1)
            n += 1
    assert n > 300


def _alu_p0(cmd):
    """p0 of a layer-command ALU record (the retired ARG layout of the
    committed scripts): low 16 bits of ARG2 with bit 18 of ARG0 as bit 16,
    sign-extended from 17 bits."""
    a0, a2 = int(cmd[1]), int(cmd[3])
    p0 = (a2 & 0xFFFF) | (((a0 >> 18) & 1) << 16)
    return p0 - (1 << 17) if p0 >= (1 << 16) else p0


def test_swiglu_chain_from_scripts(scripts):
    # gen_layer_script.py:2166-2190 mlp_block: gate y32 -> SILU32 (its
    # command's p0), up y32 -> SHIFT32W (its p0), EMUL32 by the gate at
    # p0 = 12, DYNQ8 over the FFN width = the down projection's R record
    # (x8) and E record (e_x), for the first MLP block of every script
    n = 0
    for tag in script_tags():
        gv, uv, dv = (int(v) for v in scripts[f"{tag}_mlp_v"])
        cg, cu = scripts[f"{tag}_v{gv}_cmd"], scripts[f"{tag}_v{uv}_cmd"]
        assert int(cg[1]) & 0xF == 6 and int(cu[1]) & 0xF == 9   # SILU32, SHIFT32W
        sg = law.alu_silu32(scripts[f"{tag}_mlp_gate_y32"], _alu_p0(cg))
        u = law.alu_shift32w(scripts[f"{tag}_mlp_up_y32"], _alu_p0(cu))
        prod = law.alu_emul32(u, sg, 12)
        x8, e = law.dyn_quant_i8(prod)
        assert np.array_equal(x8, scripts[f"{tag}_mlp_down_x8"]), tag
        assert e == int(scripts[f"{tag}_mlp_down_e"][0]), tag
        # the down record reads exactly this vector
        assert np.array_equal(scripts[f"{tag}_v{dv}_x8"], x8)
        n += 1
    assert n == 8


def test_emul32_of_clipped_up_equals_unclipped():
    # ref/layer_fixed.py:1597-1602 multiplies the unclipped int64 up value
    # u; the engine's SHIFT32W keeps clip32(u).  clip16(rshift_round(sg * u,
    # 12)) is the same for both whenever |u| < 2^48 (the reference's int64
    # product exact): beyond int32 both saturate to the rail of sg * u.
    # Brute force over every sg and rail-adjacent, random and extreme u.
    sg = np.arange(-32768, 32768, dtype=np.int64)
    rng = np.random.default_rng(11)
    us = [0, 1, -1, 2 ** 31 - 1, -2 ** 31, 2 ** 31, -2 ** 31 - 1, 2 ** 47, -2 ** 47,
          2 ** 48 - 1, -(2 ** 48 - 1)]
    us += list(rng.integers(-2 ** 48 + 1, 2 ** 48, 40))
    us += list(rng.integers(-2 ** 33, 2 ** 33, 40))
    us += list(rng.integers(-2 ** 20, 2 ** 20, 20))
    for u in us:
        u = np.int64(u)
        ref = law.clip16(law.rshift_round(sg * u, 12))
        eng = law.alu_emul32(np.full(sg.shape, law.clip32(np.array([u]))[0]), sg, 12)
        assert np.array_equal(ref, eng), int(u)


# ----------------------------------------------------------- a12 AMAX32
def test_amax32_a_records(scripts):
    n = 0
    for tag in script_tags():
        for idx, val, y in script_argmax(scripts, tag):
            assert law.amax32(y) == (idx, val)
            assert idx == int(np.argmax(y)) and val == int(y[idx])
            n += 1
    assert n == 12


def test_amax32_ties_lowest_index():
    rng = np.random.default_rng(3)
    for _ in range(50):
        y = rng.integers(-1000, 1000, 5000)
        top = int(y.max())
        pos = rng.choice(5000, 4, replace=False)
        y[pos] = top + 7
        assert law.amax32(y) == (int(pos.min()), top + 7)
    assert law.amax32(np.full(4097, -5)) == (0, -5)
    st = law.Amax32().feed([1, 9, 9], fresh=True)
    assert (st.idx, st.val) == (1, 9)
    st.feed([9, 10])           # continues the scan: global index 4
    assert (st.idx, st.val) == (4, 10)


# ----------------------------------------------------------- TOPK-32
def _topk_lexsort(y):
    """the first 32 elements by (value desc, arrival asc)"""
    y = np.asarray(y, dtype=np.int64)
    order = np.lexsort((np.arange(y.size), -y))[:32]
    return y[order], order


def _ovf_prefix_counts(y):
    """overflow, independently: some arrival i >= 32 had fewer than 32
    earlier elements above it and at least 32 at or above it (it tied the
    32nd largest value so far and was rejected)"""
    y = np.asarray(y, dtype=np.int64)
    for i in range(32, y.size):
        g = int(np.count_nonzero(y[:i] > y[i]))
        ge = int(np.count_nonzero(y[:i] >= y[i]))
        if g < 32 <= ge:
            return True
    return False


def test_topk32_is_lexsort_and_prefix_count_overflow():
    rng = np.random.default_rng(21)
    for trial in range(200):
        n = int(rng.integers(1, 400))
        alpha = int(rng.choice([3, 8, 40, 1 << 30]))
        y = rng.integers(-alpha, alpha + 1, n)
        vals, idx, count, ovf = law.topk32(y, chunk=int(rng.integers(1, 300)))
        ev, ei = _topk_lexsort(y)
        assert count == min(32, n)
        assert np.array_equal(vals, ev) and np.array_equal(idx, ei), trial
        assert ovf == _ovf_prefix_counts(y), trial


def test_topk32_entry0_is_amax32_on_script_heads(scripts):
    n = 0
    for tag in script_tags():
        for idx, val, y in script_argmax(scripts, tag):
            vals, ids, count, _ = law.topk32(y)
            assert (int(ids[0]), int(vals[0])) == (idx, val)
            assert count == 32
            n += 1
    assert n == 12


def test_topk32_named_cases():
    I32MAX, I32MIN = (1 << 31) - 1, -(1 << 31)
    rng = np.random.default_rng(7)
    # fewer than 32 elements: count stops at n, no overflow possible
    for n in (1, 2, 8, 17, 31):
        y = rng.integers(I32MIN, I32MAX, n)
        _, _, count, ovf = law.topk32(y)
        assert count == n and not ovf
    # 40 x MAX then 40 x MIN: 32 copies of MAX, first 32 indices, overflow
    vals, idx, count, ovf = law.topk32([I32MAX] * 40 + [I32MIN] * 40)
    assert count == 32 and ovf and (vals == I32MAX).all()
    assert np.array_equal(idx, np.arange(32))
    # the 33rd element ties entry[31] exactly: literal overflow
    v = sorted(rng.choice(np.arange(1000, 9000), 32, replace=False).tolist(), reverse=True)
    y = v + [v[31]]
    assert law.topk32(y)[3]
    # entries 30 and 31 equal, then a bigger element displaces entry 31:
    # the literal bit stays clear, the displaced-tie reading sets
    v = sorted(rng.choice(np.arange(1000, 9000), 31, replace=False).tolist(), reverse=True)
    y = v + [v[30], I32MAX]
    st = law.Topk32().feed(y, fresh=True)
    assert not st.ovf_lit and st.ovf_disp
    assert st.lst[0] == (I32MAX, 32)
    # rails among random values: signed compare at both ends
    y = rng.integers(I32MIN, I32MAX, 200)
    y[[0, 5, 77, 199, 3, 100]] = I32MAX
    y[[1, 6, 78, 198]] = I32MIN
    vals, idx, _, _ = law.topk32(y)
    assert list(idx[:6]) == [0, 3, 5, 77, 100, 199] and (vals[:6] == I32MAX).all()
    # chained chunks without fresh accumulate into one list; fresh clears
    st = law.Topk32().feed([5, 1], fresh=True).feed([9])
    assert st.lst[:3] == [(9, 2), (5, 0), (1, 1)]
    st.feed([3], fresh=True)
    assert st.lst == [(3, 0)]
    # the index is the 18-bit element counter: it wraps, ties still go by
    # arrival
    y = np.zeros((1 << 18) + 10, dtype=np.int64)
    y[(1 << 18) + 4] = 7
    vals, idx, _, _ = law.topk32(y)
    assert (int(vals[0]), int(idx[0])) == (7, 4)
    assert list(idx[1:4]) == [0, 1, 2]


# ---------------------------------------------- matvec_to / dequant bound
def test_matvec_to_float_bound():
    # the integer pipeline equals dequantised float math to the final
    # rounding (w4a8_ref.py:460-481): |y32 - exact| <= 0.5 (+fp slop)
    rng = np.random.default_rng(17)
    N, K = 64, 1024
    w4 = rng.integers(-8, 8, (N, K)).astype(np.int8)
    m = rng.integers(256, 16385, (N, K // 128)).astype(np.uint16)
    x8 = rng.integers(-127, 128, K).astype(np.int8)
    sh = law.sh_for_k(K)
    y = law.matvec_y32(w4, m, sh, x8)
    deq = (w4.reshape(N, -1, 128).astype(np.float64)
           * m[:, :, None].astype(np.float64)).reshape(N, K)
    exact = deq @ x8.astype(np.float64) / (1 << sh)
    assert np.abs(y - exact).max() <= 0.51
