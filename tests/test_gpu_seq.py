"""The .seq matvec records on the device (fable5_llm_amd.seq.SeqMachine)
against the oracle's machine model (oracle/seq_model.py) and the reference
scripts' V records: MOVX / MVGO / MOVY with XRF indirection, XOP, no-wait
MVGOs and FENCE, RES-sized row chunks of one image, the XWIN / RES banks."""
import json

import numpy as np
import pytest

from fable5_llm_amd import seq as S
from fable5_llm_amd.artifacts import Artifacts, load_weights_manifest
from fable5_llm_amd.w4a8_ref import row_beats
from oracle import law
from oracle.fixtures import script_tags
from oracle.seq_model import SeqOracle, load_images
from tests.helpers import rand_w4_m, write_fixture_artifacts
from tests.seq_streams import (I16_ADDR, PAIRS_ADDR, SEQ_STREAMS, X_ADDR, LayerShim,
                               golden_plan, golden_streams, golden_wids, movx, movy, mvgo,
                               script_stream, swin_stage, v_record_stream,
                               write_golden_artifacts, xrf_write)

pytestmark = pytest.mark.gpu


def test_script_records_on_device(engine, scripts, tmp_path):
    nv = 0
    for tag in script_tags():
        write_fixture_artifacts(tmp_path, scripts, tag)
        prefix = str(tmp_path / tag)
        ents, _ = load_weights_manifest(prefix)
        with Artifacts(engine, prefix) as art:
            m = S.SeqMachine(engine, art)
            for v in range(int(scripts[f"{tag}_counts"][0])):
                x8, recs, y, p0 = v_record_stream(scripts, tag, v, ents, m.plan)
                m.write_scratch(X_ADDR, x8)
                m.run(recs)
                assert np.array_equal(m.read_pairs(PAIRS_ADDR, y.size), y), (tag, v)
                if p0 is not None:
                    got = m.read_scratch(I16_ADDR, y.size).astype(np.int64)
                    assert np.array_equal(got, law.movy(y, p0, law.MOVY_INT16)), (tag, v)
                nv += 1
    assert nv == 372


def _synthetic(tmp_path, nrows=9000, K=1024, seed=8):
    rng = np.random.default_rng(seed)
    w4, m = rand_w4_m(rng, nrows, K)
    img, stride = law.pack_ddr_rows(w4, m)
    (tmp_path / "q_w0.bin").write_bytes(bytes(img))
    w4b, mb = rand_w4_m(rng, 512, 2048)
    imgb, strideb = law.pack_ddr_rows(w4b, mb)
    (tmp_path / "q_w1.bin").write_bytes(bytes(imgb))
    man = {"0": {"file": "q_w0.bin", "nrows": nrows, "k": K, "ng": K // 128,
                 "sh": law.sh_for_k(K), "e": -4, "nbeats": nrows * sum(row_beats(K)),
                 "stride": stride},
           "1": {"file": "q_w1.bin", "nrows": 512, "k": 2048, "ng": 16,
                 "sh": law.sh_for_k(2048), "e": -5, "nbeats": 512 * sum(row_beats(2048)),
                 "stride": strideb}}
    (tmp_path / "q.weights.json").write_text(json.dumps(man))
    return str(tmp_path / "q"), man, rng


def _both(engine, prefix, man, stage, recs):
    """Run recs on the device and in the oracle after staging scratch."""
    ents, _ = load_weights_manifest(prefix)
    plan = S.plan_weights(ents)
    o = SeqOracle(load_images(prefix, ents), plan)
    with Artifacts(engine, prefix) as art:
        m = S.SeqMachine(engine, art)
        for addr, vals in stage:
            m.write_scratch(addr, vals)
            o.mem[addr:addr + len(vals)] = vals
        m.run(recs)
        o.run(S.pack_stream(recs))
        got = m.read_scratch(0, o.mem.size).astype(np.int64)
    return got, o


def test_row_chunks_banks_xop_nowait(engine, tmp_path):
    prefix, man, rng = _synthetic(tmp_path)
    plan = S.plan_weights({k: v for k, v in man.items()})
    e0, e1 = man["0"], man["1"]
    s0, s1 = e0["stride"], e1["stride"]
    xa = rng.integers(-127, 128, 1024)
    xb = rng.integers(-127, 128, 2048)
    stage = [(0, xa), (2048, xb)]
    recs = [xrf_write(S.XRF_EX, 3), xrf_write(S.XRF_K_ATTN, 2),
            # o_proj-style shift in XRF[5]: 21 - e_x - k_a
            S.Rec(S.EXT_XOP, target=S.XRF_OSHIFT,
                  imm32=S.xop_imm(0, S.XOP_NEG, 2, S.XOP_NEG, 21)),
            movx(0, 0, 0, 1024),
            movx(1, S.XBANK_WORD, 2048, 2048)]
    # the 9000-row image in RES-sized chunks (WBASE = base + r0 * stride),
    # alternating RES banks on channel 0
    out = 16384
    for i, r0 in enumerate(range(0, 9000, 2048)):
        n = min(2048, 9000 - r0)
        recs += [mvgo(0, plan[0] + r0 * s0, 8, n, e0["sh"], s0, rbank=i & 1),
                 movy(0, S.RBANK_ROW * (i & 1), n, out + 2 * r0)]
    # channel 1: no-wait MVGO from the x bank, FENCE, then MOVY int16 through
    # XRF[5] (IND_ADD) and through XRF[0] (IND_SUB)
    recs += [mvgo(1, plan[1], 16, 512, e1["sh"], s1, xbank=1, nowait=True),
             S.Rec(S.OP_FENCE, target=0b0010),
             movy(1, 0, 512, 40000, imm=0, int16=True, ind=S.IND_ADD, xrf=S.XRF_OSHIFT),
             movy(1, 100, 300, 41000, imm=12, int16=True, ind=S.IND_SUB, xrf=S.XRF_EX),
             S.Rec(S.OP_HALT), movx(0, 0, 0, 1024)]          # after HALT: not run
    got, o = _both(engine, prefix, man, stage, recs)
    assert np.array_equal(got, o.mem)
    assert o.xrf[S.XRF_OSHIFT] == 16
    # the chunks joined give the whole image's y32
    y_full = o.pairs(out, 9000)
    assert np.array_equal(y_full, np.concatenate(
        [o.pairs(out + 2 * r0, min(2048, 9000 - r0)) for r0 in range(0, 9000, 2048)]))
    assert np.count_nonzero(y_full) > 8000


def test_hazards_refused_on_device(engine, tmp_path):
    prefix, man, rng = _synthetic(tmp_path, nrows=64)
    plan = S.plan_weights(man)
    e0 = man["0"]
    with Artifacts(engine, prefix) as art:
        m = S.SeqMachine(engine, art)
        m.write_scratch(0, rng.integers(-127, 128, 1024))
        m.run([movx(2, 0, 0, 1024), mvgo(2, plan[0], 8, 64, e0["sh"], e0["stride"],
                                         nowait=True)])
        for bad in (movy(2, 0, 64, 9000), movx(2, 0, 0, 1024),
                    mvgo(2, plan[0], 8, 64, e0["sh"], e0["stride"])):
            with pytest.raises(S.RunningChannelError):
                m.step(bad)
        m.run([S.Rec(S.OP_FENCE), movy(2, 0, 64, 9000)])
        with pytest.raises(RuntimeError, match="not inside one MVGO"):
            m.step(movy(2, 32, 64, 9000))
        with pytest.raises(S.SeqUnsupported):
            m.step(S.Rec(S.OP_CMD))
        # ranges outside scratch, the x window, RES or the channels are
        # refused on the host, before any kernel is launched
        words = m.scratch.numel()
        for bad in (movx(0, 0, words - 100, 1024),                  # scratch source
                    movx(0, S.XBANK_WORD + 1500, 0, 1024),           # x window
                    movx(5, 0, 0, 1024),                             # channel
                    movy(2, 0, 64, words - 10, int16=True),          # scratch target
                    movy(2, 0, 64, words - 100),                     # pairs32 target
                    mvgo(2, plan[0], 8, 4096, e0["sh"], e0["stride"], rbank=1)):   # RES
            with pytest.raises(ValueError):
                m.step(bad)
        m.run([movx(3, 0, 0, 512)])
        with pytest.raises(ValueError, match="x bytes"):             # x shorter than K
            m.step(mvgo(3, plan[0], 8, 64, e0["sh"], e0["stride"]))
        # a MOVX of a value outside int8 is reported at the next sync
        m.write_scratch(0, [200] + [0] * 1023)
        m.step(movx(0, 0, 0, 1024))
        with pytest.raises(AssertionError, match="int8"):
            engine.sync()


@pytest.mark.parametrize("tag", ["layer2", "token1", "token4"])
def test_whole_script_stream_on_device(engine, scripts, tmp_path, tag):
    # all of a script's V records in one stream: four channels, both x banks,
    # no-wait MVGOs drained by FENCEs, MOVYs through XRF[0]; the device's
    # scratch against the generator's y32 and the oracle machine's scratch
    write_fixture_artifacts(tmp_path, scripts, tag)
    prefix = str(tmp_path / tag)
    ents, _ = load_weights_manifest(prefix)
    with Artifacts(engine, prefix) as art, S.SeqMachine(engine, art,
                                                        scratch_words=1 << 18) as m:
        stage, recs, checks, words = script_stream(scripts, tag, ents, m.plan)
        assert words <= 1 << 18
        for a, v in stage:
            m.write_scratch(a, v)
        m.run(recs)
        for kind, a, y, p0 in checks:
            if kind == "pairs":
                assert np.array_equal(m.read_pairs(a, y.size), y), (tag, a)
            else:
                got = m.read_scratch(a, y.size).astype(np.int64)
                assert np.array_equal(got, law.movy(y, p0, law.MOVY_INT16)), (tag, a)
        o = SeqOracle(load_images(prefix, ents), m.plan, scratch_words=1 << 18)
        for a, v in stage:
            o.mem[a:a + v.size] = v
        o.run(S.pack_stream(recs))
        assert np.array_equal(m.read_scratch(0, words).astype(np.int64), o.mem[:words])


def test_broadcast_movx_on_device(engine, tmp_path):
    prefix, man, rng = _synthetic(tmp_path, nrows=256)
    plan = S.plan_weights(man)
    e0 = man["0"]
    x = rng.integers(-127, 128, 1024)
    recs = [movx(S.MOVX_BCAST, 0, 0, 1024),
            mvgo(0, plan[0], 8, 64, e0["sh"], e0["stride"]),
            mvgo(3, plan[0] + 64 * e0["stride"], 8, 128, e0["sh"], e0["stride"], nowait=True),
            movy(0, 0, 64, 4096), S.Rec(S.OP_FENCE), movy(3, 0, 128, 8192), S.Rec(S.OP_HALT)]
    got, o = _both(engine, prefix, man, [(0, x)], recs)
    assert np.array_equal(got, o.mem)
    assert np.count_nonzero(o.pairs(8192, 128)) > 100
    with Artifacts(engine, prefix) as art, S.SeqMachine(engine, art) as m:
        m.write_scratch(0, x)
        m.run([movx(2, 0, 0, 1024), mvgo(2, plan[0], 8, 64, e0["sh"], e0["stride"], nowait=True)])
        with pytest.raises(S.RunningChannelError, match="mv2"):   # a broadcast meets mv2's stream
            m.step(movx(S.MOVX_BCAST, 0, 0, 1024))


def test_pre_g3_shape_on_device(engine, scripts, tmp_path):
    # frozen artifacts' SHAPE layout (isa 1), stated to the machine
    tag = "token3"
    write_fixture_artifacts(tmp_path, scripts, tag)
    prefix = str(tmp_path / tag)
    ents, _ = load_weights_manifest(prefix)
    with Artifacts(engine, prefix) as art, S.SeqMachine(engine, art,
                                                        shape_isa=S.SHAPE_ISA_PRE_G3) as m:
        for v in range(3):
            x8, recs, y, _ = v_record_stream(scripts, tag, v, ents, m.plan)
            go = recs[2]
            ng, nrows, sh, _, _ = S.shape_fields(go.imm32)
            recs[2] = S.Rec(go.opcode, go.flags, go.target, (nrows << 12) | (sh << 6) | ng,
                            go.addr_lo, go.len_or_addr_hi)
            m.write_scratch(X_ADDR, x8)
            m.run(recs)
            assert np.array_equal(m.read_pairs(PAIRS_ADDR, y.size), y), v


def test_swin_staging_on_device(engine, scripts, tmp_path):
    from tests.test_seq import _swin_stream
    tag = "token1"
    write_fixture_artifacts(tmp_path, scripts, tag)
    prefix = str(tmp_path / tag)
    ents, _ = load_weights_manifest(prefix)
    with Artifacts(engine, prefix) as art, S.SeqMachine(engine, art) as m:
        recs, y = _swin_stream(scripts, tag, ents, m.plan)
        m.run(recs)
        got = m.read_pairs(PAIRS_ADDR, y.size)
        assert np.array_equal(got[1:], y[1:]) and m.read_scratch(PAIRS_ADDR, 1)[0] == -2
        assert m.tcnt_seq == 7


def test_host_write_after_swin_wins(engine, scripts, tmp_path):
    """A host write to a scratch word that an earlier SWIN targeted is the
    last writer (SWIN writes scratch at once, ref/seq_model.py:763-766), and
    a SWIN after the host write wins in turn; SWIN words the host write does
    not cover still land."""
    tag = "token1"
    write_fixture_artifacts(tmp_path, scripts, tag)
    prefix = str(tmp_path / tag)
    with Artifacts(engine, prefix) as art, S.SeqMachine(engine, art) as m:
        a = 3000
        for r in swin_stage(a, [11, 12, 13, 14]):
            m.step(r)                       # queued, no MOVX / MOVY / EMB after
        m.write_scratch(a + 1, [-7, -8])
        assert list(m.read_scratch(a, 4)) == [11, -7, -8, 14]
        for r in swin_stage(a + 2, [21]):
            m.step(r)
        assert list(m.read_scratch(a, 4)) == [11, -7, 21, 14]


@pytest.mark.parametrize("name", SEQ_STREAMS)
def test_reference_stream_on_device(engine, tmp_path, name):
    """A stream the reference's encoder wrote (one channel, one channel with
    no-wait MVGOs and FENCE, four channels with the head interleaved) run by
    SeqMachine, the head's AMAX32 commands applied by the test over the
    staged pairs each MOVY leaves: the scratch the reference's executor left,
    word for word, and its AMAX32 index and value
    (tests/golden/make_seq_fixtures.py)."""
    z = golden_streams()
    prefix = write_golden_artifacts(tmp_path, z)
    with Artifacts(engine, prefix) as art, \
            S.SeqMachine(engine, art, plan=golden_plan(z, name)) as m:
        for wid in golden_wids(z):
            m.write_scratch(int(z[f"w{wid}_meta"][6]), z[f"w{wid}_x8"])
        shim = LayerShim(m.read_pairs)
        n = 0
        for r in S.unpack_stream(z[f"{name}_rec"].tobytes()):
            n += 1
            if not shim.take(r) and not m.step(r):
                break
        want = z[f"{name}_mem"]
        got = m.read_scratch(0, want.size).astype(np.int64)
    assert n == z[f"{name}_rec"].size // 16
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:10]
    assert [shim.amax.idx, shim.amax.val] == list(z[f"{name}_amax"]) and shim.ncmd == 5


def _emb_artifacts(tmp_path, ntok=40, width=1024):
    """The synthetic images plus an int16 embedding table of int8-range
    values (so a MOVX can take an EMB's words), width in the manifest."""
    prefix, man, rng = _synthetic(tmp_path, nrows=256)
    emb = rng.integers(-127, 128, (ntok, width)).astype("<i2")
    (tmp_path / "q.emb.bin").write_bytes(emb.tobytes())
    man2 = dict(man, emb_row_bytes=2 * width)
    (tmp_path / "q.weights.json").write_text(json.dumps(man2))
    return prefix, man, emb


def test_emb_feeds_the_matvec_on_device(engine, tmp_path):
    prefix, man, emb = _emb_artifacts(tmp_path)
    ents, _ = load_weights_manifest(prefix)
    plan = S.plan_weights(ents)
    e0 = man["0"]
    recs = []
    for tok, addr in ((17, 0), (39, 2048), (0, 4096)):
        recs += [xrf_write(S.XRF_TOK, tok), S.Rec(S.OP_EMB, addr_lo=addr, len_or_addr_hi=1024)]
    recs += [movx(0, 0, 2048, 1024), mvgo(0, plan[0], 8, 256, e0["sh"], e0["stride"]),
             movy(0, 0, 256, 8192), S.Rec(S.OP_EMB, addr_lo=12000, len_or_addr_hi=100),
             S.Rec(S.OP_HALT)]
    o = SeqOracle(load_images(prefix, ents), plan, emb=emb)
    with Artifacts(engine, prefix) as art, S.SeqMachine(engine, art) as m:
        m.run(recs)
        o.run(S.pack_stream(recs))
        got = m.read_scratch(0, o.mem.size).astype(np.int64)
        assert np.array_equal(got, o.mem)
        assert np.array_equal(got[2048:3072], emb[39]) and np.array_equal(got[12000:12100], emb[0, :100])
        assert np.count_nonzero(o.pairs(8192, 256)) > 200
        m.set_xrf(S.XRF_TOK, 40)
        with pytest.raises(ValueError, match="token 40"):
            m.step(S.Rec(S.OP_EMB, addr_lo=0, len_or_addr_hi=8))
        m.set_xrf(S.XRF_TOK, 1)
        with pytest.raises(ValueError, match="1025 words"):
            m.step(S.Rec(S.OP_EMB, addr_lo=0, len_or_addr_hi=1025))
        with pytest.raises(ValueError, match="no flags"):
            m.step(S.Rec(S.OP_EMB, flags=1, addr_lo=0, len_or_addr_hi=8))
        with pytest.raises(ValueError, match="outside"):
            m.step(S.Rec(S.OP_EMB, addr_lo=m.scratch.numel() - 4, len_or_addr_hi=8))
