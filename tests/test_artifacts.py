"""Generator-artifact ingestion (fable5_llm_amd.artifacts) on the CPU: the
manifest split (sw/hwmap.py:502-532), each image record against the wire
format's law, the record-script grammar (gen_layer_script.py:648-702,
1487-1545), and -- where the reference's checkout is present -- every
manifest, script and V / A record of tb/scripts on the full images, the
records replayed through the oracle."""
import json
import os

import numpy as np
import pytest

from fable5_llm_amd import artifacts as A
from fable5_llm_amd.w4a8_ref import row_beats, row_stride
from oracle import cfast, law

REF_SCRIPTS = "/root/reference/tb/scripts"
TAGS = [f"{k}_s{s}" for k in ("layer", "token") for s in range(1, 5)]


def _entry(nrows, k, **kw):
    e = {"file": "x_w0.bin", "nrows": nrows, "k": k, "ng": k // 128,
         "sh": law.sh_for_k(k), "e": -4, "nbeats": nrows * sum(row_beats(k)),
         "stride": row_stride(k)}
    e.update(kw)
    return e


def test_split_manifest_defaults_and_filter():
    wids, meta = A.split_manifest({"0": _entry(16, 1024), "rs_f": 7, "state": {"a": 1}})
    assert list(wids) == ["0"]
    assert meta["rs_f"] == 7 and meta["emb_row_bytes"] == 8192
    assert meta["state"] == {"a": 1} and meta["conv_images"] is None


def test_check_entry_law_and_rejections():
    e = _entry(100, 2048)
    assert A.check_entry(0, e, 100 * row_stride(2048)) == (100, 2048, law.sh_for_k(2048))
    with pytest.raises(AssertionError, match="holds"):
        A.check_entry(0, e, 100 * row_stride(2048) - 64)
    with pytest.raises(AssertionError, match="stride"):
        A.check_entry(0, _entry(100, 2048, stride=1024), 100 * 1024)
    with pytest.raises(AssertionError, match="nbeats"):
        A.check_entry(0, _entry(100, 2048, nbeats=5), 100 * row_stride(2048))
    with pytest.raises(AssertionError, match="ng"):
        A.check_entry(0, _entry(100, 2048, ng=8), 100 * row_stride(2048))
    with pytest.raises(ValueError, match="8-bit"):
        A.check_entry(0, _entry(100, 2048, w8=True), 0)
    with pytest.raises(ValueError, match="group size"):
        A.check_entry(0, _entry(100, 2048, g=64), 0)


def test_parse_script_grammar(tmp_path):
    p = tmp_path / "s.txt"
    p.write_text("W 10 2\nffff\n0001\nT 0\nM 737 0 400\nR 20 3\n007f\nff81\n0000\n"
                 "E 3\nV 2 20 3 2\n80000000\n7fffffff\nC a 1 2 3\nA 5 fffffffe\nQ\n")
    recs = list(A.parse_script(str(p)))
    assert [r.kind for r in recs] == ["W", "T", "M", "R", "E", "V", "C", "A", "Q"]
    assert recs[0].fields == (0x10, 2) and list(recs[0].data) == [-1, 1]
    assert list(recs[3].data) == [127, -127, 0]
    assert recs[5].fields == (2, 0x20, 3, 2)
    assert list(recs[5].data) == [-(1 << 31), (1 << 31) - 1]
    assert recs[7].fields == (5, 0xFFFFFFFE) and recs[8].fields == ()


def _have_reference():
    return os.path.isdir(REF_SCRIPTS)


@pytest.mark.skipif(not _have_reference(), reason="the reference's tb/scripts are not here")
@pytest.mark.parametrize("tag", TAGS)
def test_reference_artifacts_replay_through_oracle(tag, scripts):
    # every image record validates against its file; every V record's y32
    # and every A record's (idx, val) come back from the oracle on the FULL
    # images, exactly as the generator asserted them
    prefix = f"{REF_SCRIPTS}/{tag}"
    ents, meta = A.load_weights_manifest(prefix)
    imgs = {}
    for key, e in ents.items():
        path = os.path.join(REF_SCRIPTS, e["file"])
        nrows, k, sh = A.check_entry(int(key), e, os.path.getsize(path))
        imgs[int(key)] = (np.memmap(path, dtype=np.uint8, mode="r"), nrows, k, sh)
    last_r = last_v = None
    nv = na = 0
    for rec in A.parse_script(prefix + ".txt"):
        if rec.kind == "R":
            last_r = rec
        elif rec.kind == "V":
            wid, xa, nin, nout = rec.fields
            img, nrows, k, sh = imgs[wid]
            assert last_r.fields == (xa, nin) and (nin, nout) == (k, nrows)
            x8 = last_r.data.astype(np.int8)
            y = cfast.matvec_y32_img(np.asarray(img), nrows, k, sh, x8)
            assert np.array_equal(y.astype(np.int64), rec.data), (tag, nv)
            last_v = (wid, y)
            nv += 1
        elif rec.kind == "A":
            idx, val = rec.fields
            val = val - (1 << 32) if val >= (1 << 31) else val
            assert last_v[0] == max(imgs)          # the head's rows
            assert law.amax32(last_v[1]) == (idx, val), (tag, na)
            na += 1
    fx = {"layer": "layer", "token": "token"}[tag.split("_")[0]] + tag[-1]
    assert (nv, na) == tuple(int(v) for v in scripts[f"{fx}_counts"])
