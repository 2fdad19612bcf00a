"""Generator artifacts through the device (fable5_llm_amd.artifacts): an
artifact directory written in the generators' formats from the reference
scripts' committed rows -- each image cut to its fixture rows, each V record
cut to the same rows -- loaded, uploaded and replayed on the GPU; and a
synthetic head whose A record and embedding rows the replay checks."""
import json

import numpy as np
import pytest

from fable5_llm_amd import artifacts as A
from fable5_llm_amd.w4a8_ref import row_beats
from oracle import cfast, law
from oracle.fixtures import script_tags
from tests.helpers import hexlines as _hex, rand_w4_m, write_fixture_artifacts as _write_from_fixtures

pytestmark = pytest.mark.gpu


def test_replay_script_rows(engine, scripts, tmp_path):
    total = 0
    for tag in script_tags():
        nv = _write_from_fixtures(tmp_path, scripts, tag)
        with A.Artifacts(engine, str(tmp_path / tag)) as art:
            s = A.replay(art)
        assert s["bad"] == [] and s["V"] == nv, (tag, s["bad"][:3])
        total += nv
    assert total == 372


def test_replay_head_argmax_and_embedding(engine, tmp_path):
    rng = np.random.default_rng(44)
    nrows, K = 5000, 1024
    w4, m = rand_w4_m(rng, nrows, K)
    img, stride = law.pack_ddr_rows(w4, m)
    sh = law.sh_for_k(K)
    (tmp_path / "h_w0.bin").write_bytes(bytes(img))
    man = {"0": {"file": "h_w0.bin", "nrows": nrows, "k": K, "ng": K // 128, "sh": sh,
                 "e": -4, "nbeats": nrows * sum(row_beats(K)), "stride": stride},
           "rs_f": 8}
    (tmp_path / "h.weights.json").write_text(json.dumps(man))
    emb = rng.integers(-32767, 32768, (64, K)).astype("<i2")
    (tmp_path / "h.emb.bin").write_bytes(emb.tobytes())
    x8 = rng.integers(-127, 128, K).astype(np.int8)
    y = cfast.matvec_y32_img(img, nrows, K, sh, x8)
    idx, val = law.amax32(y)
    (tmp_path / "h.txt").write_text(
        "T 0\nM 2a 0 400\n" + f"R 0 {K:x}\n" + _hex(x8, 16) + "E 3\n"
        + f"V 0 0 {K:x} {nrows:x}\n" + _hex(y, 32) + f"A {idx:x} {val & 0xFFFFFFFF:x}\nQ\n")
    with A.Artifacts(engine, str(tmp_path / "h")) as art:
        s = A.replay(art)
        assert s["bad"] == [] and (s["V"], s["A"], s["M"]) == (1, 1, 1)
        assert np.array_equal(art.embedding(K).cpu().numpy(), emb)
        # a wrong A record is reported, not raised
        (tmp_path / "h2.txt").write_text(
            f"R 0 {K:x}\n" + _hex(x8, 16) + f"V 0 0 {K:x} {nrows:x}\n" + _hex(y, 32)
            + f"A {idx + 1:x} {val & 0xFFFFFFFF:x}\n")
        bad = A.replay(art, str(tmp_path / "h2.txt"))["bad"]
        assert bad == [{"A": 0, "expected": [idx + 1, val], "got": [idx, val]}]


def test_artifacts_reject_bad_image(engine, tmp_path):
    (tmp_path / "b_w0.bin").write_bytes(bytes(576 * 15))
    man = {"0": {"file": "b_w0.bin", "nrows": 16, "k": 1024, "ng": 8, "sh": 5, "e": -4,
                 "nbeats": 144, "stride": 576}}
    (tmp_path / "b.weights.json").write_text(json.dumps(man))
    with pytest.raises(AssertionError, match="holds"):
        A.Artifacts(engine, str(tmp_path / "b"))


def test_replay_cli(scripts, tmp_path, capsys):
    # python -m fable5_llm_amd.artifacts <prefix>: one JSON line per script,
    # exit status 0 when every record matches
    tag = script_tags()[0]
    nv = _write_from_fixtures(tmp_path, scripts, tag)
    assert A.main([str(tmp_path / tag)]) == 0
    out = [l for l in capsys.readouterr().out.splitlines() if l.startswith("{")]
    s = json.loads(out[-1])
    assert s["V"] == nv and s["bad"] == []
