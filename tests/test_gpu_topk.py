"""TOPK-32 on the device (docs/SEQ_ISA.md B8) against the oracle's running
list (oracle/law.py Topk32, the model of tb/scripts/gen_topk_cases.py),
on the reference scripts' heads and on adversarial vectors: every entry,
the count and the overflow bit, bit-exact."""
import numpy as np
import pytest

from fable5_llm_amd import _native as N
from oracle import cfast, law
from oracle.fixtures import script_argmax, script_tags
from tests.helpers import activation_x16, rand_w4_m

pytestmark = pytest.mark.gpu

I32MAX, I32MIN = (1 << 31) - 1, -(1 << 31)


def _same(got, y):
    vals, rows, count, ovf = law.topk32(y)
    g_vals, g_rows, g_count, g_ovf = got
    assert g_count == count
    assert np.array_equal(g_vals, vals) and np.array_equal(g_rows, rows)
    assert g_ovf == ovf
    return ovf


def test_topk32_script_heads(engine, scripts):
    n = 0
    for tag in script_tags():
        for idx, val, y in script_argmax(scripts, tag):
            got = engine.topk32(y)
            _same(got, y)
            assert (int(got[1][0]), int(got[0][0])) == (idx, val)
            n += 1
    assert n == 12


def _cases():
    rng = np.random.default_rng(31)
    out = {}
    for n in (1, 2, 31, 32, 33, 1023, 1024, 1025):
        out[f"n{n}"] = rng.integers(I32MIN, I32MAX, n)
    out["rails_only"] = np.array([I32MAX] * 40 + [I32MIN] * 40)
    v = sorted(rng.choice(np.arange(1000, 9000), 32, replace=False).tolist(), reverse=True)
    out["tie_at_31"] = np.array(v + [v[31]])
    v = sorted(rng.choice(np.arange(1000, 9000), 31, replace=False).tolist(), reverse=True)
    out["tie_displaced"] = np.array(v + [v[30], I32MAX])
    for a in (3, 8, 40):
        out[f"alpha{a}"] = rng.integers(-a, a + 1, 248320)
    out["random_head"] = rng.integers(I32MIN, I32MAX, 248320)
    out["rising"] = np.arange(1 << 18, dtype=np.int64) - (1 << 17)   # every row inserts
    out["falling"] = -np.arange(1 << 18, dtype=np.int64)
    out["all_equal"] = np.full(248320, 5)
    # a tie with entry[31] only at the first row of a later chunk: on a
    # rising ramp, entry[31] at row 5120 is 5120 - 32
    y = np.arange(100000, dtype=np.int64)
    y[5 * 1024] = 5 * 1024 - 32
    out["tie_after_chunk_edge"] = y
    # entry[31] rises to a value that a late row then ties exactly
    y = rng.integers(0, 1000, 200000)
    y[:32] = np.arange(10000, 10032)
    y[150000] = 10000
    out["late_tie"] = y
    return out


CASES = _cases()


@pytest.mark.parametrize("name", sorted(CASES))
def test_topk32_adversarial(engine, name):
    y = CASES[name]
    ovf = _same(engine.topk32(y), y)
    if name in ("rails_only", "tie_at_31", "all_equal", "alpha3", "tie_after_chunk_edge",
                "late_tie"):
        assert ovf
    if name in ("tie_displaced", "rising", "falling", "n31"):
        assert not ovf


def test_topk32_rejects_more_than_2_18(engine):
    with pytest.raises(AssertionError, match="2\\^18"):
        engine.topk32(np.zeros((1 << 18) + 1, np.int32))


@pytest.mark.parametrize("nrows", [50000, 248320])
def test_head_topk32_matches_oracle(engine, nrows):
    K = 4096
    rng = np.random.default_rng(nrows)
    w4, m = rand_w4_m(rng, nrows, K)
    img, _ = law.pack_ddr_rows(w4, m)
    sh = law.sh_for_k(K)
    w = engine.upload(img, nrows, K, sh)
    try:
        x16 = activation_x16(rng, K)
        got = engine.head_topk32(w, x16, prologue=N.PRO_DYNQ8)
        x8, _ = law.dyn_quant_i8(x16)
        y = cfast.matvec_y32_img(img, nrows, K, sh, x8)
        _same(got, y)
        assert (int(got[1][0]), int(got[0][0])) == engine.head_argmax(w, x16, prologue=N.PRO_DYNQ8)
    finally:
        w.free()


def test_head_topk32_zero_weights_tie_storm(engine):
    nrows, K = 5000, 1024
    w4 = np.zeros((nrows, K), np.int8)
    m = np.full((nrows, K // 128), 300, np.uint16)
    img, _ = law.pack_ddr_rows(w4, m)
    w = engine.upload(img, nrows, K, law.sh_for_k(K))
    try:
        vals, rows, count, ovf = engine.head_topk32(w, np.ones(K, np.int8))
        assert count == 32 and ovf and (vals == 0).all()
        assert np.array_equal(rows, np.arange(32))
    finally:
        w.free()


def test_head_topk32_async_graph_replays(engine):
    # Captured, the launch clears the look-back flags itself (a graph replays
    # one fixed epoch); every replay, with eager launches between them that
    # move the epoch on, gives the oracle's list.
    import torch
    nrows, K = 20000, 1024
    rng = np.random.default_rng(77)
    w4, m = rand_w4_m(rng, nrows, K)
    img, _ = law.pack_ddr_rows(w4, m)
    sh = law.sh_for_k(K)
    w = engine.upload(img, nrows, K, sh)
    dev = torch.device("cuda", 0)
    try:
        x16 = activation_x16(rng, K)
        x8, _ = law.dyn_quant_i8(x16)
        vals, rows, count, ovf = law.topk32(cfast.matvec_y32_img(img, nrows, K, sh, x8))
        ref = np.concatenate([vals, rows, [count, int(ovf)]]).astype(np.int32)
        xd = torch.from_numpy(x16.copy()).to(dev)
        out = torch.zeros(66, dtype=torch.int32, device=dev)
        eager = torch.zeros(66, dtype=torch.int32, device=dev)
        engine.head_topk32_async(w, xd, eager)   # sizes the engine's buffers
        engine.sync()
        assert np.array_equal(eager.cpu().numpy(), ref)
        side = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(g, stream=side):
                engine.set_stream(side)
                engine.head_topk32_async(w, xd, out)
        finally:
            engine.set_stream(None)
        for _ in range(3):
            out.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy(), ref)
            eager.zero_()
            torch.cuda.synchronize()
            engine.head_topk32_async(w, xd, eager)
            engine.sync()
            assert np.array_equal(eager.cpu().numpy(), ref)
    finally:
        w.free()
