"""TOPK-32 as a plan's LM head (w4a8_plan_add_head_topk32): the layer_topk32
block fed from the head's own pass over its rows (docs/SEQ_ISA.md:582-610),
in every plan mode -- graph (the head's y32, then the TOPK-32 kernel) and
both persistent launches (the scan runs inside the launch, each 1024-row
chunk as soon as its rows are stored) -- against the oracle's running list
(oracle/law.py Topk32) on the oracle's y32: every entry, the count and the
overflow bit, bit-exact, on two runs in a row and on graph replays."""
import numpy as np
import pytest
import torch

from fable5_llm_amd import _native as N
from fable5_llm_amd.engine import Plan
from oracle import cfast, law
from tests.helpers import activation_x16, rand_image

pytestmark = pytest.mark.gpu

K = 4096
MODES = [N.PLAN_GRAPH, N.PLAN_PERSISTENT, N.PLAN_PERSISTENT_COOP]


def _want(y):
    vals, rows, count, ovf = law.topk32(y)
    out = np.zeros(66, dtype=np.int64)
    out[:count] = vals
    out[32:32 + count] = rows
    out[64], out[65] = count, int(ovf)
    return out


def _run(engine, img, nrows, x16, modes=MODES, with_site=True, runs=2):
    """The head (and, with_site, a 4096 x 4096 site before it) as a plan in
    each mode; the 66 result words of every run."""
    dev = torch.device("cuda", 0)
    sh = law.sh_for_k(K)
    w = engine.upload(img, nrows, K, sh)
    rng = np.random.default_rng(9)
    img0, _ = rand_image(rng, 4096, K)
    w0 = engine.upload(img0, 4096, K, sh)
    x0 = torch.from_numpy(activation_x16(rng, K)).to(dev)
    y0 = torch.zeros(4096, dtype=torch.int16, device=dev)
    xd = torch.from_numpy(x16.copy()).to(dev)
    out = torch.full((66,), -9, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    got = {}
    try:
        plan = Plan(engine)
        try:
            if with_site:
                plan.add_site([w0], [N.EPI_MOVY_I16], [9], [y0], x0, prologue=N.PRO_DYNQ8)
            plan.add_head_topk32(w, xd, out, prologue=N.PRO_DYNQ8)
            for mode in modes:
                plan.set_mode(mode)
                got[mode] = []
                for _ in range(runs):
                    out.fill_(-9)
                    torch.cuda.synchronize()
                    plan.run()
                    engine.sync()
                    got[mode].append(out.cpu().numpy().astype(np.int64))
                # an instrumented pass (per-site times) runs the head and its
                # scan too
                out.fill_(-9)
                torch.cuda.synchronize()
                prof = plan.profile()
                engine.sync()
                assert prof.shape == (plan.nsites,) and (prof > 0).all(), (mode, prof)
                got[mode].append(out.cpu().numpy().astype(np.int64))
        finally:
            plan.close()
    finally:
        w.free()
        w0.free()
    return got


def _check(got, want):
    for mode, outs in got.items():
        for i, o in enumerate(outs):
            assert np.array_equal(o, want), (mode, i, o[:4], want[:4], o[64:], want[64:])


@pytest.fixture(scope="module")
def head():
    rng = np.random.default_rng(123)
    n = 248320
    img, _ = rand_image(rng, n, K)
    x16 = activation_x16(rng, K)
    x8, _ = law.dyn_quant_i8(x16)
    return img.reshape(n, -1), x16, x8


def test_plan_topk_full_head(engine, head):
    rows, x16, x8 = head
    n = rows.shape[0]
    y = cfast.matvec_y32_img(rows.reshape(-1), n, K, law.sh_for_k(K), x8)
    want = _want(y)
    assert want[64] == 32
    _check(_run(engine, rows.reshape(-1), n, x16), want)


def test_plan_topk_planted_ties_and_overflow(engine, head):
    # the winner's row copied to 40 rows across chunks, super-chunks and
    # workgroups: 32 copies fill the list, the 33rd is rejected while equal
    # to entry[31] (overflow), and the lowest 32 rows are kept
    rows, x16, x8 = head
    n = rows.shape[0]
    sh = law.sh_for_k(K)
    y = cfast.matvec_y32_img(rows.reshape(-1), n, K, sh, x8)
    best = int(np.argmax(y))
    planted = rows.copy()
    rng = np.random.default_rng(4)
    at = np.unique(np.concatenate([rng.choice(n, 36, replace=False),
                                   [0, 255, 256, 1279, 1280, n - 1]]))
    planted[at] = rows[best]
    y2 = cfast.matvec_y32_img(planted.reshape(-1), n, K, sh, x8)
    want = _want(y2)
    assert want[65] == 1 and (want[:32] == y2.max()).all()
    _check(_run(engine, planted.reshape(-1), n, x16), want)


def test_plan_topk_all_zero_weights(engine, head):
    # every y32 is 0: rows 0..31 in order, and row 32 sets the overflow bit
    rows, x16, _x8 = head
    zero = rows.copy()
    zero[:, :K // 2] = 0
    want = np.zeros(66, dtype=np.int64)
    want[32:64] = np.arange(32)
    want[64], want[65] = 32, 1
    _check(_run(engine, zero.reshape(-1), rows.shape[0], x16), want)


def test_plan_topk_few_distinct_rows(engine):
    # 200,000 rows drawn from 60 distinct rows, so every value recurs
    # thousands of times, across every chunk edge
    rng = np.random.default_rng(17)
    n = 200000
    base, _ = rand_image(rng, 60, K)
    base = base.reshape(60, -1)
    pick = rng.integers(0, 60, n)
    img = base[pick]
    x16 = activation_x16(rng, K)
    x8, _ = law.dyn_quant_i8(x16)
    y = cfast.matvec_y32_img(img.reshape(-1), n, K, law.sh_for_k(K), x8)
    want = _want(y)
    _check(_run(engine, img.reshape(-1), n, x16), want)


@pytest.mark.parametrize("n", [16, 200, 256, 300, 1280, 5000])
def test_plan_topk_small_heads(engine, n):
    # one chunk (<= 256 rows), a partial second chunk, chunk edges
    rng = np.random.default_rng(n)
    img, _ = rand_image(rng, n, K)
    x16 = activation_x16(rng, K)
    x8, _ = law.dyn_quant_i8(x16)
    y = cfast.matvec_y32_img(img, n, K, law.sh_for_k(K), x8)
    want = _want(y)
    _check(_run(engine, img, n, x16, with_site=(n % 2 == 0)), want)


def test_plan_topk_graph_replays(engine, head):
    # a persistent plan with a TOPK-32 head captured into a HIP graph:
    # every replay clears the scan's flags and words and gives the same
    # result, with eager work and synchronisations between the replays
    rows, x16, x8 = head
    n = rows.shape[0]
    y = cfast.matvec_y32_img(rows.reshape(-1), n, K, law.sh_for_k(K), x8)
    want = _want(y)
    dev = torch.device("cuda", 0)
    w = engine.upload(rows.reshape(-1), n, K, law.sh_for_k(K))
    xd = torch.from_numpy(x16.copy()).to(dev)
    out = torch.full((66,), -9, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    plan = Plan(engine)
    side = torch.cuda.Stream(dev)
    try:
        plan.add_head_topk32(w, xd, out, prologue=N.PRO_DYNQ8)
        plan.set_mode(N.PLAN_PERSISTENT)
        plan.run()     # builds the plan's device tables
        engine.sync()
        assert np.array_equal(out.cpu().numpy().astype(np.int64), want)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            engine.set_stream(side)
            plan.run()
        engine.set_stream(None)
        for i in range(4):
            out.fill_(-9)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy().astype(np.int64), want), i
            plan.run()            # eager runs between the replays
            engine.sync()
            assert np.array_equal(out.cpu().numpy().astype(np.int64), want), i
    finally:
        engine.set_stream(None)
        plan.close()
        w.free()


def test_plan_topk_one_per_plan(engine):
    rng = np.random.default_rng(2)
    img, _ = rand_image(rng, 64, K)
    w = engine.upload(img, 64, K, law.sh_for_k(K))
    dev = torch.device("cuda", 0)
    x = torch.zeros(K, dtype=torch.int16, device=dev)
    out = torch.zeros(66, dtype=torch.int32, device=dev)
    plan = Plan(engine)
    try:
        plan.add_head_topk32(w, x, out)
        with pytest.raises(ValueError, match="one TOPK-32 head"):
            plan.add_head_topk32(w, x, out)
    finally:
        plan.close()
        w.free()
