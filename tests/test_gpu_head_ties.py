"""Planted argmax ties on the 248,320 x 4096 LM head inside a plan, in every
plan mode: graph (gemv_kernel's per-workgroup keys, then
argmax_final_kernel) and both persistent launches (stream_kernel: each
workgroup folds its tiles' keys in LDS, then one device-wide atomic max,
the last workgroup to arrive writing the result).

AMAX32 updates only on a strictly greater value, so among equal maxima the
lowest row wins (gen_layer_script.py:1424-1433; the head loop
gen_model_script.py:633-643 feeds the rows in ascending order), i.e.
np.argmax's first maximum.  Identical image rows give identical y32, so
copying the winning row's bytes elsewhere plants exact ties.  The copies
sit in tiles (16 rows) owned by different workgroups, and different XCDs
(the dispatcher deals workgroups to the 8 XCDs round-robin), of the plan's
one-workgroup-per-CU grid: tile t of the head goes to workgroup
(tiles before the head + t) mod G."""
import numpy as np
import pytest
import torch

from fable5_llm_amd import _native as N
from fable5_llm_amd import stream9b
from oracle import cfast, law
from tests.helpers import activation_x16, rand_image

pytestmark = pytest.mark.gpu

V, K = 248320, 4096
MODES = [N.PLAN_GRAPH, N.PLAN_PERSISTENT, N.PLAN_PERSISTENT_COOP]


@pytest.fixture(scope="module")
def head_case():
    rng = np.random.default_rng(77)
    img, _ = rand_image(rng, V, K)
    x16 = activation_x16(rng, K)
    x8, _e = law.dyn_quant_i8(x16)
    return img.reshape(V, -1), x16, x8


def _plan_run(engine, w_head, x16, mode, runs=2):
    """A plan of one 4096 x 4096 site (so that the head's tiles start one
    full grid in) and the head; the head's (index, value) after each of
    `runs` replays."""
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(5)
    img0, _ = rand_image(rng, 4096, 4096)
    w0 = engine.upload(img0, 4096, 4096, law.sh_for_k(4096))
    x0 = torch.from_numpy(activation_x16(rng, 4096)).to(dev)
    y0 = torch.zeros(4096, dtype=torch.int16, device=dev)
    xd = torch.from_numpy(x16.copy()).to(dev)
    res = torch.full((2,), -7, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    from fable5_llm_amd.engine import Plan
    plan = Plan(engine)
    got = []
    try:
        plan.add_site([w0], [N.EPI_MOVY_I16], [9], [y0], x0, prologue=N.PRO_DYNQ8)
        plan.add_head(w_head, xd, res, prologue=N.PRO_DYNQ8)
        plan.set_mode(mode)
        for _ in range(runs):
            res.fill_(-7)
            torch.cuda.synchronize()
            plan.run()
            engine.sync()
            got.append(tuple(int(v) for v in res.cpu().numpy()))
    finally:
        plan.close()
        w0.free()
    return got


def _owner(row, G, before=256):
    return (before + row // 16) % G


@pytest.mark.parametrize("lower_copy", [True, False])
def test_head_planted_ties_every_mode(engine, head_case, lower_copy):
    rows, x16, x8 = head_case
    sh = law.sh_for_k(K)
    y = cfast.matvec_y32_img(rows.reshape(-1), V, K, sh, x8)
    best = int(np.argmax(y))
    G = engine.num_cu
    t0 = best // 16
    # copies: one in the last tile, one in another tile of the winner's own
    # workgroup, and on three other XCDs; with lower_copy the lowest of them
    # lies below the winner, on another workgroup and XCD
    plant = [V - 1, V - 16, best + 16 * G if best + 16 * G < V - 16 else best - 16 * G]
    for dx in (1, 2, 5):
        t = (t0 + dx + 8 * 37) % (V // 16)
        if t == t0:
            continue
        plant.append(16 * t + (best + dx) % 16)
    if lower_copy:
        lo_t = (t0 + 3) % 8 + 8 * 11 if t0 > 8 * 12 else t0 + 8 * 9 + 3
        lo = 16 * lo_t + 9
        plant.append(lo if lo < best else 9 * 16 + 3)
    planted = rows.copy()
    for r in plant:
        planted[r] = rows[best]
    y2 = cfast.matvec_y32_img(planted.reshape(-1), V, K, sh, x8)
    want = law.amax32(y2)
    ties = np.flatnonzero(y2 == y2.max())
    assert want == (int(ties[0]), int(y2.max())) and ties.size >= len(set(plant)) + 1
    owners = {_owner(int(r), G) % 8 for r in ties}
    assert len(owners) >= 3, owners   # the tie spans XCDs
    if lower_copy:
        assert _owner(want[0], G) != _owner(best, G)
    w = engine.upload(planted.reshape(-1), V, K, sh)
    try:
        for mode in MODES:
            got = _plan_run(engine, w, x16, mode)
            assert got == [want, want], (mode, got, want)
    finally:
        w.free()


def test_head_all_zero_weights_index_zero(engine, head_case):
    # every y32 is 0: the first row, index 0, wins the 248,320-way tie
    rows, x16, _x8 = head_case
    zero = rows.copy()
    zero[:, :K // 2] = 0x00          # every int4 weight 0 (scales kept)
    w = engine.upload(zero.reshape(-1), V, K, law.sh_for_k(K))
    try:
        for mode in MODES:
            got = _plan_run(engine, w, x16, mode)
            assert got == [(0, 0), (0, 0)], (mode, got)
    finally:
        w.free()


def test_head_tie_in_the_stream_schedule(engine, head_case):
    # the headline step's own shape: the head after all 128 sites of the
    # 9B stream, so its tiles start where those sites' round-robin ends;
    # the winner's row copied to a lower row of another workgroup
    rows, x16, x8 = head_case
    sh = law.sh_for_k(K)
    y = cfast.matvec_y32_img(rows.reshape(-1), V, K, sh, x8)
    best = int(np.argmax(y))
    planted = rows.copy()
    lo = 16 * 101 + 2 if best > 16 * 101 + 2 else 2
    planted[lo] = rows[best]
    planted[V - 1] = rows[best]
    y2 = cfast.matvec_y32_img(planted.reshape(-1), V, K, sh, x8)
    want = law.amax32(y2)
    assert want[0] == min(lo, best)
    sites = stream9b.schedule()
    before = sum(-(-m.nrows // 16) for s in sites[:-1] for m in s.mats)
    G = engine.num_cu
    assert _owner(lo, G, before) != _owner(best, G, before)
    dev = torch.device("cuda", 0)
    st = stream9b.Stream9B(engine, seed=1, mode=N.PLAN_PERSISTENT, fences=N.FENCE_AUTO)
    try:
        # swap in the planted head: same shape, so the plan's site is rebuilt
        # from a fresh plan of the same sites with the head's weights replaced
        from fable5_llm_amd.engine import Plan
        w = engine.upload(planted.reshape(-1), V, K, sh)
        res = torch.full((2,), -7, dtype=torch.int32, device=dev)
        xd = torch.from_numpy(x16.copy()).to(dev)
        torch.cuda.synchronize()
        plan = Plan(engine)
        try:
            for si, s in enumerate(st.sites[:-1]):
                x, nw = st.inputs[si]
                plan.add_site(st.weights[si], [m.epi for m in s.mats],
                              [m.p0(s.in_f) for m in s.mats], st.outs[si], x,
                              prologue=s.prologue, norm_w=nw, in_f=s.in_f,
                              one_plus=s.one_plus)
            plan.add_head(w, xd, res, prologue=N.PRO_DYNQ8)
            for mode in (N.PLAN_PERSISTENT, N.PLAN_PERSISTENT_COOP):
                plan.set_mode(mode)
                plan.set_fences(N.FENCE_AUTO)
                for _ in range(2):
                    res.fill_(-7)
                    torch.cuda.synchronize()
                    plan.run()
                    engine.sync()
                    assert tuple(int(v) for v in res.cpu().numpy()) == want, mode
        finally:
            plan.close()
            w.free()
    finally:
        st.close()
