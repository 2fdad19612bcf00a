"""Parity of the HIP engine with the oracle and the reference's goldens.

Every test calls the engine through the C ABI (fable5_llm_amd.engine ->
libfable5_w4a8.so) and compares bit-exactly: integer law, integer results.
"""
import numpy as np
import pytest

from fable5_llm_amd import _native as N
from oracle import cfast, law
from oracle.fixtures import script_records, script_tags, vec_case
from tests.helpers import (activation_x16, log_uniform_m, norm_weight_q14,
                           rand_image, rand_w4_m)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _oracle_built():
    cfast.lib()


# ------------------------------------------------------------- tables
def test_device_tables_match_roms(engine, vectors):
    r, s = engine.tables()
    assert np.array_equal(r, vectors["rom_rsqrt"])
    assert np.array_equal(s, vectors["rom_sigmoid"])


# ------------------------------------------------------ wire round trip
def test_upload_download_roundtrip_vec(engine, vectors):
    for s in range(1, 5):
        c = vec_case(vectors, s)
        w = engine.upload(c["img"], c["N"], c["K"], c["SH"])
        assert w.download() == c["img"]
        w.free()


def test_upload_download_roundtrip_scripts(engine, scripts):
    seen = set()
    for tag in script_tags():
        for rec in script_records(scripts, tag):
            if (tag, rec["wid"]) in seen:
                continue
            seen.add((tag, rec["wid"]))
            n = rec["rows"].size
            w = engine.upload(rec["img"], n, rec["K"], rec["sh"])
            assert w.download() == rec["img"], (tag, rec["wid"])
            w.free()


def test_q9_images_and_y32(engine, q9):
    """Reference bytes and y32 at K = 4096 / 8192 / 12288 (1-3 scale beats)."""
    from tests.conftest import q9_cases
    for c in q9_cases(q9):
        w = engine.upload(c["img"], c["N"], c["K"], c["sh"])
        assert w.download() == c["img"], c["tag"]
        assert np.array_equal(engine.matvec_y32(w, c["x8"]), c["y32"]), c["tag"]
        ext = np.full(c["K"], -128, dtype=np.int8)
        assert np.array_equal(engine.matvec_y32(w, ext), c["y32_ext"]), c["tag"]
        w.free()


# ---------------------------------------------------- matvec goldens
def test_matvec_vec_goldens(engine, vectors):
    for s in range(1, 5):
        c = vec_case(vectors, s)
        w = engine.upload(c["img"], c["N"], c["K"], c["SH"])
        y = engine.matvec_y32(w, c["x8"])
        assert np.array_equal(y, c["y32"]), f"tb/vec_s{s}"
        w.free()


def test_matvec_script_v_records(engine, scripts):
    n = 0
    cache = {}
    for tag in script_tags():
        for rec in script_records(scripts, tag):
            key = (tag, rec["wid"])
            if key not in cache:
                cache[key] = engine.upload(rec["img"], rec["rows"].size, rec["K"],
                                           rec["sh"])
            y = engine.matvec_y32(cache[key], rec["x8"])
            assert np.array_equal(y, rec["y32"]), (tag, rec["v"])
            n += 1
    for w in cache.values():
        w.free()
    assert n == 372


# -------------------------------------------------- synthetic shapes
@pytest.mark.parametrize("N,K,seed", [
    (4096, 4096, 101),      # 4096 x 4096 single matvec shape
    (12288, 4096, 102),     # FFN gate/up
    (4096, 12288, 103),     # FFN down
    (1, 128, 104), (15, 256, 105), (17, 1024, 106), (33, 3584, 107),
    (100, 2048, 108), (7, 8192, 109), (1000, 1152, 110),
])
def test_matvec_synthetic(engine, N, K, seed):
    rng = np.random.default_rng(seed)
    img, m = rand_image(rng, N, K)
    x8 = rng.integers(-128, 128, K).astype(np.int8)   # -128 is a legal input
    sh = law.sh_for_k(K)
    w = engine.upload(img, N, K, sh)
    y = engine.matvec_y32(w, x8)
    assert np.array_equal(y, cfast.matvec_y32_img(img, N, K, sh, x8))
    if N * K <= 1 << 22:
        assert np.array_equal(y, law.matvec_y32_image(img.tobytes(), N, K, sh, x8))
    w.free()


def test_matvec_extremes(engine):
    # all weights -8, all x8 -128, all scales 65535: the largest |p| the
    # wire format allows; sh from the rule keeps |y| < 2^31
    K, N = 4096, 48
    w4 = np.full((N, K), -8, dtype=np.int8)
    w4[1::2] = 7
    m = np.full((N, K // 128), 65535, dtype=np.uint16)
    x8 = np.full(K, -128, dtype=np.int8)
    img, _ = law.pack_ddr_rows(w4, m)
    sh = law.sh_for_k(K)
    w = engine.upload(img, N, K, sh)
    assert np.array_equal(engine.matvec_y32(w, x8), law.matvec_y32(w4, m, sh, x8))
    w.free()


def test_matvec_y32_overflow_raises(engine):
    K = 1024
    w4 = np.full((3, K), -8, dtype=np.int8)
    m = np.full((3, K // 128), 65535, dtype=np.uint16)
    img, _ = law.pack_ddr_rows(w4, m)
    w = engine.upload(img, 3, K, 0)
    with pytest.raises(AssertionError, match="y32 overflow"):
        engine.matvec_y32(w, np.full(K, -128, dtype=np.int8))
    # the error is reported once and cleared
    y = engine.matvec_y32(w, np.zeros(K, dtype=np.int8))
    assert not y.any()
    w.free()


def test_bad_shapes_raise(engine):
    from fable5_llm_amd.engine import wire_stride
    with pytest.raises(AssertionError, match="multiple of 128"):       # K % 128
        engine.upload(np.zeros(100 * wire_stride(1000), np.uint8), 100, 1000, 7)
    with pytest.raises(AssertionError, match="envelope"):              # ng 97
        engine.upload(np.zeros(8 * wire_stride(12416), np.uint8), 8, 12416, 9)
    with pytest.raises(AssertionError, match="sh=64"):
        engine.upload(np.zeros(8 * 2112, np.uint8), 8, 4096, 64)


# --------------------------------------------------- DYNQ8 / RMSNorm
def test_dynq8_vectors(engine, vectors):
    for s in range(1, 5):
        x8, e = engine.dynq8(vectors[f"s{s}_alu_dynq8_x"])
        assert np.array_equal(x8.astype(np.int64), vectors[f"s{s}_alu_dynq8_y"])
        assert e == int(vectors[f"s{s}_alu_dynq8_e"][0])


@pytest.mark.parametrize("K,seed", [(4096, 1), (12288, 2), (64, 3), (1000, 4)])
def test_dynq8_random(engine, K, seed):
    rng = np.random.default_rng(seed)
    for scale in (1, 100, 3000, 32767):
        x = np.clip(rng.normal(0, scale, K), -32768, 32767).astype(np.int16)
        x[0] = -32768 if scale == 32767 else x[0]
        got = engine.dynq8(x)
        want = law.dyn_quant_i8(x)
        assert got[1] == want[1] and np.array_equal(got[0], want[0])


def test_rmsnorm_vectors(engine, vectors):
    for s in range(1, 5):
        y = engine.rmsnorm(vectors[f"s{s}_rmsnorm_x16"], vectors[f"s{s}_rmsnorm_w14"],
                           8, True)
        assert np.array_equal(y.astype(np.int64), vectors[f"s{s}_rmsnorm_y16"])


@pytest.mark.parametrize("n,in_f,one_plus", [(4096, 7, False), (4096, 7, True),
                                             (8192, 8, True), (256, 11, False)])
def test_rmsnorm_random(engine, n, in_f, one_plus):
    rng = np.random.default_rng(n + in_f)
    x = activation_x16(rng, n, in_f)
    w = norm_weight_q14(rng, n) - ((1 << 14) if one_plus else 0)
    assert np.array_equal(engine.rmsnorm(x, w, in_f, one_plus).astype(np.int64),
                          law.rmsnorm_fx(x, w, in_f, one_plus))
    z = np.zeros(n, np.int16)           # ss == 0 -> 1 path
    assert np.array_equal(engine.rmsnorm(z, w, in_f, one_plus).astype(np.int64),
                          law.rmsnorm_fx(z, w, in_f, one_plus))


def test_rmsnorm_rejects_non_pow2(engine):
    with pytest.raises(AssertionError, match="power of 2"):
        engine.rmsnorm(np.ones(3072, np.int16), np.ones(3072, np.int16), 7, True)


def test_rmsnorm_in_f_domain(engine):
    """in_f 0..40 keeps the reference's int64 left shift from wrapping; the
    edges of that range still match the oracle, beyond it the engine refuses."""
    rng = np.random.default_rng(5)
    x = rng.integers(-32768, 32768, 4096).astype(np.int16)
    w = rng.integers(-4000, 4000, 4096).astype(np.int16)
    for in_f in (0, 40):
        got = engine.rmsnorm(x, w, in_f, True)
        assert np.array_equal(got, law.rmsnorm_fx(x, w, in_f, True)), in_f
    for in_f in (-1, 41):
        with pytest.raises(AssertionError, match="in_f"):
            engine.rmsnorm(x, w, in_f, True)


# --------------------------------------------- MOVY / ALU / rounding
def test_movy_alu_vectors(engine, vectors):
    for s in range(1, 5):
        v = vectors[f"s{s}_alu_shift32_v"]
        assert np.array_equal(engine.alu(N.ALU_SHIFT32, v, 5), vectors[f"s{s}_alu_shift32_y"])
        assert np.array_equal(engine.alu(N.ALU_SHIFT32W, v, -8),
                              vectors[f"s{s}_alu_shift32w_y"])
        assert np.array_equal(engine.alu(N.ALU_SILU32, v, 0), vectors[f"s{s}_alu_silu32_y"])
        assert np.array_equal(engine.alu(N.ALU_EMUL32, v, 15, b=vectors[f"s{s}_alu_emul_b"]),
                              vectors[f"s{s}_alu_emul32_y"])
        assert np.array_equal(engine.movy(v, 5, N.MOVY_INT16), vectors[f"s{s}_alu_shift32_y"])
        assert np.array_equal(engine.movy(v, -8, N.MOVY_PAIRS32),
                              vectors[f"s{s}_alu_shift32w_y"])


def test_silu_cases(engine, vectors):
    for s in range(1, 5):
        c = vectors[f"silu_cases{s}"]
        got = engine.alu(N.ALU_SILU32, c[:, 0], 0)
        assert np.array_equal(got.astype(np.int64), c[:, 1])


def test_movy_random_shifts(engine):
    rng = np.random.default_rng(77)
    y = rng.integers(-(2**31) + 1, 2**31, 5000).astype(np.int32)
    y[:6] = [0, 1, -1, 2**31 - 1, -(2**31) + 1, 3]
    for shift in (-45, -40, -17, -1, 0, 1, 2, 9, 30, 62, 63, 80):
        for mode in (N.MOVY_INT16, N.MOVY_PAIRS32):
            assert np.array_equal(engine.movy(y, shift, mode).astype(np.int64),
                                  law.movy(y, shift, mode)), (shift, mode)


def test_rshift_round(engine):
    rng = np.random.default_rng(5)
    v = rng.integers(-(1 << 50), 1 << 50, 10000)
    for s in (-13, -1, 0, 1, 2, 7, 31, 50):
        assert np.array_equal(engine.rshift_round(v, s), law.rshift_round(v, s))


# ---------------------------------------------- fused prologue/epilogue
@pytest.mark.parametrize("epi", [N.EPI_Y32, N.EPI_MOVY_I16, N.EPI_MOVY_P32,
                                 N.EPI_SILU32, N.EPI_SHIFT_I64])
def test_fused_dynq8_epilogues(engine, epi):
    rng = np.random.default_rng(40 + epi)
    N_, K = 1000, 4096
    w4, _ = rand_w4_m(rng, N_, K)
    m = log_uniform_m(rng, (N_, K // 128))
    img, _ = law.pack_ddr_rows(w4, m)
    sh, e = law.sh_for_k(K), -3
    x16 = activation_x16(rng, K)
    out_f = {N.EPI_SILU32: 12}.get(epi, 7)
    p0 = (15 - e - sh) + 7 - out_f
    w = engine.upload(img, N_, K, sh)
    got, x8, e_x, _ = engine.matvec_fused(w, x16, prologue=N.PRO_DYNQ8, epilogue=epi, p0=p0)
    wx8, we = law.dyn_quant_i8(x16)
    assert e_x == we and np.array_equal(x8, wx8)
    y32 = law.matvec_y32(w4, m, sh, wx8)
    shift = p0 - we
    want = {N.EPI_Y32: y32,
            N.EPI_MOVY_I16: law.movy(y32, shift, law.MOVY_INT16),
            N.EPI_MOVY_P32: law.movy(y32, shift, law.MOVY_PAIRS32),
            N.EPI_SILU32: law.alu_silu32(y32, shift),
            N.EPI_SHIFT_I64: law.matvec_to(w4, m, e, sh, x16, 7, out_f)}[epi]
    assert np.array_equal(got.astype(np.int64), np.asarray(want, dtype=np.int64))
    w.free()


def test_fused_rmsnorm_prologue(engine):
    rng = np.random.default_rng(9)
    N_, K = 777, 4096
    w4, _ = rand_w4_m(rng, N_, K)
    m = log_uniform_m(rng, (N_, K // 128))
    img, _ = law.pack_ddr_rows(w4, m)
    sh = law.sh_for_k(K)
    x16 = activation_x16(rng, K)
    nw = norm_weight_q14(rng, K)
    w = engine.upload(img, N_, K, sh)
    for one_plus, wq in ((False, nw), (True, (nw.astype(np.int32) - (1 << 14)).astype(np.int16))):
        got, x8, e_x, xn = engine.matvec_fused(
            w, x16, prologue=N.PRO_RMSNORM_DYNQ8, epilogue=N.EPI_Y32,
            norm_w=wq, in_f=7, one_plus=one_plus)
        wxn = law.rmsnorm_fx(x16, wq, 7, one_plus)
        assert np.array_equal(xn.astype(np.int64), wxn)
        wx8, we = law.dyn_quant_i8(wxn)
        assert e_x == we and np.array_equal(x8, wx8)
        assert np.array_equal(got, law.matvec_y32(w4, m, sh, wx8))
    w.free()


# ------------------------------------------------------------- LM head
def test_head_argmax_synthetic_and_ties(engine):
    rng = np.random.default_rng(2024)
    N_, K = 20000, 4096
    img, m = rand_image(rng, N_, K)
    x8 = rng.integers(-127, 128, K).astype(np.int8)
    sh = law.sh_for_k(K)
    w = engine.upload(img, N_, K, sh)
    y = cfast.matvec_y32_img(img, N_, K, sh, x8)
    assert engine.head_argmax(w, x8) == law.amax32(y)
    w.free()
    # planted duplicate maxima: identical rows -> identical y; lowest wins
    img2 = img.reshape(N_, -1).copy()
    best = int(np.argmax(y))
    for r in (19999, 12345, best + 1 if best + 1 < N_ else 0, 5):
        img2[r] = img2[best]
    img2 = img2.reshape(-1)
    y2 = cfast.matvec_y32_img(img2, N_, K, sh, x8)
    w = engine.upload(img2, N_, K, sh)
    idx, val = engine.head_argmax(w, x8)
    assert (idx, val) == law.amax32(y2) and idx == int(np.argmax(y2))
    w.free()


def test_head_argmax_full_vocab(engine):
    # 248,320 x 4096 head (524 MB image) with a DYNQ8 hidden vector
    rng = np.random.default_rng(31)
    N_, K = 248320, 4096
    img, m = rand_image(rng, N_, K)
    x16 = activation_x16(rng, K)
    sh = law.sh_for_k(K)
    w = engine.upload(img, N_, K, sh)
    x8, e = law.dyn_quant_i8(x16)
    y = cfast.matvec_y32_img(img, N_, K, sh, x8)
    assert engine.head_argmax(w, x16, prologue=N.PRO_DYNQ8) == law.amax32(y)
    w.free()


def test_head_vocab_limit(engine):
    rng = np.random.default_rng(1)
    N_ = (1 << 18) + 16
    img, _ = rand_image(rng, N_, 128)
    w = engine.upload(img, N_, 128, 0)
    with pytest.raises(AssertionError, match="2\\^18"):
        engine.head_argmax(w, np.zeros(128, np.int8))
    w.free()


# --------------------------------------------------------- batched MFMA
@pytest.mark.parametrize("B,N_,K", [(8, 12288, 4096), (32, 4096, 12288), (1, 40, 256),
                                    (17, 100, 1024), (64, 33, 3584)])
def test_matmul_matches_per_token(engine, B, N_, K):
    rng = np.random.default_rng(B * 1000 + N_)
    img, m = rand_image(rng, N_, K)
    x8 = rng.integers(-128, 128, (B, K)).astype(np.int8)
    sh = law.sh_for_k(K)
    w = engine.upload(img, N_, K, sh)
    got = engine.matmul_y32(w, x8)
    for b in range(B):
        assert np.array_equal(got[b], cfast.matvec_y32_img(img, N_, K, sh, x8[b])), b
    w.free()


@pytest.mark.parametrize("B", [1, 5, 16, 33, 64])
def test_matmul_multi_matches_per_token(engine, B):
    # matrices of different shapes in one launch, two sharing x8, some with
    # fewer tiles than the grid (workgroups with no tile of a job skip it)
    import torch
    rng = np.random.default_rng(900 + B)
    shapes = [(12288, 4096), (12288, 4096), (40, 256), (4096, 12288), (100, 1024), (33, 3584)]
    dev = torch.device("cuda", 0)
    ws, imgs, xs, ys = [], [], [], []
    xk = {}
    for i, (N_, K) in enumerate(shapes):
        img, _ = rand_image(rng, N_, K)
        ws.append(engine.upload(img, N_, K, law.sh_for_k(K)))
        imgs.append(img)
        if K not in xk or i == 3:
            xk[K] = rng.integers(-128, 128, (B, K)).astype(np.int8)
        xs.append(xk[K])
        ys.append(torch.full((B, N_), 0x5A5A5A5A, dtype=torch.int32, device=dev))
    xd = {id(x): torch.from_numpy(x).to(dev) for x in xs}
    try:
        engine.matmul_multi_async(ws, [xd[id(x)] for x in xs], ys)
        engine.sync()
        for i, (N_, K) in enumerate(shapes):
            got = ys[i].cpu().numpy()
            for b in range(B):
                ref = cfast.matvec_y32_img(imgs[i], N_, K, law.sh_for_k(K), xs[i][b])
                assert np.array_equal(got[b], ref), (i, b)
        with pytest.raises(AssertionError, match="1..16"):
            engine.matmul_multi_async(ws * 3, [xd[id(x)] for x in xs] * 3, ys * 3)
    finally:
        for w in ws:
            w.free()


@pytest.mark.parametrize("B", [1, 8, 17, 32, 64])
def test_matmul_plan_one_launch(engine, B):
    """A matmul plan of 40 matrices (more than one launch of the per-launch
    path holds; shapes from 40 x 256 to 4096 x 12288, several sharing x8)
    in one launch: every output equal to the per-launch path's (itself
    checked per token above) and the oracle's on three tokens; a second run
    on overwritten outputs and graph replays give the same.  Up to 32 tokens
    the 4096- and 4000-row matrices (and at 17..32 the 2048-row one) run
    split into K slices whose sums meet across workgroups, so the reruns and
    replays also check that a run leaves its reduction buffers zero."""
    import torch
    from fable5_llm_amd.engine import MatmulPlan
    rng = np.random.default_rng(4100 + B)
    dev = torch.device("cuda", 0)
    base = [(12288, 4096), (4096, 12288), (40, 256), (100, 1024), (33, 3584), (2048, 2048),
            (777, 4096), (16, 128), (4000, 12288)]
    shapes = [base[i % len(base)] for i in range(40)]
    ws, imgs = {}, {}
    for N_, K in set(shapes):
        img, _ = rand_image(rng, N_, K)
        imgs[(N_, K)] = img
        ws[(N_, K)] = engine.upload(img, N_, K, law.sh_for_k(K))
    xk = {K: torch.from_numpy(rng.integers(-128, 128, (B, K)).astype(np.int8)).to(dev)
          for K in {k for _, k in shapes}}
    ys = [torch.full((B, N_), 0x5A5A5A5A, dtype=torch.int32, device=dev) for N_, _ in shapes]
    ref = [torch.zeros_like(y) for y in ys]
    plan = MatmulPlan(engine, B)
    try:
        for (N_, K), y in zip(shapes, ys):
            plan.add(ws[(N_, K)], xk[K], y)
        for i in range(0, len(shapes), 16):
            sl = shapes[i:i + 16]
            engine.matmul_multi_async([ws[s] for s in sl], [xk[k] for _, k in sl], ref[i:i + 16])
        plan.run()
        engine.sync()
        want = [r.cpu().numpy() for r in ref]
        for i, (N_, K) in enumerate(shapes):
            got = ys[i].cpu().numpy()
            assert np.array_equal(got, want[i]), i
            for b in sorted({0, B // 2, B - 1}):
                o = cfast.matvec_y32_img(imgs[(N_, K)], N_, K, law.sh_for_k(K),
                                         xk[K][b].cpu().numpy())
                assert np.array_equal(got[b], o), (i, b)
        for y in ys:
            y.fill_(-1)
        torch.cuda.synchronize()
        plan.run()
        engine.sync()
        assert all(np.array_equal(y.cpu().numpy(), w) for y, w in zip(ys, want))
        side = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(g, stream=side):
                engine.set_stream(side)
                plan.run()
        finally:
            engine.set_stream(None)
        for _ in range(2):
            for y in ys:
                y.fill_(-1)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert all(np.array_equal(y.cpu().numpy(), w) for y, w in zip(ys, want))
        with pytest.raises(AssertionError, match="at most 128"):
            for _ in range(100):
                plan.add(ws[(16, 128)], xk[128], ys[7])
    finally:
        plan.close()
        for w in ws.values():
            w.free()
