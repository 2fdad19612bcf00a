"""The persistent plan's prologue arithmetic when a site reads its input
through an earlier site's stamped words, on extreme inputs: each consumer
site's x is a producer site's MOVY int16 output driven to the rails
(-32768 everywhere, alternating +32767 / -32768, one outlier among zeros),
to zero, to small values or over the full range.  The consumers run RMSNorm
(mode 0 and 1, in_f at 0, 7 and 40) or DYNQ8 at K = 4096 and 2048, right
after their producer (the prologue shared with the control wavefront) or
with another producer in between (the three prologue wavefronts alone).
Every consumer's x8, e_x, RMSNorm output and MOVY output, and every
producer's output, is checked bit-exactly against the oracle
(layer_fixed.py:1242-1278, fixedpoint.py:24-33)."""
import numpy as np
import pytest
import torch

from fable5_llm_amd import _native as N
from fable5_llm_amd.engine import Plan
from oracle import cfast, law

pytestmark = pytest.mark.gpu

KA = 128        # the producers' K: one scale group
NROWS = 64      # the consumers' rows
P0 = 11         # the consumers' MOVY p0


def _producer(rng, kind, n):
    """(w4 [n, KA], m [n, 1], x16 [KA], p0): a producer whose outputs, n
    rows, are of the given kind."""
    w4 = np.zeros((n, KA), np.int8)
    m = np.full((n, 1), 16384, np.uint16)
    x16 = np.full(KA, 1000, np.int16)        # DYNQ8: e = 3, x8 = 125
    p0 = 3                                   # MOVY shift 0: clip16(y32)
    if kind == "min":
        w4[:] = -8
    elif kind == "rails":
        w4[0::2] = 7
        w4[1::2] = -8
    elif kind == "outlier":
        w4[n // 3] = 7
    elif kind == "zeros":
        pass
    elif kind == "small":
        w4 = rng.integers(-1, 2, (n, KA)).astype(np.int8)
        m[:] = 1
        p0 = 3 + 4                           # y32 of a few units, shifted right by 4
    else:                                    # "full": the int16 range, some clipped
        w4 = rng.integers(-8, 8, (n, KA)).astype(np.int8)
        m = rng.integers(1, 2048, (n, 1)).astype(np.uint16)
        x16 = rng.integers(-32768, 32768, KA).astype(np.int16)
        p0 = 3 + 2
    return w4, m, x16, p0


def _cases(rng):
    """(producer kind, consumer K, prologue, norm_w, in_f, one_plus)"""
    R, D = N.PRO_RMSNORM_DYNQ8, N.PRO_DYNQ8
    full = lambda k: rng.integers(-32768, 32768, k).astype(np.int16)
    return [
        ("min", 4096, R, np.full(4096, -32768, np.int16), 0, True),
        ("rails", 4096, R, np.full(4096, 32767, np.int16), 40, True),
        ("outlier", 4096, R, full(4096), 7, True),
        ("zeros", 4096, R, full(4096), 7, True),
        ("small", 4096, R, full(4096), 40, False),
        ("small", 2048, R, full(2048), 0, True),
        ("full", 4096, R, full(4096), int(rng.integers(0, 41)), False),
        ("full", 2048, R, full(2048), int(rng.integers(0, 41)), True),
        ("min", 4096, D, None, 0, True),
        ("rails", 2048, D, None, 0, True),
        ("zeros", 4096, D, None, 0, True),
        ("full", 4096, D, None, 0, True),
    ]


def _consumer_oracle(img, k, x16, prologue, nw, in_f, one_plus):
    x = x16
    xn = None
    if prologue == N.PRO_RMSNORM_DYNQ8:
        x = xn = law.rmsnorm_fx(x16, nw, in_f, one_plus)
    x8, e = law.dyn_quant_i8(x)
    y = cfast.matvec_y32_img(img, NROWS, k, law.sh_for_k(k), x8, 0)
    return xn, x8, e, law.movy(y, P0 - e, law.MOVY_INT16)


@pytest.mark.parametrize("mode", [N.PLAN_PERSISTENT, N.PLAN_PERSISTENT_COOP])
@pytest.mark.parametrize("gap", [False, True])
def test_stamped_prologues_extreme(engine, mode, gap):
    rng = np.random.default_rng(7 + gap)
    dev = torch.device("cuda", 0)
    cases = _cases(rng)
    weights, keep, pairs = [], [], []
    plan = Plan(engine)
    try:
        for kind, k, pro, nw, in_f, one_plus in cases:
            w4a, ma, xa, p0a = _producer(rng, kind, k)
            imga, _ = law.pack_ddr_rows(w4a, ma)
            wa = engine.upload(imga, k, KA, law.sh_for_k(KA))
            w4b = rng.integers(-8, 8, (NROWS, k)).astype(np.int8)
            mb = rng.integers(256, 16385, (NROWS, k // 128)).astype(np.uint16)
            imgb, _ = law.pack_ddr_rows(w4b, mb)
            wb = engine.upload(imgb, NROWS, k, law.sh_for_k(k))
            weights += [wa, wb]
            outa = torch.full((k,), 0x5A5A, dtype=torch.int16, device=dev)
            outb = torch.full((NROWS,), 0x5A5A, dtype=torch.int16, device=dev)
            x8 = torch.zeros(k, dtype=torch.int8, device=dev)
            e_x = torch.full((1,), -99, dtype=torch.int32, device=dev)
            xn = torch.zeros(k, dtype=torch.int16, device=dev) if nw is not None else None
            pairs.append(dict(wa=wa, xa=torch.from_numpy(xa).to(dev), p0a=p0a, outa=outa, wb=wb,
                              outb=outb, pro=pro,
                              nw=None if nw is None else torch.from_numpy(nw).to(dev),
                              in_f=in_f, one_plus=one_plus, x8=x8, e_x=e_x, xn=xn))
            keep.append((kind, k, pro, nw, in_f, one_plus, np.frombuffer(imga, np.uint8), xa,
                         p0a, np.frombuffer(imgb, np.uint8)))

        def add_producer(q):
            plan.add_site([q["wa"]], [N.EPI_MOVY_I16], [q["p0a"]], [q["outa"]], q["xa"],
                          prologue=N.PRO_DYNQ8, in_f=7)

        def add_consumer(q):
            plan.add_site([q["wb"]], [N.EPI_MOVY_I16], [P0], [q["outb"]], q["outa"],
                          prologue=q["pro"], norm_w=q["nw"], in_f=q["in_f"],
                          one_plus=q["one_plus"], x8_out=q["x8"], e_x_out=q["e_x"],
                          xn_out=q["xn"])

        if not gap:
            for q in pairs:
                add_producer(q)
                add_consumer(q)
        else:
            # producer i + 1 sits between producer i and its consumer
            add_producer(pairs[0])
            for i in range(len(pairs)):
                if i + 1 < len(pairs):
                    add_producer(pairs[i + 1])
                add_consumer(pairs[i])
        plan.set_mode(mode)
        plan.set_fences(N.FENCE_AUTO)
        torch.cuda.synchronize()
        for rep in range(2):
            for q in pairs:
                q["outa"].fill_(0x5A5A)
                q["outb"].fill_(0x5A5A)
            torch.cuda.synchronize()
            plan.run()
            engine.sync()
            for q, (kind, k, pro, nw, in_f, one_plus, imga, xa, p0a, imgb) in zip(pairs, keep):
                name = (kind, k, pro, in_f, one_plus, rep)
                x8a, ea = law.dyn_quant_i8(xa)
                ya = cfast.matvec_y32_img(imga, k, KA, law.sh_for_k(KA), x8a, 0)
                xb = np.asarray(law.movy(ya, p0a - ea, law.MOVY_INT16), np.int16)
                assert np.array_equal(q["outa"].cpu().numpy().astype(np.int64),
                                      xb.astype(np.int64)), name
                r_xn, r_x8, r_e, r_out = _consumer_oracle(imgb, k, xb, pro, nw, in_f, one_plus)
                assert int(q["e_x"].item()) == r_e, name
                assert np.array_equal(q["x8"].cpu().numpy(), r_x8), name
                if r_xn is not None:
                    assert np.array_equal(q["xn"].cpu().numpy().astype(np.int64),
                                          np.asarray(r_xn, np.int64)), name
                assert np.array_equal(q["outb"].cpu().numpy().astype(np.int64),
                                      np.asarray(r_out, np.int64)), name
    finally:
        plan.close()
        for w in weights:
            w.free()


def test_extreme_producers_reach_the_rails():
    """The producers above give what their names say (checked on the oracle,
    on the CPU): the consumers' inputs do reach the rails, zero and small
    values."""
    rng = np.random.default_rng(1)
    for kind, want in (("min", {-32768}), ("rails", {32767, -32768}), ("zeros", {0}),
                       ("outlier", {0, 32767})):
        w4, m, x16, p0 = _producer(rng, kind, 256)
        img, _ = law.pack_ddr_rows(w4, m)
        x8, e = law.dyn_quant_i8(x16)
        y = cfast.matvec_y32_img(np.frombuffer(img, np.uint8), 256, KA, law.sh_for_k(KA), x8, 0)
        out = set(int(v) for v in law.movy(y, p0 - e, law.MOVY_INT16))
        assert out == want, (kind, out)
    w4, m, x16, p0 = _producer(rng, "small", 256)
    img, _ = law.pack_ddr_rows(w4, m)
    x8, e = law.dyn_quant_i8(x16)
    y = cfast.matvec_y32_img(np.frombuffer(img, np.uint8), 256, KA, law.sh_for_k(KA), x8, 0)
    out = np.asarray(law.movy(y, p0 - e, law.MOVY_INT16))
    assert np.abs(out).max() <= 64 and np.count_nonzero(out) > 0
