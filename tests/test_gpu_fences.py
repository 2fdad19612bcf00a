"""Plan ordering: a small plan whose sites depend on each other through
their buffers -- a site reading an earlier site's output (read after write)
and a site writing over an earlier site's input (write after read) -- run in
graph mode and in persistent mode with every fence (W4A8_FENCE_ALL) and with
fences derived from the buffers (W4A8_FENCE_AUTO), checked bit-exactly
against the oracle run site after site."""
import numpy as np
import pytest
import torch

from fable5_llm_amd import _native as N
from fable5_llm_amd import stream9b as S
from oracle import cfast, law

pytestmark = pytest.mark.gpu

K = 4096
SH = S.sh_for_k(K)


def _mat(engine, gen, nrows):
    img = S.synth_image(gen, nrows, K)
    torch.cuda.synchronize()
    return engine.upload(img, nrows, K, SH), img.cpu().numpy()


def _site_ref(img, nrows, x16, prologue, in_f, p0, norm_w=None, one_plus=True):
    x = x16
    if prologue == N.PRO_RMSNORM_DYNQ8:
        x = law.rmsnorm_fx(x16, norm_w, in_f, one_plus)
    x8, e = law.dyn_quant_i8(x)
    y = cfast.matvec_y32_img(img, nrows, K, SH, x8, 0)
    return y, e


@pytest.mark.parametrize("mode,fences", [(N.PLAN_GRAPH, N.FENCE_ALL),
                                         (N.PLAN_PERSISTENT, N.FENCE_ALL),
                                         (N.PLAN_PERSISTENT, N.FENCE_AUTO),
                                         (N.PLAN_PERSISTENT_COOP, N.FENCE_AUTO)])
def test_dependent_sites(engine, mode, fences):
    from fable5_llm_amd.engine import Plan
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(11)
    I16 = N.EPI_MOVY_I16
    # A: RMSNorm site -> outA (K rows, the next site's input)
    wA, iA = _mat(engine, gen, K)
    xA = S.synth_x16(gen, K, S.RS_F)
    nwA = S.synth_norm_w(gen, K, True)
    outA = torch.full((K,), 0x5A5A, dtype=torch.int16, device=dev)   # stale
    # B: reads outA
    wB, iB = _mat(engine, gen, K)
    outB = torch.full((K,), 0x5A5A, dtype=torch.int16, device=dev)
    # C: independent input xC
    wC, iC = _mat(engine, gen, 1024)
    xC = S.synth_x16(gen, K, S.RS_F)
    outC = torch.zeros(1024, dtype=torch.int16, device=dev)
    # D: independent input, writes its K outputs over xC (C's input)
    wD, iD = _mat(engine, gen, K)
    xD = S.synth_x16(gen, K, S.RS_F)
    xC_host = xC.cpu().numpy().copy()
    # head: argmax over outB's projection
    wH, iH = _mat(engine, gen, 2048)
    res = torch.zeros(2, dtype=torch.int32, device=dev)
    p0 = 15 - S.E_SCALE - SH   # in_f = out_f: shift = p0 - e_x

    plan = Plan(engine)
    plan.add_site([wA], [I16], [p0], [outA], xA, prologue=N.PRO_RMSNORM_DYNQ8,
                  norm_w=nwA, in_f=S.RS_F, one_plus=True)
    plan.add_site([wB], [I16], [p0], [outB], outA, prologue=N.PRO_DYNQ8, in_f=S.RS_F)
    plan.add_site([wC], [I16], [p0], [outC], xC, prologue=N.PRO_DYNQ8, in_f=S.RS_F)
    plan.add_site([wD], [I16], [p0], [xC], xD, prologue=N.PRO_DYNQ8, in_f=S.RS_F)
    plan.add_head(wH, outB, res, prologue=N.PRO_DYNQ8)
    try:
        plan.set_mode(mode)
        plan.set_fences(fences)
        torch.cuda.synchronize()
        plan.run()
        engine.sync()

        # the oracle, site after site
        yA, eA = _site_ref(iA, K, xA.cpu().numpy(), N.PRO_RMSNORM_DYNQ8, S.RS_F, p0,
                           nwA.cpu().numpy())
        refA = law.movy(yA, p0 - eA, law.MOVY_INT16)
        yB, eB = _site_ref(iB, K, np.asarray(refA, np.int16), N.PRO_DYNQ8, S.RS_F, p0)
        refB = law.movy(yB, p0 - eB, law.MOVY_INT16)
        yC, eC = _site_ref(iC, 1024, xC_host, N.PRO_DYNQ8, S.RS_F, p0)
        refC = law.movy(yC, p0 - eC, law.MOVY_INT16)
        yD, eD = _site_ref(iD, K, xD.cpu().numpy(), N.PRO_DYNQ8, S.RS_F, p0)
        refD = law.movy(yD, p0 - eD, law.MOVY_INT16)
        yH, _ = _site_ref(iH, 2048, np.asarray(refB, np.int16), N.PRO_DYNQ8, 0, 0)
        refH = law.amax32(yH)

        assert np.array_equal(outA.cpu().numpy().astype(np.int64), np.asarray(refA, np.int64))
        assert np.array_equal(outB.cpu().numpy().astype(np.int64), np.asarray(refB, np.int64))
        assert np.array_equal(outC.cpu().numpy().astype(np.int64), np.asarray(refC, np.int64))
        assert np.array_equal(xC.cpu().numpy().astype(np.int64), np.asarray(refD, np.int64))
        assert tuple(res.cpu().numpy().tolist()) == tuple(int(v) for v in refH)
    finally:
        plan.close()
        for w in (wA, wB, wC, wD, wH):
            w.free()


@pytest.mark.parametrize("kb,pro", [(128, N.PRO_RMSNORM_DYNQ8), (256, N.PRO_DYNQ8),
                                    (640, N.PRO_DYNQ8), (1152, N.PRO_DYNQ8),
                                    (2048, N.PRO_RMSNORM_DYNQ8), (4224, N.PRO_DYNQ8),
                                    (5248, N.PRO_DYNQ8)])
@pytest.mark.parametrize("mode", [N.PLAN_PERSISTENT, N.PLAN_PERSISTENT_COOP])
@pytest.mark.parametrize("gap", [False, True])
def test_stamped_sites_any_k(engine, kb, pro, mode, gap):
    """Sites reading an earlier site's output through stamped words when
    that output (the reader's K) does not fill the prologue's 512-element
    chunks: A (kb rows) -> B (K = kb) -> LM head (K = 256), each waiting for
    the words of the one before, bit-exact against the oracle.  Reading the
    site just before it, a site's prologue is shared with the control
    wavefront (four wavefronts); with `gap`, an independent site C sits
    between A and B, and B's prologue runs on the three prologue wavefronts
    alone.  K = 4224 takes the three-chunk prologue past K = 4096 (the
    control wavefront's share stops there), its ninth chunk a quarter full;
    K = 5248 the eight-chunk prologue with its chunks past K skipped."""
    from fable5_llm_amd.engine import Plan
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(kb)
    I16 = N.EPI_MOVY_I16

    def mat(nrows, k):
        img = S.synth_image(gen, nrows, k, S.CHAIN_LOG2_LO)
        torch.cuda.synchronize()
        return engine.upload(img, nrows, k, S.sh_for_k(k)), img.cpu().numpy()

    def ref(img, nrows, k, x16, prologue, norm_w=None):
        x = x16
        if prologue == N.PRO_RMSNORM_DYNQ8:
            x = law.rmsnorm_fx(x16, norm_w, S.RS_F, True)
        x8, e = law.dyn_quant_i8(x)
        return cfast.matvec_y32_img(img, nrows, k, S.sh_for_k(k), x8, 0), e

    wA, iA = mat(kb, K)
    xA = S.synth_x16(gen, K, S.RS_F)
    outA = torch.full((kb,), 0x5A5A, dtype=torch.int16, device=dev)
    wB, iB = mat(256, kb)
    nwB = S.synth_norm_w(gen, kb, True) if pro == N.PRO_RMSNORM_DYNQ8 else None
    outB = torch.full((256,), 0x5A5A, dtype=torch.int16, device=dev)
    wH, iH = mat(512, 256)
    wC, iC = mat(256, 256)
    xC = S.synth_x16(gen, 256, S.RS_F)
    outC = torch.full((256,), 0x5A5A, dtype=torch.int16, device=dev)
    res = torch.zeros(2, dtype=torch.int32, device=dev)
    p0A = 15 - S.E_SCALE - S.sh_for_k(K)
    p0B = 15 - S.E_SCALE - S.sh_for_k(kb)
    p0C = 15 - S.E_SCALE - S.sh_for_k(256)
    plan = Plan(engine)
    plan.add_site([wA], [I16], [p0A], [outA], xA, prologue=N.PRO_DYNQ8, in_f=S.RS_F)
    if gap:
        plan.add_site([wC], [I16], [p0C], [outC], xC, prologue=N.PRO_DYNQ8, in_f=S.RS_F)
    plan.add_site([wB], [I16], [p0B], [outB], outA, prologue=pro, norm_w=nwB, in_f=S.RS_F,
                  one_plus=True)
    plan.add_head(wH, outB, res, prologue=N.PRO_DYNQ8)
    try:
        plan.set_mode(mode)
        plan.set_fences(N.FENCE_AUTO)
        torch.cuda.synchronize()
        yA, eA = ref(iA, kb, K, xA.cpu().numpy(), N.PRO_DYNQ8)
        refA = law.movy(yA, p0A - eA, law.MOVY_INT16)
        yB, eB = ref(iB, 256, kb, np.asarray(refA, np.int16), pro,
                     None if nwB is None else nwB.cpu().numpy())
        refB = law.movy(yB, p0B - eB, law.MOVY_INT16)
        yH, _ = ref(iH, 512, 256, np.asarray(refB, np.int16), N.PRO_DYNQ8)
        refH = tuple(int(v) for v in law.amax32(yH))
        yC, eC = ref(iC, 256, 256, xC.cpu().numpy(), N.PRO_DYNQ8)
        refC = law.movy(yC, p0C - eC, law.MOVY_INT16)
        for rep in range(2):
            outA.fill_(0x5A5A)
            outB.fill_(0x5A5A)
            outC.fill_(0x5A5A)
            res.zero_()
            torch.cuda.synchronize()
            plan.run()
            engine.sync()
            assert np.array_equal(outA.cpu().numpy().astype(np.int64),
                                  np.asarray(refA, np.int64)), rep
            assert np.array_equal(outB.cpu().numpy().astype(np.int64),
                                  np.asarray(refB, np.int64)), rep
            if gap:
                assert np.array_equal(outC.cpu().numpy().astype(np.int64),
                                      np.asarray(refC, np.int64)), rep
            assert tuple(res.cpu().numpy().tolist()) == refH, rep
    finally:
        plan.close()
        for w in (wA, wB, wC, wH):
            w.free()
