"""Plans over shapes the decode stream does not have: K of 128, 384 and 1280
(a partial scale block, chunks of the prologue only partly filled), row
counts that are not multiples of 16, every epilogue (Y32, MOVY int16 and
pairs32, SILU32, SHIFT_I64), the X8, DYNQ8 and RMSNorm prologues with their
exports, sites reading a slice of an earlier output at a word offset
(stamped words), a write over an earlier site's input (a grid-wide fence)
and a 300-row LM head.  Run in graph mode and in both persistent modes with
every fence and with fences derived from the buffers, twice each, and
checked bit-exactly against the oracle run site after site."""
import numpy as np
import pytest
import torch

from fable5_llm_amd import _native as N
from fable5_llm_amd import stream9b as S
from oracle import cfast, law

pytestmark = pytest.mark.gpu

I16, P32, Y32, SILU, I64 = (N.EPI_MOVY_I16, N.EPI_MOVY_P32, N.EPI_Y32, N.EPI_SILU32,
                            N.EPI_SHIFT_I64)
MODES = [(N.PLAN_GRAPH, N.FENCE_ALL), (N.PLAN_PERSISTENT, N.FENCE_ALL),
         (N.PLAN_PERSISTENT, N.FENCE_AUTO), (N.PLAN_PERSISTENT_COOP, N.FENCE_AUTO)]


def _shift64(y, s):
    """EPI_SHIFT_I64: the MOVY shift without the clip (right by at most 63,
    left by at most 40, as law.movy)."""
    y = np.asarray(y, dtype=np.int64)
    if s >= 0:
        return law.rshift_round(y, min(s, 63))
    return y << np.int64(min(-s, 40))


def _epilogue(y, epi, shift):
    if epi == Y32:
        return np.asarray(y, np.int64)
    if epi == I16:
        return law.movy(y, shift, law.MOVY_INT16)
    if epi == P32:
        return law.movy(y, shift, law.MOVY_PAIRS32)
    if epi == SILU:
        return law.alu_silu32(y, shift)
    return _shift64(y, shift)


class _Case:
    """One plan and its oracle.  Buffers are named host arrays mirrored by
    device tensors; a site's x is (buffer, first element, K)."""

    def __init__(self, engine, seed):
        self.engine = engine
        self.dev = torch.device("cuda", 0)
        self.gen = torch.Generator(device=self.dev)
        self.gen.manual_seed(seed)
        self.bufs = {}
        self.sites = []
        self.weights = []

    def buf(self, name, t):
        self.bufs[name] = t
        return t

    def mat(self, nrows, K):
        img = S.synth_image(self.gen, nrows, K, S.CHAIN_LOG2_LO)
        torch.cuda.synchronize()
        w = self.engine.upload(img, nrows, K, S.sh_for_k(K))
        self.weights.append(w)
        return w, img.cpu().numpy()

    def site(self, K, x, prologue, jobs, e_x=0, norm=None, in_f=S.RS_F, exports=False):
        """jobs: (nrows, epilogue, output buffer, first row)"""
        mats = [self.mat(n, K) for n, _, _, _ in jobs]
        nw = S.synth_norm_w(self.gen, K, True) if norm else None
        ex = None
        if exports:
            ex = (torch.zeros(K, dtype=torch.int8, device=self.dev),
                  torch.full((1,), -99, dtype=torch.int32, device=self.dev),
                  torch.zeros(K, dtype=torch.int16, device=self.dev) if norm else None)
        self.sites.append(dict(K=K, x=x, pro=prologue, jobs=jobs, mats=mats, e_x=e_x, nw=nw,
                               in_f=in_f, ex=ex))

    def head(self, K, x, nrows):
        w = self.mat(nrows, K)
        res = torch.zeros(2, dtype=torch.int32, device=self.dev)
        self.sites.append(dict(K=K, x=x, head=True, mat=w, res=res))

    def _view(self, spec):
        name, first, n = spec
        return self.bufs[name][first:first + n]

    def build(self):
        from fable5_llm_amd.engine import Plan
        plan = Plan(self.engine)
        for st in self.sites:
            x = self._view(st["x"])
            if st.get("head"):
                plan.add_head(st["mat"][0], x, st["res"], prologue=N.PRO_DYNQ8)
                continue
            K = st["K"]
            sh = S.sh_for_k(K)
            p0 = 15 - S.E_SCALE - sh
            outs = [self.bufs[b][r0:r0 + n] for n, _, b, r0 in st["jobs"]]
            ex = st["ex"] or (None, None, None)
            plan.add_site([m[0] for m in st["mats"]], [e for _, e, _, _ in st["jobs"]],
                          [p0] * len(outs), outs, x, prologue=st["pro"], e_x=st["e_x"],
                          norm_w=st["nw"], in_f=st["in_f"], one_plus=True,
                          x8_out=ex[0], e_x_out=ex[1], xn_out=ex[2])
        return plan

    def oracle(self, host):
        """host: the buffers' initial contents; returns the final buffers,
        the exports of each site and the heads' results."""
        h = {k: v.copy() for k, v in host.items()}
        exports, heads = [], []
        for st in self.sites:
            name, first, n = st["x"]
            xv = h[name][first:first + n]
            if st.get("head"):
                x8, _ = law.dyn_quant_i8(np.asarray(xv, np.int16))
                m = st["mat"]
                y = cfast.matvec_y32_img(m[1], m[0].nrows, n, S.sh_for_k(n), x8, 0)
                heads.append(tuple(int(v) for v in law.amax32(y)))
                continue
            K = st["K"]
            xn = None
            if st["pro"] == N.PRO_X8:
                x8, e = np.asarray(xv, np.int8), st["e_x"]
            elif st["pro"] == N.PRO_RMSNORM_DYNQ8:
                xn = law.rmsnorm_fx(np.asarray(xv, np.int16), st["nw"].cpu().numpy(),
                                    st["in_f"], True)
                x8, e = law.dyn_quant_i8(xn)
            else:
                x8, e = law.dyn_quant_i8(np.asarray(xv, np.int16))
            exports.append((np.asarray(x8, np.int64), e,
                            None if xn is None else np.asarray(xn, np.int64)))
            sh = S.sh_for_k(K)
            p0 = 15 - S.E_SCALE - sh
            for (nrows, epi, b, r0), (w, img) in zip(st["jobs"], st["mats"]):
                y = cfast.matvec_y32_img(img, nrows, K, sh, x8, 0)
                h[b][r0:r0 + nrows] = _epilogue(y, epi, p0 - e)
        return h, exports, heads

    def close(self):
        for w in self.weights:
            w.free()


def _plan_a(engine):
    c = _Case(engine, 5150)
    g, dev = c.gen, c.dev
    c.buf("xa", S.synth_x16(g, 1280, S.RS_F))
    c.buf("x8b", torch.randint(-127, 128, (384,), dtype=torch.int8, device=dev, generator=g))
    c.buf("o0a", torch.zeros(200, dtype=torch.int16, device=dev))
    c.buf("o0b", torch.zeros(56, dtype=torch.int32, device=dev))
    c.buf("o1", torch.zeros(136, dtype=torch.int16, device=dev))
    c.buf("o2a", torch.zeros(64, dtype=torch.int64, device=dev))
    c.buf("o2b", torch.zeros(96, dtype=torch.int32, device=dev))
    c.buf("o3", torch.zeros(48, dtype=torch.int16, device=dev))
    # S0: X8 prologue at a given e_x; an int16 and a Y32 output
    c.site(384, ("x8b", 0, 384), N.PRO_X8, [(200, I16, "o0a", 0), (56, Y32, "o0b", 0)], e_x=4)
    # S1: reads S0's first 128 outputs (stamped words), 136 rows
    c.site(128, ("o0a", 0, 128), N.PRO_DYNQ8, [(136, I16, "o1", 0)], exports=True)
    # S2: RMSNorm over S1's rows 8..135 (x is 16-byte aligned: word offset 4);
    # SHIFT_I64 and pairs32
    c.site(128, ("o1", 8, 128), N.PRO_RMSNORM_DYNQ8, [(64, I64, "o2a", 0), (96, P32, "o2b", 0)],
           norm=True, exports=True)
    # S3: an independent input of K = 1280 (a partial scale block), SILU32
    c.site(1280, ("xa", 0, 1280), N.PRO_DYNQ8, [(48, SILU, "o3", 0)], exports=True)
    # S4: writes rows 512..767 of S3's input (write after read)
    c.site(384, ("xa", 0, 384), N.PRO_DYNQ8, [(256, I16, "xa", 512)])
    # LM head of 300 rows over S0's outputs 64..191 (word offset 32)
    c.head(128, ("o0a", 64, 128), 300)
    return c


@pytest.mark.parametrize("mode,fences", MODES)
def test_plan_shapes(engine, mode, fences):
    c = _plan_a(engine)
    plan = c.build()
    try:
        plan.set_mode(mode)
        plan.set_fences(fences)
        torch.cuda.synchronize()
        init = {k: v.clone() for k, v in c.bufs.items()}
        host0 = {k: v.cpu().numpy().astype(np.int64) for k, v in init.items()}
        want, exports, heads = c.oracle(host0)
        # the plan's activations must have a spread worth checking
        assert len(np.unique(want["o1"])) > 16 and len(np.unique(want["o3"])) > 8
        for rep in range(2):
            for k, v in c.bufs.items():
                v.copy_(init[k])
            torch.cuda.synchronize()
            plan.run()
            engine.sync()
            for k, v in c.bufs.items():
                assert np.array_equal(v.cpu().numpy().astype(np.int64), want[k]), (k, rep)
            ei = 0
            for st in c.sites:
                if st.get("head"):
                    assert tuple(st["res"].cpu().numpy().tolist()) == heads[0], rep
                    continue
                if st["ex"] is not None:
                    x8, e, xn = exports[ei]
                    assert np.array_equal(st["ex"][0].cpu().numpy().astype(np.int64), x8), (ei, rep)
                    assert int(st["ex"][1].item()) == e, (ei, rep)
                    if xn is not None:
                        assert np.array_equal(st["ex"][2].cpu().numpy().astype(np.int64), xn), \
                            (ei, rep)
                ei += 1
    finally:
        plan.close()
        c.close()
