"""Bounded waits that give up, and persistent launches captured in a graph.

Every wait of the persistent plan and of TOPK-32 is bounded.  With the
context's spin limit set to one poll (w4a8_ctx_set_spin_limit), a wait gives
up from the host's side while every kernel still runs to its end: the next
sync reports W4A8_E_HIP with the wait's message, and the next run on the
default limits is bit-exact again.  No test here makes a kernel fault or
hang.

A captured persistent launch (or TOPK-32 launch) replays one fixed epoch
with its own clearing of the flags; eager launches before the capture leave
higher flag values behind, so the first eager launch after a capture must
clear them again -- checked by eager runs, a capture, an eager run on a
changed input and replays, each against the oracle."""
import numpy as np
import pytest
import torch

from fable5_llm_amd import _native as N
from fable5_llm_amd import stream9b as S
from fable5_llm_amd.engine import Plan
from oracle import cfast, law

pytestmark = pytest.mark.gpu

K = 4096
SH = S.sh_for_k(K)
NSITES = 6


class Chain:
    """NSITES sites of 4096 x 4096, each reading the previous site's int16
    output (RMSNorm and DYNQ8 prologues alternating), on the device, with
    the oracle's run site after site."""

    def __init__(self, engine, independent=False):
        dev = torch.device("cuda", 0)
        gen = torch.Generator(device=dev)
        gen.manual_seed(31)
        self.engine, self.dev = engine, dev
        self.x0 = S.synth_x16(gen, K, S.RS_F)
        self.xs, self.ws, self.imgs, self.outs, self.nws = [], [], [], [], []
        self.plan = Plan(engine)
        m = S.Mat("chain", K, K, S.RS_F, N.EPI_MOVY_I16)
        self.p0 = m.p0(S.RS_F)
        for i in range(NSITES):
            img = S.synth_image(gen, K, K, S.CHAIN_LOG2_LO)
            torch.cuda.synchronize()
            self.ws.append(engine.upload(img, K, K, SH))
            self.imgs.append(img.cpu().numpy())
            rms = i % 2 == 0
            nw = S.synth_norm_w(gen, K, True) if rms else None
            if i == 0:
                x = self.x0
            else:
                x = S.synth_x16(gen, K, S.RS_F) if independent else self.outs[-1]
            out = torch.zeros(K, dtype=torch.int16, device=dev)
            self.plan.add_site([self.ws[-1]], [N.EPI_MOVY_I16], [self.p0], [out], x,
                               prologue=N.PRO_RMSNORM_DYNQ8 if rms else N.PRO_DYNQ8,
                               norm_w=nw, in_f=S.RS_F, one_plus=True)
            self.xs.append(x)
            self.nws.append(nw)
            self.outs.append(out)
        self.independent = independent
        torch.cuda.synchronize()

    def reference(self):
        """the oracle's outputs for the current inputs"""
        prev = None
        ref = []
        for i in range(NSITES):
            x = self.xs[i].cpu().numpy() if (self.independent or i == 0) else prev
            if self.nws[i] is not None:
                x = law.rmsnorm_fx(x, self.nws[i].cpu().numpy(), S.RS_F, True)
            x8, e = law.dyn_quant_i8(x)
            y = cfast.matvec_y32_img(self.imgs[i], K, K, SH, x8, 0)
            prev = np.asarray(law.movy(y, self.p0 - e, law.MOVY_INT16), np.int64).astype(np.int16)
            ref.append(prev)
        return ref

    def check(self, what):
        for i, (o, r) in enumerate(zip(self.outs, self.reference())):
            assert np.array_equal(o.cpu().numpy(), r), (what, i)

    def clear(self):
        for o in self.outs:
            o.fill_(-1)
        torch.cuda.synchronize()

    def close(self):
        self.plan.close()
        for w in self.ws:
            w.free()


@pytest.mark.parametrize("independent,fences,grid_polls,lds_polls,message", [
    (False, N.FENCE_AUTO, 1, 0, "wait for other workgroups timed out"),   # stamped words
    (False, N.FENCE_ALL, 1, 0, "wait for other workgroups timed out"),    # grid-wide flags
    (True, N.FENCE_AUTO, 1, 0, "wait for other workgroups timed out"),    # staged prologues
    (False, N.FENCE_AUTO, 0, 1, "a wait between wavefronts of one workgroup timed out"),
    (True, N.FENCE_AUTO, 0, 1, "a wait between wavefronts of one workgroup timed out"),
])
def test_plan_wait_gives_up(engine, independent, fences, grid_polls, lds_polls, message):
    ch = Chain(engine, independent)
    try:
        ch.plan.set_mode(N.PLAN_PERSISTENT)
        ch.plan.set_fences(fences)
        ch.plan.run()
        engine.sync()
        ch.check("before")
        engine.set_spin_limit(grid_polls, lds_polls)
        try:
            ch.clear()
            ch.plan.run()
            with pytest.raises(RuntimeError, match=message):
                engine.sync()
        finally:
            engine.set_spin_limit(0, 0)
        ch.clear()
        ch.plan.run()
        engine.sync()
        ch.check("after")
    finally:
        ch.close()


def test_topk_wait_gives_up(engine):
    nrows = 20000
    rng = np.random.default_rng(78)
    w4 = rng.integers(-8, 8, (nrows, K)).astype(np.int8)
    m = rng.integers(256, 16385, (nrows, K // 128)).astype(np.uint16)
    img, _ = law.pack_ddr_rows(w4, m)
    w = engine.upload(img, nrows, K, SH)
    dev = torch.device("cuda", 0)
    try:
        x16 = np.clip(np.rint(rng.normal(0, 1, K) * 128), -32768, 32767).astype(np.int16)
        x8, _ = law.dyn_quant_i8(x16)
        vals, rows, count, ovf = law.topk32(cfast.matvec_y32_img(img, nrows, K, SH, x8))
        ref = np.concatenate([vals, rows, [count, int(ovf)]]).astype(np.int32)
        xd = torch.from_numpy(x16).to(dev)
        out = torch.zeros(66, dtype=torch.int32, device=dev)
        engine.head_topk32_async(w, xd, out)
        engine.sync()
        assert np.array_equal(out.cpu().numpy(), ref)
        engine.set_spin_limit(1, 0)
        try:
            engine.head_topk32_async(w, xd, out)
            with pytest.raises(RuntimeError, match="TOPK-32's wait"):
                engine.sync()
        finally:
            engine.set_spin_limit(0, 0)
        out.zero_()
        torch.cuda.synchronize()
        engine.head_topk32_async(w, xd, out)
        engine.sync()
        assert np.array_equal(out.cpu().numpy(), ref)
    finally:
        w.free()


def test_persistent_plan_capture_after_eager_runs(engine):
    """Eager runs move the flags' epoch on; a capture replays epoch 1 with
    its own clear; the eager run after the capture clears again."""
    ch = Chain(engine)
    side = torch.cuda.Stream()
    try:
        ch.plan.set_mode(N.PLAN_PERSISTENT)
        ch.plan.set_fences(N.FENCE_AUTO)
        for _ in range(3):
            ch.clear()
            ch.plan.run()
            engine.sync()
        ch.check("eager")
        g = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(g, stream=side):
                engine.set_stream(side)
                ch.plan.run()
        finally:
            engine.set_stream(None)
        gen = torch.Generator(device=ch.dev)
        for k in range(3):
            gen.manual_seed(100 + k)
            ch.x0.copy_(S.synth_x16(gen, K, S.RS_F))   # a changed input
            ch.clear()
            ch.plan.run()                              # eager, after the capture
            engine.sync()
            ch.check(("eager after capture", k))
            ch.clear()
            g.replay()
            torch.cuda.synchronize()
            ch.check(("replay", k))
    finally:
        ch.close()


def test_topk_capture_after_eager_runs(engine):
    nrows = 20000
    rng = np.random.default_rng(79)
    w4 = rng.integers(-8, 8, (nrows, K)).astype(np.int8)
    m = rng.integers(256, 16385, (nrows, K // 128)).astype(np.uint16)
    img, _ = law.pack_ddr_rows(w4, m)
    w = engine.upload(img, nrows, K, SH)
    dev = torch.device("cuda", 0)
    side = torch.cuda.Stream()

    def ref_for(x16):
        x8, _ = law.dyn_quant_i8(x16)
        vals, rows, count, ovf = law.topk32(cfast.matvec_y32_img(img, nrows, K, SH, x8))
        return np.concatenate([vals, rows, [count, int(ovf)]]).astype(np.int32)
    try:
        x16 = np.clip(np.rint(rng.normal(0, 1, K) * 128), -32768, 32767).astype(np.int16)
        xd = torch.from_numpy(x16).to(dev)
        out = torch.zeros(66, dtype=torch.int32, device=dev)
        for _ in range(3):
            engine.head_topk32_async(w, xd, out)
        engine.sync()
        assert np.array_equal(out.cpu().numpy(), ref_for(x16))
        g = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(g, stream=side):
                engine.set_stream(side)
                engine.head_topk32_async(w, xd, out)
        finally:
            engine.set_stream(None)
        for k in range(3):
            x16 = np.clip(np.rint(rng.normal(0, 1, K) * 128), -32768, 32767).astype(np.int16)
            xd.copy_(torch.from_numpy(x16))
            out.zero_()
            torch.cuda.synchronize()
            engine.head_topk32_async(w, xd, out)       # eager, after the capture
            engine.sync()
            want = ref_for(x16)
            assert np.array_equal(out.cpu().numpy(), want), ("eager", k)
            out.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy(), want), ("replay", k)
    finally:
        w.free()
