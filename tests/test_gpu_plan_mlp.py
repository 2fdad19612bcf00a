"""A decoder layer's FFN block inside a plan (w4a8_plan_add_mlp and the
two sites it is made of): RMSNorm -> DYNQ8 -> gate SILU32 / up SHIFT32W,
then EMUL32 -> DYNQ8 -> down SHIFT32 -> residual ADD
(ref/layer_fixed.py:1597-1604, gen_layer_script.py:2166-2190, 1399-1400),
for several layers, in graph mode and as one persistent launch.

Layers are independent (each its own input) or chained through the
residual stream (layer l + 1 reads layer l's res_out, which the persistent
plan hands over through res_out's stamped words), with each layer's down
site right after its gate and up site or after the next layer's.  Every
layer's block output and residual are checked against the oracle's mlp_fx,
twice, with every output overwritten before each run."""
import numpy as np
import pytest
import torch

from fable5_llm_amd import _native as N
from fable5_llm_amd.engine import Plan
from oracle import law
from tests.helpers import activation_x16, norm_weight_q14
from tests.test_gpu_mlp import E_SCALE, _mats, _oracle_mlp, _upload

pytestmark = pytest.mark.gpu

RS_F = 7
MODES = [(N.PLAN_GRAPH, N.FENCE_ALL), (N.PLAN_PERSISTENT, N.FENCE_AUTO),
         (N.PLAN_PERSISTENT, N.FENCE_ALL)]


class Layers:
    def __init__(self, engine, H, FFN, nl, seed):
        rng = np.random.default_rng(seed)
        self.engine, self.H, self.FFN, self.nl = engine, H, FFN, nl
        self.dev = torch.device("cuda", 0)
        self.q, self.imgs, self.ws, self.nw, self.p0s = [], [], [], [], []
        for _ in range(nl):
            q = _mats(rng, H, FFN)
            ws, imgs = {}, {}
            for k, v in q.items():
                ws[k], imgs[k] = _upload(engine, v)
            self.q.append(q)
            self.imgs.append(imgs)
            self.ws.append(ws)
            self.nw.append(norm_weight_q14(rng, H))
            self.p0s.append([(15 - E_SCALE - q[k][3]) + RS_F - out_f
                             for k, out_f in (("gate", 12), ("up", RS_F), ("down", RS_F))])
        self.x16 = [activation_x16(rng, H, RS_F) for _ in range(nl)]

    def free(self):
        for ws in self.ws:
            for w in ws.values():
                w.free()

    def reference(self, chained):
        ys, rs = [], []
        x = self.x16[0]
        for l in range(self.nl):
            if not chained:
                x = self.x16[l]
            xn = law.rmsnorm_fx(x, self.nw[l], RS_F, True)
            y = _oracle_mlp(self.q[l], self.imgs[l], xn, RS_F)
            r = law.clip16(x.astype(np.int64) + y)
            ys.append(y)
            rs.append(r)
            x = r.astype(np.int16)
        return ys, rs

    def plan(self, chained, interleave, mode, fences):
        """(plan, inputs, mlp outputs, residual outputs)"""
        d = self.dev
        xs = [torch.from_numpy(self.x16[l].copy()).to(d) for l in range(self.nl)]
        ys = [torch.zeros(self.H, dtype=torch.int16, device=d) for _ in range(self.nl)]
        rs = [torch.zeros(self.H, dtype=torch.int16, device=d) for _ in range(self.nl)]
        nws = [torch.from_numpy(w).to(d) for w in self.nw]
        ins = [xs[0]] + ([rs[l - 1] for l in range(1, self.nl)] if chained else xs[1:])
        plan = Plan(self.engine)
        if not interleave:
            for l in range(self.nl):
                w = self.ws[l]
                plan.add_mlp(w["gate"], w["up"], w["down"], self.p0s[l], ins[l], norm_w=nws[l],
                             in_f=RS_F, one_plus=True, mlp_out=ys[l], res_out=rs[l])
        else:
            tmp = [(torch.zeros(self.FFN, dtype=torch.int16, device=d),
                    torch.zeros(self.FFN, dtype=torch.int32, device=d)) for _ in range(self.nl)]

            def up(l):
                w = self.ws[l]
                plan.add_site([w["gate"], w["up"]], [N.EPI_SILU32, N.EPI_MOVY_P32],
                              self.p0s[l][:2], list(tmp[l]), ins[l],
                              prologue=N.PRO_RMSNORM_DYNQ8, norm_w=nws[l], in_f=RS_F,
                              one_plus=True)

            def down(l):
                plan.add_site_emul_res(self.ws[l]["down"], self.p0s[l][2], tmp[l][0], tmp[l][1],
                                       ins[l], rs[l], out=ys[l])
            up(0)
            for l in range(1, self.nl):
                up(l)
                down(l - 1)
            down(self.nl - 1)
            plan._keep.append(tmp)
        plan.set_mode(mode)
        plan.set_fences(fences)
        torch.cuda.synchronize()
        return plan, ys, rs


@pytest.mark.parametrize("H,FFN,nl", [(1024, 3584, 5), (4096, 12288, 3)])
@pytest.mark.parametrize("chained", [False, True])
def test_plan_mlp_blocks(engine, H, FFN, nl, chained):
    L = Layers(engine, H, FFN, nl, seed=H + nl + 7 * chained)
    try:
        want_y, want_r = L.reference(chained)
        orders = [False] if chained else [False, True]   # a chain cannot interleave layers
        for interleave in orders:
            for mode, fences in MODES:
                plan, ys, rs = L.plan(chained, interleave, mode, fences)
                try:
                    if mode == N.PLAN_PERSISTENT and fences == N.FENCE_AUTO and not interleave:
                        f = plan.fenced()
                        paired = (FFN // 16) % engine.grid == 0
                        # layer l: the gate / up site, then the down site
                        for l in range(nl):
                            g, dn = f[2 * l], f[2 * l + 1]
                            assert g == (N.WAIT_INPUT if chained and l > 0 else N.WAIT_NONE), f
                            if chained and l > 0:
                                assert dn == N.WAIT_GRID, f   # its res is the last residual
                            else:
                                assert dn == (N.WAIT_INPUT if paired else N.WAIT_GRID), f
                    for rep in range(2):
                        for t in ys + rs:
                            t.fill_(-1)
                        torch.cuda.synchronize()
                        plan.run()
                        engine.sync()
                        for l in range(nl):
                            what = (mode, fences, interleave, rep, l)
                            assert np.array_equal(ys[l].cpu().numpy().astype(np.int64),
                                                  want_y[l]), what
                            assert np.array_equal(rs[l].cpu().numpy().astype(np.int64),
                                                  want_r[l]), what
                finally:
                    plan.close()
    finally:
        L.free()
