"""The persistent plan's prologue arithmetic on adversarial inputs: RMSNorm
(mode 0 and 1, in_f at both ends of 0..40, rails, zeros, one outlier, full
int16 ranges of x and of the weights) and DYNQ8 (values on the rounding
boundaries of every exponent, -32768), each a site of its own.

Run as independent sites (each prologue computed once and staged), with
every site fenced (each CU computes every prologue itself) and in graph
mode; every site's x8, e_x, RMSNorm output and MOVY output is checked
bit-exactly against the oracle (layer_fixed.py:1242-1278,
fixedpoint.py:24-33)."""
import numpy as np
import pytest
import torch

from fable5_llm_amd import _native as N
from fable5_llm_amd.engine import Plan
from oracle import cfast, law

pytestmark = pytest.mark.gpu

K = 4096
NROWS = 64
SH = law.sh_for_k(K)
P0 = 11


def _cases(rng):
    """(name, prologue, x16, norm_w, in_f, one_plus)"""
    R, D = N.PRO_RMSNORM_DYNQ8, N.PRO_DYNQ8
    full = lambda: rng.integers(-32768, 32768, K).astype(np.int16)
    out = [
        ("rms_all_min_w_min", R, np.full(K, -32768, np.int16), np.full(K, -32768, np.int16), 0, True),
        ("rms_rails_w_max_inf40", R, np.where(np.arange(K) % 2, 32767, -32767).astype(np.int16),
         np.full(K, 32767, np.int16), 40, True),
        ("rms_one_outlier", R, np.where(np.arange(K) == 1234, 32767, 0).astype(np.int16),
         full(), 7, True),
        ("rms_zeros", R, np.zeros(K, np.int16), full(), 7, True),
        ("rms_full_mode0", R, full(), full(), int(rng.integers(0, 41)), True),
        ("rms_full_mode1", R, full(), full(), int(rng.integers(0, 41)), False),
        ("rms_small_mode1_inf40", R, rng.integers(-3, 4, K).astype(np.int16), full(), 40, False),
        ("rms_small_inf0", R, rng.integers(-2, 3, K).astype(np.int16), full(), 0, True),
        ("dq_min", D, np.full(K, -32768, np.int16), None, 0, True),
        ("dq_zeros", D, np.zeros(K, np.int16), None, 0, True),
        ("dq_full", D, full(), None, 0, True),
    ]
    # DYNQ8 on the rounding boundaries of each exponent e: values k * 2^e
    # and k * 2^e +- half (half - 1), with the largest magnitude that still
    # rounds to 127 at e; and the smallest that carries past 127 (e + 1)
    for e in range(1, 9):
        half = 1 << (e - 1)
        base = rng.integers(-126, 127, K) << e
        x = base + rng.choice([-half, half - 1, half, 0], K)
        x[0] = (127 << e) + half - 1      # rounds to 127: exponent e
        x[1] = -((127 << e) + half - 1)
        out.append((f"dq_boundary_e{e}", D, x.astype(np.int16), None, 0, True))
        y = x.copy()
        y[2] = (127 << e) + half          # rounds to 128: exponent e + 1
        out.append((f"dq_carry_e{e}", D, np.clip(y, -32768, 32767).astype(np.int16), None, 0,
                    True))
    return out


def _oracle(img, x16, prologue, nw, in_f, one_plus):
    x = x16
    xn = None
    if prologue == N.PRO_RMSNORM_DYNQ8:
        x = xn = law.rmsnorm_fx(x16, nw, in_f, one_plus)
    x8, e = law.dyn_quant_i8(x)
    y = cfast.matvec_y32_img(img, NROWS, K, SH, x8, 0)
    return xn, x8, e, law.movy(y, P0 - e, law.MOVY_INT16)


@pytest.mark.parametrize("mode,fences", [(N.PLAN_PERSISTENT, N.FENCE_AUTO),
                                         (N.PLAN_PERSISTENT, N.FENCE_ALL),
                                         (N.PLAN_GRAPH, N.FENCE_ALL)])
def test_plan_prologues_adversarial(engine, mode, fences):
    rng = np.random.default_rng(4242)
    dev = torch.device("cuda", 0)
    cases = _cases(rng)
    w4 = rng.integers(-8, 8, (NROWS, K)).astype(np.int8)
    m = rng.integers(256, 16385, (NROWS, K // 128)).astype(np.uint16)
    img, _ = law.pack_ddr_rows(w4, m)
    w = engine.upload(img, NROWS, K, SH)
    imgn = np.frombuffer(img, dtype=np.uint8)
    plan = Plan(engine)
    keep = []
    try:
        for name, pro, x16, nw, in_f, one_plus in cases:
            xd = torch.from_numpy(x16).to(dev)
            nwd = None if nw is None else torch.from_numpy(nw).to(dev)
            out = torch.full((NROWS,), 0x5A5A, dtype=torch.int16, device=dev)
            x8 = torch.zeros(K, dtype=torch.int8, device=dev)
            e_x = torch.full((1,), -99, dtype=torch.int32, device=dev)
            xn = torch.zeros(K, dtype=torch.int16, device=dev) if nw is not None else None
            plan.add_site([w], [N.EPI_MOVY_I16], [P0], [out], xd, prologue=pro, norm_w=nwd,
                          in_f=in_f, one_plus=one_plus, x8_out=x8, e_x_out=e_x, xn_out=xn)
            keep.append((name, pro, x16, nw, in_f, one_plus, out, x8, e_x, xn))
        plan.set_mode(mode)
        plan.set_fences(fences)
        torch.cuda.synchronize()
        for rep in range(2):
            plan.run()
            engine.sync()
            for name, pro, x16, nw, in_f, one_plus, out, x8, e_x, xn in keep:
                r_xn, r_x8, r_e, r_out = _oracle(imgn, x16, pro, nw, in_f, one_plus)
                assert int(e_x.item()) == r_e, (name, rep)
                assert np.array_equal(x8.cpu().numpy(), r_x8), (name, rep)
                if r_xn is not None:
                    assert np.array_equal(xn.cpu().numpy().astype(np.int64),
                                          np.asarray(r_xn, np.int64)), (name, rep)
                assert np.array_equal(out.cpu().numpy().astype(np.int64),
                                      np.asarray(r_out, np.int64)), (name, rep)
    finally:
        plan.close()
        w.free()
