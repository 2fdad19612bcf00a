"""The SwiGLU FFN block on the device (w4a8_mlp_async): RMSNorm -> DYNQ8 ->
gate (SILU32) / up (SHIFT32W) -> EMUL32 -> DYNQ8 -> down (SHIFT32) ->
residual ADD, against the oracle's mlp_fx (ref/layer_fixed.py:1597-1604)
and the reference scripts' own gate / up / down records."""
import numpy as np
import pytest
import torch

from fable5_llm_amd import _native as N
from fable5_llm_amd import layer_fixed as LF
from oracle import cfast, law
from oracle.fixtures import script_tags
from tests.helpers import activation_x16, norm_weight_q14, rand_w4_m

pytestmark = pytest.mark.gpu

E_SCALE = -3   # the scale exponent of m in [256, 16384] (log-uniform 2^-10 .. 2^-4)


def _alu_p0(cmd):
    a0, a2 = int(cmd[1]), int(cmd[3])
    p0 = (a2 & 0xFFFF) | (((a0 >> 18) & 1) << 16)
    return p0 - (1 << 17) if p0 >= (1 << 16) else p0


def test_swiglu_chain_from_scripts_on_device(engine, scripts):
    # the engine's ALU ops and DYNQ8 turn the scripts' full gate and up
    # outputs into exactly the down record's x8 and e_x
    for tag in script_tags():
        gv, uv, _ = (int(v) for v in scripts[f"{tag}_mlp_v"])
        sg = engine.alu(N.ALU_SILU32, scripts[f"{tag}_mlp_gate_y32"],
                        _alu_p0(scripts[f"{tag}_v{gv}_cmd"]))
        u = engine.alu(N.ALU_SHIFT32W, scripts[f"{tag}_mlp_up_y32"],
                       _alu_p0(scripts[f"{tag}_v{uv}_cmd"]))
        prod = engine.alu(N.ALU_EMUL32, u, 12, b=sg)
        x8, e = engine.dynq8(prod)
        assert np.array_equal(x8, scripts[f"{tag}_mlp_down_x8"]), tag
        assert e == int(scripts[f"{tag}_mlp_down_e"][0]), tag


def _mats(rng, H, FFN):
    out = {}
    for name, (n, k) in (("gate", (FFN, H)), ("up", (FFN, H)), ("down", (H, FFN))):
        w4, m = rand_w4_m(rng, n, k)
        out[name] = (w4, m, E_SCALE, law.sh_for_k(k))
    return out


def _upload(engine, q):
    w4, m, _e, sh = q
    img, _ = law.pack_ddr_rows(w4, m)
    return engine.upload(img, w4.shape[0], w4.shape[1], sh), img


def _oracle_mlp(q, imgs, xn16, rs_f):
    """The oracle's mlp_fx with its three matvec_y32 calls done by the C
    restatement (same law, oracle/law_c.c); the rest is law.py."""
    def mv_to(name, x16, out_f):
        w4, _m, e, sh = q[name]
        x8, e_x = law.dyn_quant_i8(x16)
        y = cfast.matvec_y32_img(imgs[name], w4.shape[0], w4.shape[1], sh, x8).astype(np.int64)
        s = law.shift_for(e, sh, e_x, rs_f, out_f)
        return law.rshift_round(y, s) if s >= 0 else y << np.int64(-s)
    g = mv_to("gate", xn16, 12)
    u = mv_to("up", xn16, rs_f)
    sg = law.clip16(np.array([law.silu_q(int(np.clip(v, -(1 << 20), (1 << 20) - 1)))
                              for v in g], dtype=np.int64))
    prod = law.clip16(law.rshift_round(sg * u, 12))
    return law.clip16(mv_to("down", prod, rs_f))


def test_oracle_mlp_helper_is_law_mlp_fx():
    # the C-backed helper above is law.mlp_fx on a shape numpy finishes fast
    rng = np.random.default_rng(5)
    q = _mats(rng, 256, 512)
    imgs = {k: law.pack_ddr_rows(v[0], v[1])[0] for k, v in q.items()}
    xn = activation_x16(rng, 256)
    ref = law.mlp_fx(xn, q["gate"], q["up"], q["down"], rs_f=7)
    assert np.array_equal(_oracle_mlp(q, imgs, xn, 7), ref)


@pytest.mark.parametrize("H,FFN,norm,inplace", [(256, 512, False, False),
                                                (1024, 3584, True, False),
                                                (4096, 12288, True, True)])
def test_mlp_async_matches_oracle(engine, H, FFN, norm, inplace):
    rng = np.random.default_rng(H + FFN)
    q = _mats(rng, H, FFN)
    ws, imgs = {}, {}
    for k, v in q.items():
        ws[k], imgs[k] = _upload(engine, v)
    rs_f = 7
    x16 = activation_x16(rng, H, rs_f)
    nw = norm_weight_q14(rng, H) if norm else None
    p0s = [(15 - E_SCALE - q[k][3]) + rs_f - out_f
           for k, out_f in (("gate", 12), ("up", rs_f), ("down", rs_f))]
    dev = torch.device("cuda", 0)
    xd = torch.from_numpy(x16.copy()).to(dev)
    nwd = None if nw is None else torch.from_numpy(nw).to(dev)
    yd = torch.full((H,), 0x5A5A, dtype=torch.int16, device=dev)
    rd = xd if inplace else torch.zeros(H, dtype=torch.int16, device=dev)
    torch.cuda.synchronize()
    try:
        engine.mlp_async(ws["gate"], ws["up"], ws["down"], p0s, xd, norm_w=nwd,
                         in_f=rs_f, one_plus=True, mlp_out=yd, res_out=rd)
        engine.sync()
        xn = law.rmsnorm_fx(x16, nw, rs_f, True) if norm else x16
        ref_y = _oracle_mlp(q, imgs, xn, rs_f)
        assert np.array_equal(yd.cpu().numpy().astype(np.int64), ref_y)
        ref_r = law.clip16(x16.astype(np.int64) + ref_y)
        assert np.array_equal(rd.cpu().numpy().astype(np.int64), ref_r)
    finally:
        for w in ws.values():
            w.free()


def test_mlp_fx_dropin_matches_oracle(engine):
    rng = np.random.default_rng(9)
    q = _mats(rng, 512, 1024)
    qm = {k: {"w4": v[0], "m": v[1], "e": v[2], "sh": v[3]} for k, v in q.items()}
    xn = activation_x16(rng, 512)
    got = LF.mlp_fx(xn, qm, rs_f=7)
    assert np.array_equal(got, law.mlp_fx(xn, q["gate"], q["up"], q["down"], rs_f=7))
    for v in qm.values():
        v["dev"].free()


@pytest.mark.parametrize("e_up,live", [(11, False), (19, True)])
def test_mlp_fx_left_shifted_up_matches_oracle(engine, e_up, live):
    # the up projection's scale exponent makes its shift p0 - e_x negative
    # (K = 512: sh = 4, p0 = 15 - e - sh = 0 at e = 11, -8 at e = 19; e_x = 5
    # for these inputs), so u = y32 << s; at e = 19 it leaves int32 for
    # some rows: the engine's SHIFT32W clip must give the product of the
    # unclipped int64 u (layer_fixed.py:1597-1604) exactly
    rng = np.random.default_rng(40 + e_up)
    q = _mats(rng, 512, 1024)
    w4, m, _e, sh = q["up"]
    q["up"] = (w4, m, e_up, sh)
    qm = {k: {"w4": v[0], "m": v[1], "e": v[2], "sh": v[3]} for k, v in q.items()}
    xn = activation_x16(rng, 512)
    try:
        got = LF.mlp_fx(xn, qm, rs_f=7)
        ref = law.mlp_fx(xn, q["gate"], q["up"], q["down"], rs_f=7)
        assert np.array_equal(got, ref)
        # the case is live: some up values left int32 before the product
        x8, e_x = law.dyn_quant_i8(xn)
        y = law.matvec_y32(w4, m, sh, x8).astype(np.int64)
        s = law.shift_for(e_up, sh, e_x, 7, 7)
        assert s < 0
        assert (np.abs(y << np.int64(-s)).max() >= 2 ** 31) == live
    finally:
        for v in qm.values():
            if "dev" in v:
                v["dev"].free()


def test_mlp_fx_refuses_wrapping_shifts(engine):
    # a left shift of more than 17 bits on the up projection is where the
    # reference's int64 product could wrap: refused before any device work
    rng = np.random.default_rng(3)
    q = _mats(rng, 256, 512)
    qm = {k: {"w4": v[0], "m": v[1], "e": v[2], "sh": v[3]} for k, v in q.items()}
    qm["up"]["e"] = 24   # p0 = 15 - 24 - 3 = -12: up to 21 bits left
    with pytest.raises(AssertionError, match="up projection"):
        LF.mlp_fx(activation_x16(rng, 256), qm, rs_f=7)
    assert all("dev" not in v for v in qm.values())


def test_mlp_async_rejects_mismatched_shapes(engine):
    rng = np.random.default_rng(2)
    q = _mats(rng, 256, 512)
    ws = {k: _upload(engine, v)[0] for k, v in q.items()}
    x = torch.zeros(256, dtype=torch.int16, device="cuda")
    try:
        with pytest.raises(ValueError, match="FFN x H"):
            engine.mlp_async(ws["gate"], ws["down"], ws["down"], [0, 0, 0], x)
    finally:
        for w in ws.values():
            w.free()


def test_mlp_async_residual_only_and_no_output(engine):
    # d_mlp_out null: only the residual sum is written; both null is refused
    rng = np.random.default_rng(12)
    H, FFN = 512, 1536
    q = _mats(rng, H, FFN)
    ws, imgs = {}, {}
    for k, v in q.items():
        ws[k], imgs[k] = _upload(engine, v)
    rs_f = 7
    x16 = activation_x16(rng, H, rs_f)
    p0s = [(15 - E_SCALE - q[k][3]) + rs_f - out_f
           for k, out_f in (("gate", 12), ("up", rs_f), ("down", rs_f))]
    dev = torch.device("cuda", 0)
    xd = torch.from_numpy(x16.copy()).to(dev)
    rd = torch.full((H,), 0x1234, dtype=torch.int16, device=dev)
    torch.cuda.synchronize()
    try:
        engine.mlp_async(ws["gate"], ws["up"], ws["down"], p0s, xd, in_f=rs_f,
                         mlp_out=None, res_out=rd)
        engine.sync()
        ref_y = _oracle_mlp(q, imgs, x16, rs_f)
        ref_r = law.clip16(x16.astype(np.int64) + ref_y)
        assert np.array_equal(rd.cpu().numpy().astype(np.int64), ref_r)
        with pytest.raises(ValueError, match="no output"):
            engine.mlp_async(ws["gate"], ws["up"], ws["down"], p0s, xd, in_f=rs_f,
                             mlp_out=None, res_out=None)
    finally:
        for w in ws.values():
            w.free()
