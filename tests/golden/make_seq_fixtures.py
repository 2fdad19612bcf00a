#!/usr/bin/env python3
"""Write tests/golden/seq_streams.npz: .seq record streams emitted by the
reference's own encoder (ref/seq_format.py SeqEmitter: `on_matvec`,
`on_w32`, `on_c` -> `_fuse` / `_mvgo` / `_movy` at 1607-1632, 1570-1607,
1852-1951, and the 4-channel `_emit_matvec_4chan` / `_emit_amax_matvec`
at 2077-2231), and the scratch and AMAX32 state the reference's own
executor (ref/seq_model.py SeqExec over DDRWeights.from_files) leaves after
running each of them.

Four synthetic matrices (int4 codes, full-range uint16 mantissas, sh by the
engine rule) are packed with the reference's `pack_ddr_rows`; each is fed to
the emitter the way the generator's .txt relays a matvec: V (on_matvec), then
per 2048-row chunk a W32 (on_w32) and the ALU command that consumes it
(on_c, ARG words from gen_layer_script's enc_alu_a0 / enc_a1 / enc_alu_a2):
  wid 0  4200 x 128   SHIFT32  (sub 1: fused MOVY int16 through XRF[0])
  wid 1  2100 x 256   SHIFT32W (sub 9: fused MOVY pairs32)
  wid 2   300 x 1024  SHIFT32
  wid 3  8200 x 128   AMAX32   (sub 10: the head; MOVY to the stage + CMD)
with a CSRWR of XRF[0] = e_x before each V (the e_x that MOVY's IND_SUB
takes back out).  Three streams: one channel with waiting MVGOs, one
channel with no-wait MVGOs (each followed by FENCE), and four channels
(contiguous quarters for the sub 1 / 9 matvecs, the interleaved 2048-row
chunks of the head).

Run in the development container only (it imports the reference checkout);
the committed npz is data: images, inputs, record bytes and expected state.
"""
import json
import os
import sys
import tempfile

import numpy as np

REF = "/root/reference/ref"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "seq_streams.npz")

# wid, nrows, K, ALU sub, x8 scratch address, dst scratch address
# (the reference machine's scratch is 16384 words)
MATS = [(0, 4200, 128, 1, 0, 5632),
        (1, 2100, 256, 9, 128, 9832),
        (2, 300, 1024, 1, 384, 14032),
        (3, 8200, 128, 10, 1408, 0)]
STAGE = 1536          # the W32 relay / AMAX32 stage (2048 pairs)
SCRATCH_HI = 14336    # words of scratch the streams touch
STREAMS = [("c1", 1, False), ("c1nw", 1, True), ("c4", 4, False)]
CHUNK = 2048          # the .txt dequant chunk (inject_dequant)


class _Gen:
    """What SeqEmitter reads of the generator: its live matrices and the
    e_x of the matvec being relayed."""

    def __init__(self, wids):
        self.wids = wids
        self.eout = 0


def main():
    sys.path.insert(0, REF)
    import seq_format as SF          # puts the reference's sw/ on the path
    import hwmap as HW
    import seq_model as SM
    import w4a8_ref as R
    from gen_layer_script import enc_a1, enc_alu_a0, enc_alu_a2

    rng = np.random.default_rng(8642)
    out = {}
    wids, mats = {}, {}
    for wid, nrows, k, sub, xa, dst in MATS:
        ng = k // 128
        sh = max(0, (ng * 65535 * (128 * 8 * 127)).bit_length() - 31)
        w4 = rng.integers(-8, 8, size=(nrows, k), dtype=np.int8)
        m = rng.integers(1, 65536, size=(nrows, ng), dtype=np.int64).astype(np.uint16)
        x8 = rng.integers(-127, 128, size=k, dtype=np.int8)
        e_x = int(rng.integers(1, 6))
        p0 = int(rng.integers(6, 13)) if sub != 10 else 1
        img, stride = R.pack_ddr_rows(w4, m, g=128)
        y = np.asarray(R.matvec_y32(w4, m, sh, x8, g=128), dtype=np.int64)
        wids[f"m{wid}"] = (wid, {"w4": w4, "m": m, "sh": sh, "g": 128})
        mats[wid] = dict(nrows=nrows, k=k, sub=sub, xa=xa, dst=dst, sh=sh, x8=x8,
                         e_x=e_x, p0=p0, y=y, stride=stride)
        out[f"w{wid}_img"] = np.frombuffer(img, dtype=np.uint8)
        out[f"w{wid}_meta"] = np.array([nrows, k, ng, sh, stride, sub, xa, dst, e_x, p0],
                                       dtype=np.int64)
        out[f"w{wid}_x8"] = x8
        out[f"w{wid}_y32"] = y

    with tempfile.TemporaryDirectory() as td:
        man = {}
        for wid, mt in mats.items():
            fn = f"sq_w{wid}.bin"
            with open(os.path.join(td, fn), "wb") as f:
                f.write(out[f"w{wid}_img"].tobytes())
            man[str(wid)] = {"file": fn, "nrows": mt["nrows"], "k": mt["k"],
                             "ng": mt["k"] // 128, "sh": mt["sh"], "e": -4,
                             "stride": mt["stride"],
                             "nbeats": mt["nrows"] * mt["stride"] // 64}
        with open(os.path.join(td, "sq.weights.json"), "w") as f:
            json.dump(man, f)

        for name, nch, nowait in STREAMS:
            gen = _Gen(wids)
            em = SF.SeqEmitter(gen, os.path.join(td, name), nch=nch, nowait_mvgo=nowait)
            for wid, mt in mats.items():
                gen.eout = mt["e_x"]
                em._csrwr(SF.csr_seq_xrf(SF.XRF_EX), mt["e_x"])
                em.on_matvec(wid, wids[f"m{wid}"][1], mt["xa"], mt["k"], mt["y"])
                for r0 in range(0, mt["nrows"], CHUNK):
                    n = min(CHUNK, mt["nrows"] - r0)
                    em.on_w32(STAGE, mt["y"][r0:r0 + n])
                    sub = mt["sub"]
                    if sub == 10:
                        fresh = 1 if r0 == 0 else 0
                        em.on_c(11, enc_alu_a0(10, n, fresh), enc_a1(STAGE),
                                enc_alu_a2(fresh, 0))
                    else:
                        off = 2 if sub == 9 else 1
                        em.on_c(11, enc_alu_a0(sub, n, mt["p0"]), enc_a1(STAGE),
                                enc_alu_a2(mt["p0"], mt["dst"] + off * r0))
            em._emit(SF.Rec(SF.OP_HALT))
            SF.validate_stream(em.recs)
            buf = SF.pack_stream(em.recs)
            plan = em.wplan
            W = SM.DDRWeights.from_files(os.path.join(td, "sq"), plan)
            ex = SM.SeqExec(buf, b"", W)
            for wid, mt in mats.items():
                ex.M.mem[mt["xa"]:mt["xa"] + mt["k"]] = mt["x8"].astype(np.int64)
            ex.run()
            out[f"{name}_rec"] = np.frombuffer(buf, dtype=np.uint8)
            out[f"{name}_plan"] = np.array(
                [[w, plan[w]["base"], plan[w]["nrows"], plan[w]["k"], plan[w]["ng"],
                  plan[w]["sh"], plan[w]["stride"]] for w in sorted(plan)], dtype=np.int64)
            out[f"{name}_mem"] = np.asarray(ex.M.mem[:SCRATCH_HI], dtype=np.int64)
            out[f"{name}_amax"] = np.array([ex.M.am_idx, ex.M.am_val], dtype=np.int64)
            out[f"{name}_stats"] = np.array(
                [em.stats[k] for k in ("movx", "mvgo", "mvgo_nowait", "fence", "cmd")],
                dtype=np.int64)
            print(name, len(em.recs), "records", dict(em.stats), "amax",
                  ex.M.am_idx, ex.M.am_val, file=sys.stderr)
    out["w_base"] = np.array([HW.W_BASE], dtype=np.int64)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays")


if __name__ == "__main__":
    main()
