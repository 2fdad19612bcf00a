"""Record streams for the .seq matvec tests, built with the product's own
encoder (fable5_llm_amd.seq) from the fixtures' V records."""
import numpy as np

from fable5_llm_amd import seq as S


def alu_p0(cmd):
    """p0 of a layer-command ALU record (the committed scripts' ARG layout):
    low 16 bits of ARG2 with bit 18 of ARG0 as bit 16, sign-extended."""
    a0, a2 = int(cmd[1]), int(cmd[3])
    p0 = (a2 & 0xFFFF) | (((a0 >> 18) & 1) << 16)
    return p0 - (1 << 17) if p0 >= (1 << 16) else p0


def xrf_write(i, v):
    return S.Rec(S.OP_CSRWR, target=S.CSR_SPACE_SEQ | (S.SOFF_XRF0 + 4 * i), imm32=v)


def movx(chan, word, addr, n):
    return S.Rec(S.OP_MOVX, flags=chan << 4, target=word, addr_lo=addr, len_or_addr_hi=n)


def mvgo(chan, wbase, ng, nrows, sh, stride, xbank=0, rbank=0, nowait=False):
    return S.Rec(S.OP_MVGO, flags=chan << 4, target=1 if nowait else 0,
                 imm32=S.shape_word(ng, nrows, sh, xbank, rbank), addr_lo=wbase & 0xFFFFFFFF,
                 len_or_addr_hi=((nrows * stride // 64) << 8) | (wbase >> 32))


def movy(chan, row0, n, addr, imm=0, int16=False, ind=S.IND_NONE, xrf=0):
    return S.Rec(S.OP_MOVY, flags=(S.MOVY_MODE_BIT if int16 else 0) | ind | (xrf << 5),
                 target=(row0 << 4) | chan, imm32=imm & 0xFFFFFFFF, addr_lo=addr,
                 len_or_addr_hi=n)


X_ADDR, PAIRS_ADDR, I16_ADDR = 0, 8192, 24576


def v_record_stream(scripts, tag, v, entries, plan):
    """One fixture V record as MOVX -> MVGO -> MOVY pairs32 (shift 0) ->
    MOVY int16 through IND_SUB XRF[0] = e_x (imm32 = p0 + e_x, p0 of the
    ALU command after the record, when it has one).  Returns (x8 words to
    stage at X_ADDR, records, y32 the generator asserted, p0 or None)."""
    wid, nin, _nr, e_x = (int(x) for x in scripts[f"{tag}_v{v}_hdr"])
    x8 = scripts[f"{tag}_v{v}_x8"].astype(np.int16)
    y = scripts[f"{tag}_v{v}_y32"].astype(np.int64)
    e = entries[str(wid)]
    nrows, k, sh, stride = int(e["nrows"]), int(e["k"]), int(e["sh"]), int(e["stride"])
    key = f"{tag}_v{v}_cmd"
    p0 = alu_p0(scripts[key]) if key in scripts.files else None
    recs = [xrf_write(S.XRF_EX, e_x), movx(0, 0, X_ADDR, nin),
            mvgo(0, plan[wid], k // 128, nrows, sh, stride),
            movy(0, 0, nrows, PAIRS_ADDR)]
    if p0 is not None:
        recs.append(movy(0, 0, nrows, I16_ADDR, imm=p0 + e_x, int16=True, ind=S.IND_SUB))
    recs.append(S.Rec(S.OP_HALT))
    return x8, recs, y, p0


def script_stream(scripts, tag, entries, plan):
    """All V records of one script as ONE stream: records in groups of 4 on
    channels 0..3 (x bank alternating by group), each group's MVGOs no-wait,
    then a FENCE, then each record's MOVY pairs32 (shift 0) and, where the
    record has its ALU command, MOVY int16 through IND_SUB XRF[0].
    Returns (stage [(addr, words)], records, checks [(kind, addr, y32, p0)],
    scratch words needed)."""
    nv = int(scripts[f"{tag}_counts"][0])
    stage, recs, checks = [], [], []
    addr = 0
    for g0 in range(0, nv, 4):
        group = list(range(g0, min(nv, g0 + 4)))
        xbank = (g0 // 4) & 1
        meta = []
        for i, v in enumerate(group):
            wid, nin, _nr, e_x = (int(x) for x in scripts[f"{tag}_v{v}_hdr"])
            x8 = scripts[f"{tag}_v{v}_x8"].astype(np.int16)
            e = entries[str(wid)]
            stage.append((addr, x8))
            recs.append(movx(i, S.XBANK_WORD * xbank, addr, nin))
            addr += nin
            recs.append(mvgo(i, plan[wid], int(e["k"]) // 128, int(e["nrows"]), int(e["sh"]),
                             int(e["stride"]), xbank=xbank, nowait=True))
            meta.append((v, i, int(e["nrows"]), e_x))
        recs.append(S.Rec(S.OP_FENCE))
        for v, ch, nrows, e_x in meta:
            y = scripts[f"{tag}_v{v}_y32"].astype(np.int64)
            addr += addr & 1
            recs.append(movy(ch, 0, nrows, addr))
            checks.append(("pairs", addr, y, None))
            addr += 2 * nrows
            key = f"{tag}_v{v}_cmd"
            if key in scripts.files:
                p0 = alu_p0(scripts[key])
                recs.append(xrf_write(S.XRF_EX, e_x))
                recs.append(movy(ch, 0, nrows, addr, imm=p0 + e_x, int16=True, ind=S.IND_SUB))
                checks.append(("int16", addr, y, p0))
                addr += nrows
    recs.append(S.Rec(S.OP_HALT))
    return stage, recs, checks, addr


def swin_stage(addr, vals):
    """CSRWR SPTR = addr, then one CSRWR SWIN per 16-bit word."""
    out = [S.Rec(S.OP_CSRWR, target=S.CSR_SPACE_LAYER | S.LOFF_SPTR, imm32=addr)]
    out += [S.Rec(S.OP_CSRWR, target=S.CSR_SPACE_LAYER | S.LOFF_SWIN, imm32=int(v) & 0xFFFF)
            for v in vals]
    return out
