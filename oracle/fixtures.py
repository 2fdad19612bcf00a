"""Loaders for the committed golden fixtures (tests/golden/*.npz) --
TEST INFRASTRUCTURE.  The fixtures hold the reference's own golden vectors;
tests/golden/make_fixtures.py documents where each one comes from."""
import numpy as np

from . import law


def vec_case(d, s):
    """tb/vec_s<s>: (K, NG, SH, N, image bytes, x8, y32)."""
    K, NG, SH, N, BPR = (int(v) for v in d[f"vec{s}_params"])
    return dict(K=K, NG=NG, SH=SH, N=N, BPR=BPR, img=d[f"vec{s}_img"].tobytes(),
                x8=d[f"vec{s}_x8"], y32=d[f"vec{s}_y32"])


def script_tags():
    return [f"{k}{s}" for k in ("layer", "token") for s in range(1, 5)]


def script_records(d, tag):
    """Yield dicts for every V record of one script: the weight-image row
    subset, its metadata, x8, e_x and the golden y32 of those rows."""
    nv = int(d[f"{tag}_counts"][0])
    for v in range(nv):
        wid, nin, nr, ex = (int(x) for x in d[f"{tag}_v{v}_hdr"])
        nrows, k, ng, sh, e, stride = (int(x) for x in d[f"{tag}_w{wid}_meta"])
        assert nrows == nr and k == nin and stride == law.row_stride(k)
        rows = d[f"{tag}_w{wid}_rows"]
        rec = dict(tag=tag, v=v, wid=wid, K=k, NG=ng, sh=sh, e=e, e_x=ex,
                   nrows=nr, rows=rows, img=d[f"{tag}_w{wid}_img"].tobytes(),
                   x8=d[f"{tag}_v{v}_x8"], y32=d[f"{tag}_v{v}_y32"])
        key = f"{tag}_v{v}_cmd"
        rec["cmd"] = d[key] if key in d else None
        yield rec


def script_argmax(d, tag):
    """Yield (idx, val, full head y32) for every A record of one script."""
    na = int(d[f"{tag}_counts"][1])
    for a in range(na):
        idx, val = (int(x) for x in d[f"{tag}_a{a}"])
        yield idx, val, d[f"{tag}_a{a}_y32"]
