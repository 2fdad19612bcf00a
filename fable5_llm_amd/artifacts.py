"""Generator artifacts on the MI355X engine, and replay of their scripts.

For each script prefix the reference's generators write
(gen_layer_script.py:1555-1670):

  <prefix>.weights.json  wid -> image record {file, nrows, k, ng, sh, e,
                         nbeats, stride[, g][, w8]}, plus artifact metadata
                         under non-wid keys (sw/hwmap.py:477-533)
  <prefix>_w<wid>.bin    the packed row image (w4a8_ref.pack_ddr_rows layout)
  <prefix>.emb.bin       the int16 embedding table, one row per token
  <prefix>.txt           the record script (gen_layer_script.py:648-702,
                         910, 1487-1545)

`Artifacts` memory-maps every image, checks its record against the wire
format's law, and uploads it to the device, where the engine repacks it
into its tile layout (the role of DDRWeights.from_files,
ref/seq_model.py:305-452, and of the host's upload loop,
sw/infer.py:735-760).  `replay` runs every V record's matvec and every A
record's argmax of a script on the device and compares them with the
values the generator asserted.

    python -m fable5_llm_amd.artifacts <prefix> [<prefix> ...]

prints one JSON summary per script and exits non-zero on any mismatch.
"""
import json
import os
import sys
from dataclasses import dataclass

import numpy as np

from .w4a8_ref import row_beats, row_stride

# Artifact-level keys of a manifest and their defaults (sw/hwmap.py:502-523):
# every other key is a wid.
META_DEFAULTS = {"emb_row_bytes": 8192, "rs_f": 8}
STATE_KEYS = ("state", "conv_images")
META_KEYS = tuple(META_DEFAULTS) + STATE_KEYS


def split_manifest(man):
    """(wid entries, meta): meta holds the artifact keys, with defaults
    (sw/hwmap.py:526-532 split_manifest)."""
    wids = {k: v for k, v in man.items() if k not in META_KEYS}
    meta = {k: int(man.get(k, d)) for k, d in META_DEFAULTS.items()}
    for k in STATE_KEYS:
        meta[k] = man.get(k)
    return wids, meta


def load_weights_manifest(prefix):
    """Read `<prefix>.weights.json` -> (wid entries, meta)."""
    with open(prefix + ".weights.json") as f:
        return split_manifest(json.load(f))


def check_entry(wid, ent, nbytes):
    """Validate one image record against the wire format and its file's
    size; returns (nrows, k, sh).  Raises AssertionError, as the reference's
    own checks do, for a record the law rejects, and ValueError for an image
    this engine does not serve (8-bit codes, g = 64)."""
    if ent.get("w8"):
        raise ValueError(f"wid {wid}: 8-bit weight images are not served by "
                         "the W4A8 engine")
    g = int(ent.get("g", 128))
    if g != 128:
        raise ValueError(f"wid {wid}: group size {g}; the engine serves g = 128")
    nrows, k, ng, sh = (int(ent[x]) for x in ("nrows", "k", "ng", "sh"))
    stride = int(ent["stride"])
    assert nrows >= 1, f"wid {wid}: nrows {nrows}"
    assert k % 128 == 0 and ng == k // 128, f"wid {wid}: k {k}, ng {ng}"
    assert stride == row_stride(k), \
        f"wid {wid}: stride {stride}, the law gives {row_stride(k)}"
    beats = nrows * sum(row_beats(k))
    assert int(ent["nbeats"]) == beats, \
        f"wid {wid}: nbeats {ent['nbeats']}, the law gives {beats}"
    assert 0 <= sh < 64, f"wid {wid}: sh {sh}"
    assert nbytes == nrows * stride, \
        f"wid {wid}: {ent['file']} holds {nbytes} B, the record says {nrows * stride}"
    return nrows, k, sh


class Artifacts:
    """One script prefix's weight images resident on the device (and its
    embedding table, when present).  `weights[wid]` are engine weight
    handles; `entries[wid]` the manifest records; `meta` the artifact keys.
    """

    def __init__(self, engine, prefix, wids=None):
        self.engine = engine
        self.prefix = prefix
        self.entries, self.meta = load_weights_manifest(prefix)
        self.weights = {}
        d = os.path.dirname(prefix)
        try:
            for key in sorted(self.entries, key=int):
                wid = int(key)
                if wids is not None and wid not in wids:
                    continue
                ent = self.entries[key]
                path = os.path.join(d, ent["file"])
                img = np.memmap(path, dtype=np.uint8, mode="r")
                nrows, k, sh = check_entry(wid, ent, img.size)
                self.weights[wid] = engine.upload(img, nrows, k, sh)
                del img
        except BaseException:
            self.free()
            raise
        self._emb = None

    def entry(self, wid):
        return self.entries[str(wid)]

    def embedding(self, width):
        """The embedding table as a device int16 tensor [tokens, width]
        (`<prefix>.emb.bin`, little-endian int16 rows of `width` values; a
        manifest's emb_row_bytes gives the width when it carries the key)."""
        import torch
        if self._emb is None or self._emb.shape[1] != width:
            raw = np.fromfile(self.prefix + ".emb.bin", dtype="<i2")
            assert width >= 1 and raw.size % width == 0, \
                f"{self.prefix}.emb.bin: {raw.size} values are not rows of {width}"
            dev = torch.device("cuda", self.engine.device)
            self._emb = torch.from_numpy(raw.reshape(-1, width)).to(dev)
        return self._emb

    def free(self):
        for w in self.weights.values():
            w.free()
        self.weights = {}
        self._emb = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.free()


# ------------------------------------------------------------ record scripts
@dataclass
class Record:
    kind: str
    fields: tuple     # header fields after the kind letter, as integers
    data: object      # the record's data words (int64 array) or None


# kind -> (header field holding the word count, bits per word); the other
# kinds carry their header only (gen_layer_script.py:648-702, 1487-1545)
_DATA = {"W": (1, 16), "R": (1, 16), "V": (3, 32)}


def _words(lines, bits):
    v = np.array([int(w, 16) for w in lines], dtype=np.int64)
    return np.where(v >= (1 << (bits - 1)), v - (1 << bits), v)


def parse_script(path):
    """Yield the script's records in order.  Header fields and data words
    are hex; data words are two's complement of 16 (W, R) or 32 (V) bits."""
    with open(path) as f:
        lines = f.read().split("\n")
    i, n = 0, len(lines)
    while i < n:
        t = lines[i].split()
        i += 1
        if not t:
            continue
        kind, fields = t[0], tuple(int(x, 16) for x in t[1:])
        data = None
        if kind in _DATA:
            at, bits = _DATA[kind]
            cnt = fields[at]
            assert i + cnt <= n, f"{path}: {kind} record runs past the end"
            data = _words(lines[i:i + cnt], bits)
            i += cnt
        yield Record(kind, fields, data)


def replay(art, script=None, log=None):
    """Run the script's V records (matvec of the staged x8 against image
    wid) and A records (AMAX32 of the last V record's rows) on the device;
    returns a summary with every mismatch.

    A V record `V wid xa nin nout` follows the `R xa nin` record asserting
    its x8 (gen_layer_script.py:1506-1545); an A record `A idx val` asserts
    the running scan after the head's rows (gen_layer_script.py:1494-1503).
    """
    eng = art.engine
    script = script or art.prefix + ".txt"
    last_r = None
    last_v = None
    out = {"script": os.path.basename(script), "V": 0, "A": 0, "M": 0,
           "rows": 0, "bad": []}
    for rec in parse_script(script):
        if rec.kind == "R":
            last_r = rec
        elif rec.kind == "V":
            wid, xa, nin, nout = rec.fields
            assert last_r is not None and last_r.fields == (xa, nin), \
                f"V record {out['V']} without its R record"
            ent = art.entry(wid)
            assert nin == int(ent["k"]) and nout == int(ent["nrows"]), \
                f"V record {out['V']}: {nin} x {nout} against image {wid}"
            x8 = last_r.data.astype(np.int8)
            y = eng.matvec_y32(art.weights[wid], x8)
            if not np.array_equal(y.astype(np.int64), rec.data):
                bad = int(np.count_nonzero(y.astype(np.int64) != rec.data))
                out["bad"].append({"V": out["V"], "wid": wid, "rows_differing": bad})
            last_v = (wid, x8)
            out["V"] += 1
            out["rows"] += nout
        elif rec.kind == "A":
            idx, val = rec.fields
            val = val - (1 << 32) if val >= (1 << 31) else val
            assert last_v is not None, "A record before any V record"
            got = eng.head_argmax(art.weights[last_v[0]], last_v[1])
            if tuple(got) != (idx, val):
                out["bad"].append({"A": out["A"], "expected": [idx, val],
                                   "got": [int(got[0]), int(got[1])]})
            out["A"] += 1
        elif rec.kind == "M":
            tok, _dst, n = rec.fields
            emb = art.embedding(n) if os.path.exists(art.prefix + ".emb.bin") else None
            assert emb is not None and tok < emb.shape[0], \
                f"M record {out['M']}: token {tok} outside the embedding table"
            out["M"] += 1
        if log is not None and rec.kind in ("V", "A") and (out["V"] + out["A"]) % 50 == 0:
            log(f"{out['script']}: {out['V']} V, {out['A']} A records")
    return out


def main(argv):
    from .engine import Context
    if not argv:
        print(__doc__)
        return 2
    ctx = Context(0)
    rc = 0
    for prefix in argv:
        with Artifacts(ctx, prefix) as art:
            s = replay(art, log=lambda m: print(m, flush=True))
        print(json.dumps(s), flush=True)
        rc |= 1 if s["bad"] else 0
    return rc


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
