#!/usr/bin/env python3
"""Extract small golden fixtures from the reference's committed test data.

Reads (as data only, never imports) the reference checkout's golden vectors
and writes compressed .npz fixtures next to this script:

  ref_vectors.npz   tb/vec_s1..s4 (matvec engine vectors: params, x8 words,
                    512-bit beats, y32), tb/vectors/s1..s4 ALU/RMSNorm
                    vectors, roms/{rsqrt,sigmoid}_rom.hex,
                    tb/rsqrt_cases_s*.txt, tb/silu_cases_s*.txt
  ref_scripts.npz   every V / R / E / A record of tb/scripts/{layer,token}_s*.txt
                    with a row subset of each weight image (<prefix>_w<wid>.bin)
                    and the matching y32 rows; the full head y32 before each
                    A record (for the argmax check); for the first MLP block
                    of each script (gate and up V records sharing their input,
                    then the down V record reading their width), the full gate
                    and up y32 and the down record's x8 and e_x (the SwiGLU
                    chain between them, gen_layer_script.py:2166-2190)

File formats are those written by ref/gen_matvec_vectors.py:38-50,
ref/gen_layer_vectors.py:29-33, ref/gen_rsqrt_cases.py:10-15,
ref/gen_silu_cases.py:9-14 and the record grammar of
ref/gen_layer_script.py:648-702 / 1487-1545.

Usage: python3 tests/golden/make_fixtures.py [/root/reference]
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
ROWS_FIRST, ROWS_RANDOM, ROWS_LAST = 8, 8, 8


def hexfile(path, bits):
    """One two's-complement hex value per line -> int64 array."""
    vals = []
    with open(path) as f:
        for line in f:
            line = line.strip()
            if not line:
                continue
            v = int(line, 16) & ((1 << bits) - 1)
            if v >> (bits - 1):
                v -= 1 << bits
            vals.append(v)
    return np.array(vals, dtype=np.int64)


def vec_dirs(out):
    for s in range(1, 5):
        d = f"{REF}/tb/vec_s{s}"
        K, NG, SH, N, BPR = map(int, open(f"{d}/params.txt").read().split())
        xb = bytearray()
        for line in open(f"{d}/x8.hex"):
            if line.strip():
                xb += int(line, 16).to_bytes(4, "little")
        x8 = np.frombuffer(bytes(xb[:K]), dtype=np.int8).copy()
        img = bytearray()
        for line in open(f"{d}/beats.hex"):
            if line.strip():
                img += int(line, 16).to_bytes(64, "little")
        y32 = hexfile(f"{d}/y32.hex", 32).astype(np.int32)
        assert len(img) == N * BPR * 64 and y32.size == N
        out[f"vec{s}_params"] = np.array([K, NG, SH, N, BPR], dtype=np.int64)
        out[f"vec{s}_x8"] = x8
        out[f"vec{s}_img"] = np.frombuffer(bytes(img), dtype=np.uint8).copy()
        out[f"vec{s}_y32"] = y32


def layer_vectors(out):
    files16 = ["alu_dynq8_x", "alu_dynq8_y", "alu_dynq8_e", "alu_shift32_y",
               "alu_silu32_y", "alu_emul32_y", "alu_emul_b",
               "rmsnorm_x16", "rmsnorm_w14", "rmsnorm_y16"]
    files32 = ["alu_shift32_v", "alu_shift32w_y"]
    for s in range(1, 5):
        d = f"{REF}/tb/vectors/s{s}"
        for name in files16:
            out[f"s{s}_{name}"] = hexfile(f"{d}/{name}.hex", 16)
        for name in files32:
            out[f"s{s}_{name}"] = hexfile(f"{d}/{name}.hex", 32)
    roms = f"{REF}/tb/vectors/s1/roms"
    out["rom_rsqrt"] = hexfile(f"{roms}/rsqrt_rom.hex", 17)   # unsigned 16-bit
    out["rom_sigmoid"] = hexfile(f"{roms}/sigmoid_rom.hex", 17)
    for s in range(2, 5):
        r2 = f"{REF}/tb/vectors/s{s}/roms"
        assert np.array_equal(hexfile(f"{r2}/rsqrt_rom.hex", 17), out["rom_rsqrt"])
        assert np.array_equal(hexfile(f"{r2}/sigmoid_rom.hex", 17), out["rom_sigmoid"])


def case_files(out):
    for s in range(1, 5):
        rows = []
        for line in open(f"{REF}/tb/rsqrt_cases_s{s}.txt"):
            if line.strip():
                v, P, r, e = (int(t, 16) for t in line.split())
                rows.append((v, P, r, e - 256 if e >= 128 else e))
        out[f"rsqrt_cases{s}"] = np.array(rows, dtype=np.int64)
        rows = []
        for line in open(f"{REF}/tb/silu_cases_s{s}.txt"):
            if line.strip():
                x, y = (int(t, 16) for t in line.split())
                x = x - (1 << 21) if x >> 20 else x
                y = y - (1 << 16) if y >> 15 else y
                rows.append((x, y))
        out[f"silu_cases{s}"] = np.array(rows, dtype=np.int64)


def parse_script(path):
    """Yield (kind, header_fields, data_values) for the records we use."""
    with open(path) as f:
        lines = f.read().split("\n")
    i = 0
    n = len(lines)
    while i < n:
        line = lines[i]
        i += 1
        if not line:
            continue
        t = line.split()
        k = t[0]
        if k in ("W", "R"):
            cnt = int(t[2], 16)
            data = lines[i:i + cnt]
            i += cnt
            if k == "R":
                yield k, t[1:], data
        elif k == "V":
            cnt = int(t[4], 16)
            data = lines[i:i + cnt]
            i += cnt
            yield k, t[1:], data
        elif k in ("E", "A", "C"):
            yield k, t[1:], None


def s16(words):
    v = np.array([int(w, 16) for w in words], dtype=np.int64)
    return np.where(v >= 32768, v - 65536, v)


def s32(words):
    v = np.array([int(w, 16) for w in words], dtype=np.int64)
    return np.where(v >= (1 << 31), v - (1 << 32), v)


def scripts(out):
    for kind in ("layer", "token"):
        for s in range(1, 5):
            prefix = f"{REF}/tb/scripts/{kind}_s{s}"
            tag = f"{kind}{s}"
            man = json.load(open(f"{prefix}.weights.json"))
            rng = np.random.default_rng(1000 * s + (kind == "token"))
            rowsel = {}
            for wid, ent in man.items():
                if not wid.isdigit():
                    continue
                nr = int(ent["nrows"])
                mid = np.arange(ROWS_FIRST, max(ROWS_FIRST, nr - ROWS_LAST))
                pick = (rng.choice(mid, size=min(ROWS_RANDOM, mid.size),
                                   replace=False) if mid.size else [])
                rows = np.unique(np.concatenate([
                    np.arange(min(ROWS_FIRST, nr)), np.asarray(pick, np.int64),
                    np.arange(max(0, nr - ROWS_LAST), nr)])).astype(np.int64)
                rowsel[int(wid)] = rows
                stride = int(ent["stride"])
                img = np.fromfile(f"{os.path.dirname(prefix)}/{ent['file']}",
                                  dtype=np.uint8)
                assert img.size == nr * stride
                img = img.reshape(nr, stride)
                out[f"{tag}_w{wid}_rows"] = rows
                out[f"{tag}_w{wid}_img"] = img[rows].reshape(-1).copy()
                out[f"{tag}_w{wid}_meta"] = np.array(
                    [nr, int(ent["k"]), int(ent["ng"]), int(ent["sh"]),
                     int(ent["e"]), stride], dtype=np.int64)
            last_r = None
            last_e = None
            nv = 0
            na = 0
            last_head_y = None
            pending_v = None
            recent = []          # (v index, wid, nin, nr, full y32) of the last V records
            mlp_done = False
            for k, hdr, data in parse_script(f"{prefix}.txt"):
                if k == "R":
                    last_r = (int(hdr[0], 16), s16(data))
                elif k == "E":
                    last_e = int(hdr[0], 16)
                elif k == "V":
                    wid, xa, nin, nr = (int(h, 16) for h in hdr)
                    assert last_r is not None and last_r[0] == xa \
                        and last_r[1].size == nin, "V without its R record"
                    x8 = last_r[1]
                    assert x8.min() >= -128 and x8.max() <= 127
                    y = s32(data)
                    rows = rowsel[wid]
                    out[f"{tag}_v{nv}_hdr"] = np.array(
                        [wid, nin, nr, last_e], dtype=np.int64)
                    out[f"{tag}_v{nv}_x8"] = x8.astype(np.int8)
                    out[f"{tag}_v{nv}_y32"] = y[rows].astype(np.int32)
                    if nr == int(man[str(wid)]["nrows"]) and wid == max(rowsel):
                        last_head_y = y.astype(np.int32)
                    if (not mlp_done and len(recent) >= 2 and recent[-1][3] == nin
                            and recent[-2][3] == nin and recent[-1][2] == recent[-2][2]):
                        g, u = recent[-2], recent[-1]
                        out[f"{tag}_mlp_v"] = np.array([g[0], u[0], nv], dtype=np.int64)
                        out[f"{tag}_mlp_gate_y32"] = g[4].astype(np.int32)
                        out[f"{tag}_mlp_up_y32"] = u[4].astype(np.int32)
                        out[f"{tag}_mlp_down_x8"] = x8.astype(np.int8)
                        out[f"{tag}_mlp_down_e"] = np.array([last_e], dtype=np.int64)
                        mlp_done = True
                    recent = (recent + [(nv, wid, nin, nr, y)])[-2:]
                    pending_v = nv
                    nv += 1
                elif k == "C" and pending_v is not None:
                    # first layer command after a V record: the ALU op that
                    # dequantises that result (gen_layer_script.py:1756-1767)
                    op, a0, a1, a2 = (int(h, 16) for h in hdr)
                    out[f"{tag}_v{pending_v}_cmd"] = np.array(
                        [op, a0, a1, a2], dtype=np.int64)
                    pending_v = None
                elif k == "A":
                    idx, val = int(hdr[0], 16), int(hdr[1], 16)
                    val = val - (1 << 32) if val >= (1 << 31) else val
                    assert last_head_y is not None
                    out[f"{tag}_a{na}"] = np.array([idx, val], dtype=np.int64)
                    out[f"{tag}_a{na}_y32"] = last_head_y
                    na += 1
            out[f"{tag}_counts"] = np.array([nv, na], dtype=np.int64)
            print(f"{tag}: {nv} V records, {na} A records, "
                  f"{len(rowsel)} weight images", flush=True)


def main():
    vec = {}
    vec_dirs(vec)
    layer_vectors(vec)
    case_files(vec)
    np.savez_compressed(f"{HERE}/ref_vectors.npz", **vec)
    scr = {}
    scripts(scr)
    np.savez_compressed(f"{HERE}/ref_scripts.npz", **scr)
    for n in ("ref_vectors.npz", "ref_scripts.npz"):
        print(n, os.path.getsize(f"{HERE}/{n}"), "bytes")


if __name__ == "__main__":
    main()
