#!/usr/bin/env python3
"""Write tests/golden/q9_vectors.npz: row images and y32 of the reference's
own `pack_ddr_rows` / `matvec_y32` (ref/w4a8_ref.py:349-370, 254-289) at the
9B engine's row geometry -- K = 4096 / 8192 / 12288, i.e. 1 / 2 / 3 scale
beats per row, a format none of the reference's committed images holds
(they stop at K = 3584, one scale beat).

Shapes and seed bases follow the reference's q9 vector target
(tb/Makefile:141-166: q1 13x4096, q2 7x8192, q3 5x12288, seeds 9100+s);
inputs are drawn here with numpy (int4 codes in [-8, 7], full-range uint16
mantissas in [1, 65535], int8 activations in [-128, 127] as quantize_acts
can produce), sh from the engine rule (w4a8_ref.py:177-179).

Run in the development container only (it reads the reference checkout);
the committed npz is data: inputs and expected outputs.
"""
import os
import sys

import numpy as np

REF = "/root/reference/ref"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "q9_vectors.npz")
SHAPES = [("q1", 13, 4096, 9100), ("q2", 7, 8192, 9200), ("q3", 5, 12288, 9300)]
SEEDS = (1, 2, 3)


def main():
    sys.path.insert(0, REF)
    import w4a8_ref as R

    out = {}
    for name, n, k, base in SHAPES:
        ng = k // 128
        sh = max(0, (ng * 65535 * (128 * 8 * 127)).bit_length() - 31)
        for s in SEEDS:
            rng = np.random.default_rng(base + s)
            w4 = rng.integers(-8, 8, size=(n, k), dtype=np.int8)
            m = rng.integers(1, 65536, size=(n, ng), dtype=np.int64).astype(np.uint16)
            x8 = rng.integers(-128, 128, size=k, dtype=np.int8)
            # one row of extreme codes: every product at its largest magnitude
            w4[0, :] = -8
            x8_ext = np.full(k, -128, dtype=np.int8)
            img_bytes, stride = R.pack_ddr_rows(w4, m, g=128)
            img = np.frombuffer(img_bytes, dtype=np.uint8)
            y = np.asarray(R.matvec_y32(w4, m, sh, x8, g=128), dtype=np.int64)
            y_ext = np.asarray(R.matvec_y32(w4, m, sh, x8_ext, g=128), dtype=np.int64)
            w4b, mb = R.unpack_ddr_rows(img_bytes, n, k, g=128)
            assert np.array_equal(np.asarray(w4b), w4)
            assert np.array_equal(np.asarray(mb), m)
            tag = f"{name}s{s}"
            out[f"{tag}_w4"] = w4
            out[f"{tag}_m"] = m
            out[f"{tag}_x8"] = x8
            out[f"{tag}_img"] = img.reshape(-1)
            out[f"{tag}_y32"] = y.astype(np.int32)
            out[f"{tag}_y32_ext"] = y_ext.astype(np.int32)
            out[f"{tag}_shape"] = np.array([n, k, sh, stride], dtype=np.int64)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays")


if __name__ == "__main__":
    main()
