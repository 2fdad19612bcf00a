"""CPU check of a device-resident Stream9B against the oracle (test
infrastructure: used by the GPU tests and bench.py's cpu_baseline leg)."""
import time

import numpy as np

from fable5_llm_amd import _native as N
from fable5_llm_amd.stream9b import sh_for_k
from oracle import cfast, law


def host_inputs(st):
    """Download what the CPU needs: per site (x16, norm_w, GPU x8, GPU e_x)
    and per matrix the row image."""
    e_x = st.e_x.cpu().numpy()
    sites = []
    for si, s in enumerate(st.sites):
        x, nw = st.inputs[si]
        sites.append(dict(
            x16=x.cpu().numpy(), nw=None if nw is None else nw.cpu().numpy(),
            x8_gpu=None if st.x8[si] is None else st.x8[si].cpu().numpy(),
            e_gpu=int(e_x[si]),
            imgs=[np.frombuffer(w.download(), dtype=np.uint8) for w in st.weights[si]],
            outs=[o.cpu().numpy() for o in st.outs[si]]))
    return sites


def oracle_prologue(s, h):
    x = h["x16"]
    if s.prologue == N.PRO_RMSNORM_DYNQ8:
        x = law.rmsnorm_fx(x, h["nw"], s.in_f, s.one_plus)
    return law.dyn_quant_i8(x)


def run_cpu_stream(st, host, nthreads=0):
    """The C oracle over every matrix of the stream: returns per-site y32
    lists and the wall time of the matvec work alone."""
    ys = []
    t = 0.0
    for s, h in zip(st.sites, host):
        x8, _e = oracle_prologue(s, h)
        row = []
        for m, img in zip(s.mats, h["imgs"]):
            t0 = time.perf_counter()
            y = cfast.matvec_y32_img(img, m.nrows, m.K, sh_for_k(m.K), x8, nthreads)
            t += time.perf_counter() - t0
            row.append(y)
        ys.append(row)
    return ys, t


def compare(st, host, ys):
    """Bit-exact comparison of every GPU output with the oracle.  Returns a
    list of mismatch descriptions (empty = parity)."""
    bad = []
    for si, (s, h) in enumerate(zip(st.sites, host)):
        x8, e = oracle_prologue(s, h)
        if not s.head:
            if h["e_gpu"] != e or not np.array_equal(h["x8_gpu"], x8):
                bad.append(f"{s.name}: prologue")
        for m, y, out in zip(s.mats, ys[si], h["outs"]):
            if s.head:
                want = np.array(law.amax32(y), dtype=np.int64)
            else:
                shift = m.p0(s.in_f) - e
                if m.epi == N.EPI_SILU32:
                    want = law.alu_silu32(y, shift)
                elif m.epi == N.EPI_MOVY_P32:
                    want = law.movy(y, shift, law.MOVY_PAIRS32)
                else:
                    want = law.movy(y, shift, law.MOVY_INT16)
            if not np.array_equal(out.astype(np.int64), np.asarray(want, np.int64)):
                bad.append(f"{m.name}: output")
    return bad
