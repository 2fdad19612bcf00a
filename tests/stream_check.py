"""CPU check of a device-resident Stream9B against the oracle (test
infrastructure: used by the GPU tests and bench.py's cpu_baseline leg).

For a chained stream the oracle feeds every site from its own result for
the producing site (the device's input buffers are not used), so a site
that read its input before the producer had finished shows up as a
mismatch, and so does any error carried down the chain."""
import time

import numpy as np

from fable5_llm_amd import _native as N
from fable5_llm_amd.stream9b import sh_for_k
from oracle import cfast, law


def images(st):
    """Every matrix's row image, downloaded from the device, per site."""
    return [[np.frombuffer(w.download(), dtype=np.uint8) for w in ws] for ws in st.weights]


def host_inputs(st, imgs=None):
    """Download what the CPU needs: per site (x16, norm_w, GPU x8, GPU e_x,
    GPU outputs) and per matrix the row image (`imgs`: from images(), for
    streams on the same weights)."""
    e_x = st.e_x.cpu().numpy()
    imgs = images(st) if imgs is None else imgs
    sites = []
    for si, s in enumerate(st.sites):
        x, nw = st.inputs[si]
        sites.append(dict(
            x16=x.cpu().numpy(), nw=None if nw is None else nw.cpu().numpy(),
            x8_gpu=None if st.x8[si] is None else st.x8[si].cpu().numpy(),
            e_gpu=int(e_x[si]), imgs=imgs[si],
            outs=[o.cpu().numpy() for o in st.outs[si]]))
    return sites


def oracle_prologue(s, h, x16=None, x2=None):
    """The site's x8 and e_x: RMSNorm or, for a chained swiglu site, EMUL32
    of x16 with x2 at p0 = 12 (gen_layer_script.py:1414-1418), then DYNQ8."""
    x = h["x16"] if x16 is None else x16
    if x2 is not None:
        x = law.alu_emul32(x2, x, 12).astype(np.int16)
    if s.prologue == N.PRO_RMSNORM_DYNQ8:
        x = law.rmsnorm_fx(x, h["nw"], s.in_f, s.one_plus)
    return law.dyn_quant_i8(x)


def oracle_epilogue(s, m, y, e, topk=False):
    """The site's output for matrix m from its y32 and the site's e_x (a
    TOPK-32 head: vals[32], rows[32], count, overflow)."""
    if s.head and topk:
        vals, rows, count, ovf = law.topk32(y)
        out = np.zeros(66, dtype=np.int64)
        out[:count], out[32:32 + count] = vals, rows
        out[64], out[65] = count, int(ovf)
        return out
    if s.head:
        return np.array(law.amax32(y), dtype=np.int64)
    shift = m.p0(s.in_f) - e
    if m.epi == N.EPI_SILU32:
        return np.asarray(law.alu_silu32(y, shift), np.int64)
    if m.epi == N.EPI_MOVY_P32:
        return np.asarray(law.movy(y, shift, law.MOVY_PAIRS32), np.int64)
    return np.asarray(law.movy(y, shift, law.MOVY_INT16), np.int64)


def run_cpu_stream(st, host, nthreads=0):
    """The oracle over every site of the stream in order: the prologue (law.py),
    every matvec_y32 (oracle/law_c.c) and epilogue.  A chained site's input is
    the oracle's own output of its producer (the first site's is the device
    input as downloaded).  Returns per-site dicts (x8, e, y32 list, output
    list) and the wall time of the matvec work alone."""
    ref = []
    t = 0.0
    for si, (s, h) in enumerate(zip(st.sites, host)):
        src = st.src[si]
        if src is not None:
            psi, pmi, off = src
            x16 = ref[psi]["outs"][pmi][off:off + s.K].astype(np.int16)
        else:
            x16 = h["x16"]
        x2 = None
        if st.emul[si] is not None:
            x2 = ref[st.emul[si][0]]["outs"][st.emul[si][1]]
        x8, e = oracle_prologue(s, h, x16, x2)
        ys, outs = [], []
        for m, img in zip(s.mats, h["imgs"]):
            t0 = time.perf_counter()
            y = cfast.matvec_y32_img(img, m.nrows, m.K, sh_for_k(m.K), x8, nthreads)
            t += time.perf_counter() - t0
            ys.append(y)
            outs.append(oracle_epilogue(s, m, y, e, getattr(st, "head_topk", False)))
        ref.append(dict(x8=x8, e=e, ys=ys, outs=outs))
    return ref, t


def time_cpu_matvecs(st, host, ref, nthreads=0):
    """One timing pass of the C oracle: every matvec_y32 of the stream on
    the x8 of an earlier run_cpu_stream (matvec work only, no prologues or
    epilogues).  Returns the wall time."""
    t = 0.0
    for s, h, r in zip(st.sites, host, ref):
        for m, img in zip(s.mats, h["imgs"]):
            t0 = time.perf_counter()
            cfast.matvec_y32_img(img, m.nrows, m.K, sh_for_k(m.K), r["x8"], nthreads)
            t += time.perf_counter() - t0
    return t


def compare(st, host, ref):
    """Bit-exact comparison of every GPU output and prologue export with the
    oracle's.  Returns a list of mismatch descriptions (empty = parity)."""
    bad = []
    for si, (s, h) in enumerate(zip(st.sites, host)):
        r = ref[si]
        if not s.head:
            if h["e_gpu"] != r["e"] or not np.array_equal(h["x8_gpu"], r["x8"]):
                bad.append(f"{s.name}: prologue")
        for m, want, out in zip(s.mats, r["outs"], h["outs"]):
            if not np.array_equal(out.astype(np.int64), want):
                bad.append(f"{m.name}: output")
    return bad


def spread(ref):
    """(smallest number of distinct values, largest fraction at the int16
    rails) over the int16 outputs of at least 1024 rows that the oracle
    formed: a degenerate chain -- values stuck at a few levels or clipped --
    would check little."""
    n, sat = [], []
    for r in ref:
        for o in r["outs"]:
            if o.size >= 1024 and o.max() <= 32767 and o.min() >= -32768:
                n.append(len(np.unique(o[:4096])))
                sat.append(float(np.mean((o == 32767) | (o == -32768))))
    return min(n), max(sat)
