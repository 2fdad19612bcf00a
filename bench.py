#!/usr/bin/env python3
"""Benchmark: the Qwen3.5-9B-shaped batch-1 decode weight stream on one MI355X.

One step = one pass of the W4A8 matvec path over the whole stream: 129 DYNQ8
sites (65 with a fused RMSNorm), 249 matrices, 4,091,805,696 bytes of int4
weights + uint16 scales, every matvec followed by its MOVY / SILU32 epilogue
and the 248,320-row LM head by its argmax.  All inputs are synthetic, seeded
and resident in HBM before the timed region.
--mode persistent (default) runs the whole step in one launch of one workgroup
per CU (--mode cooperative: the same launch through the cooperative launch API);
--fences auto (default) orders a site after an earlier one only where they
share a buffer (the synthetic sites share none), --fences all after every
earlier site.  --mode graph replays one GEMV launch per site as a HIP graph,
each site starting after the previous one completes.  The same plan in graph
mode is timed in the same run and reported as `ordered` (a decode step's
chain of dependent sites).

Prints one JSON line.  `value` = stream bytes / wall time per step.
`roofline` = the dominant kernel alone: stream bytes / sum of its per-launch
durations, each launch bracketed by dispatch-recorded HIP events (with the
launches' p10 / p50 / p90).  `config.end_hash` = SHA-256 of the step's end
state (every output and export), equal after a rerun over cleared outputs
and, in the `ordered` and `chained` legs, across launch modes.
`ffn` = one layer's SwiGLU block per call (w4a8_mlp_async) over the 32
layers, with the residual add.  `head` = the LM head alone, with its
argmax and with TOPK-32.
`batched` = the int8-MFMA kernel over the stream's 96 FFN matrices at B
tokens per pass (--batch), with its GB/s and MFMA utilisation.
`cpu_baseline` = the C oracle (oracle/law_c.c, OpenMP) over the same stream
on the host cores, which also checks every GPU output bit-exactly (and the
batched leg's outputs for layer 0's FFN matrices, every token).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_INT8_TOPS = 5000.0   # dense int8 MFMA, MI355X


def traffic_profile(kernel):
    return os.path.join(ROOT, "profiles", f"{kernel}_9b_stream_traffic.md")


def pmc_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3
    FETCH_SIZE + WRITE_SIZE passes (copy-calibrated); counters cannot be
    read from inside this process, so the figure comes from that summary."""
    try:
        for line in open(traffic_profile(kernel)):
            if line.startswith("| traffic_bytes_per_launch |"):
                return int(line.split("|")[2])
    except OSError:
        pass
    return None
METRIC = "achieved HBM GB/s (% of peak) on W4A8 GEMV; ms per 9B-shape weight stream"


STEADY_BATCH, STEADY_TOL, STEADY_MAX = 10, 0.01, 400


def warm_until_steady(run, sync, stream, min_steps):
    """Untimed steps until the step time has settled: at least `min_steps`,
    then batches of STEADY_BATCH steps (event-timed) until two consecutive
    batch means differ by less than STEADY_TOL, at most STEADY_MAX steps in
    all.  The GPU's clocks take tens of steps of continuous work to reach
    their steady state after idling.  Returns (steps run, last batch ms)."""
    import torch
    for _ in range(min_steps):
        run()
    n, prev, last = min_steps, None, None
    while n < STEADY_MAX:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(STEADY_BATCH):
            run()
        e1.record(stream)
        sync()
        e1.synchronize()
        n += STEADY_BATCH
        last = e0.elapsed_time(e1) / STEADY_BATCH
        if prev is not None and abs(last - prev) < STEADY_TOL * prev:
            break
        prev = last
    return n, last


def time_steps(st, ctx, stream, steps, warmup):
    """Warm up until steady, time `steps` replays (wall clock and events),
    then -- at the same clock state, with no idle gap -- `steps` more
    persistent launches each bracketed by dispatch-recorded events (the
    roofline's kernel time; graph mode: one profiled pass)."""
    import numpy as np
    import torch
    n_warm, _ = warm_until_steady(st.run, ctx.sync, stream, warmup)
    ctx.sync()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        st.run()
    e1.record(stream)
    ctx.sync()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    out = {"ms_per_step": wall * 1e3 / steps,
           "ms_per_step_hip_events": e0.elapsed_time(e1) / steps,
           "warmup_steps_run": n_warm}
    try:
        launches = st.plan.time_launches(steps)
        out["launch_ms"] = launches
        out["kernel_ms"] = float(np.median(launches))
        out["nlaunch"] = 1
    except ValueError:   # graph mode: one launch per site
        prof = st.profile()
        out["kernel_ms"] = float(prof.sum())
        out["nlaunch"] = int(prof.size)
    return out


def time_passes(ctx, one_pass, stream, steps, warmup):
    """ms per pass of `one_pass` submitted from Python (eager) and replayed
    as one HIP graph captured from it (the launches alone, without the host
    issuing each call); both timed with events on `stream`."""
    import torch

    def timed(fn):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        ctx.sync()
        torch.cuda.synchronize(stream.device)
        return e0.elapsed_time(e1) / steps

    for _ in range(warmup):
        one_pass()
    ctx.sync()
    eager = timed(one_pass)
    side = torch.cuda.Stream(stream.device)
    g = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.graph(g, stream=side):
            ctx.set_stream(side)
            one_pass()
    except Exception as e:   # keep the eager figure rather than lose the leg
        ctx.set_stream(stream)
        torch.cuda.synchronize(stream.device)
        return eager, eager, f"eager (graph capture failed: {type(e).__name__})"
    ctx.set_stream(stream)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize(stream.device)
    return timed(g.replay), eager, "HIP graph of one pass"


def _plain(o):
    """numpy scalars and arrays in a JSON line"""
    return o.item() if hasattr(o, "item") and getattr(o, "size", 1) == 1 else o.tolist()


def batched_leg(st, ctx, batches, steps, warmup, seed):
    """The FFN matrices of the stream (32 x gate, up: 12288 x 4096; down:
    4096 x 12288; 2.49 GB, far beyond the 256 MB Infinity Cache) through the
    batched int8-MFMA kernel, B tokens per pass: per-token x16 in Q8.7
    (N(0,1), 1 % outliers), DYNQ8 per token on the GPU, then
      * one matmul plan over all 96 matrices: ONE launch per pass, each
        matrix writing its own y32 (the leg's value), and
      * one w4a8_matmul_y32_multi_async launch per site (a layer's gate and
        up share their tokens' x8 and one launch; its down takes another:
        64 launches per pass), for comparison.
    Returns the timings and, for the oracle comparison, layer 0's inputs and the
    plan's outputs."""
    import numpy as np
    import torch
    from fable5_llm_amd import stream9b
    from fable5_llm_amd.engine import MatmulPlan
    dev = torch.device("cuda", ctx.device)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed + 7)
    ffn = [(si, mi) for si, s in enumerate(st.sites) for mi, m in enumerate(s.mats)
           if m.name.split(".")[-1] in ("gate", "up", "down")]
    stream = torch.cuda.current_stream(dev)
    out, keep = [], []
    for B in batches:
        x8 = {}
        for K in sorted({st.sites[si].mats[mi].K for si, mi in ffn}):
            rows = [ctx.dynq8(stream9b.synth_x16(gen, K, stream9b.RS_F).cpu().numpy())[0]
                    for _ in range(B)]
            x8[K] = torch.from_numpy(np.stack(rows)).to(dev)
        # per-site launches: one output per matrix position in its site
        y = {(mi, st.sites[si].mats[mi].nrows): None for si, mi in ffn}
        y = {k: torch.empty((B, k[1]), dtype=torch.int32, device=dev) for k in y}
        sites = {}
        for si, mi in ffn:
            sites.setdefault(si, []).append(mi)
        nbytes = ops = 0
        for si, mi in ffn:
            m = st.sites[si].mats[mi]
            nbytes += m.bytes + B * m.K + 4 * B * m.nrows
            ops += 2 * m.nrows * m.K * B

        def one_pass():
            for si, mis in sites.items():
                ms = [st.sites[si].mats[mi] for mi in mis]
                ctx.matmul_multi_async([st.weights[si][mi] for mi in mis],
                                       [x8[m.K] for m in ms],
                                       [y[(mi, m.nrows)] for mi, m in zip(mis, ms)])

        ms_site, _eager, how_site = time_passes(ctx, one_pass, stream, steps, warmup)
        # the plan: every matrix its own output
        yp = {}
        plan = MatmulPlan(ctx, B)
        for si, mi in ffn:
            m = st.sites[si].mats[mi]
            yp[(si, mi)] = torch.empty((B, m.nrows), dtype=torch.int32, device=dev)
            plan.add(st.weights[si][mi], x8[m.K], yp[(si, mi)])
        plan.run()      # writes its device table
        ctx.sync()
        ms, ms_eager, how = time_passes(ctx, plan.run, stream, steps, warmup)
        gbs = nbytes / (ms * 1e-3) / 1e9
        tops = ops / (ms * 1e-3) / 1e12
        gbs_site = nbytes / (ms_site * 1e-3) / 1e9
        out.append({"B": B, "matrices": len(ffn), "ms_per_pass": round(ms, 4),
                    "ms_per_pass_eager": round(ms_eager, 4), "timing": how,
                    "value": round(gbs, 1), "unit": "GB/s",
                    "pct_of_peak_hbm": round(100.0 * gbs / PEAK_HBM_GBS, 1),
                    "tops": round(tops, 2),
                    "mfma_util_pct": round(100.0 * tops / PEAK_INT8_TOPS, 2),
                    "mfma_util_basis": "algorithmic int8 ops / time / 5.0 POP/s; matrix-core "
                                       "busy cycles (SQ_VALU_MFMA_BUSY_CYCLES) in "
                                       "profiles/matmul_kernel_ffn_b8_b32.md",
                    "bytes_per_pass": nbytes,
                    "kernel": "matmul_kernel + matmul_finish_kernel (matmul plan)",
                    "launches_per_pass": 1,
                    "per_site_launches": {"launches_per_pass": len(sites),
                                          "ms_per_pass": round(ms_site, 4),
                                          "value": round(gbs_site, 1), "timing": how_site,
                                          "pct_of_peak_hbm":
                                              round(100.0 * gbs_site / PEAK_HBM_GBS, 1)}})
        # layer 0's gate, up and down from the plan's last run, for the oracle comparison
        plan.run()
        ctx.sync()
        for si, mi in ffn[:3]:
            m = st.sites[si].mats[mi]
            keep.append((B, si, mi, x8[m.K].cpu().numpy(), yp[(si, mi)].cpu().numpy()))
        plan.close()
        del yp
    return out, keep


def ffn_leg(st, ctx, steps, warmup):
    """The stream's 32 decoder-layer FFN blocks (RMSNorm -> DYNQ8 -> gate
    SILU32 / up SHIFT32W -> EMUL32 -> DYNQ8 -> down -> residual ADD), each
    on its own layer's input: 77.9 MB of weights per block, 2.49 GB per
    pass, timed three ways:
      * one persistent plan, each layer's down site right after its gate and
        up site (waiting for the EMUL32 product's words): the leg's value;
      * the same plan with each layer's down site after the next layer's
        gate and up site (the product is complete before it is needed);
      * w4a8_mlp_async per layer (two launches each), as one HIP graph.
    Every layer's block output and residual must be identical across the
    three.  Returns the timings and, for the oracle comparison, layer 0's input and
    outputs."""
    import torch
    from fable5_llm_amd import _native as N
    from fable5_llm_amd.engine import Plan
    dev = torch.device("cuda", ctx.device)
    stream = torch.cuda.current_stream(dev)
    layers = []
    for si, s in enumerate(st.sites):
        if s.name.endswith(".ln2"):
            down = st.sites[si + 1]
            assert down.name.endswith(".swiglu")
            g, u = s.mats
            d = down.mats[0]
            p0s = [g.p0(s.in_f), u.p0(s.in_f), d.p0(down.in_f)]
            x, nw = st.inputs[si]
            nbytes = g.bytes + u.bytes + d.bytes
            layers.append((si, st.weights[si][0], st.weights[si][1], st.weights[si + 1][0],
                           p0s, x, nw, s, nbytes))
    nbytes = sum(l[-1] for l in layers)
    outs = {}

    def new_outs(tag):
        outs[tag] = [(torch.empty(l[3].nrows, dtype=torch.int16, device=dev),
                      torch.empty(l[3].nrows, dtype=torch.int16, device=dev)) for l in layers]
        return outs[tag]

    o_l = new_outs("launches")

    def one_pass():
        for (_si, wg, wu, wd, p0s, x, nw, s, _b), (y, res) in zip(layers, o_l):
            ctx.mlp_async(wg, wu, wd, p0s, x, norm_w=nw, in_f=s.in_f,
                          one_plus=s.one_plus, mlp_out=y, res_out=res)

    ms_l, ms_l_eager, how_l = time_passes(ctx, one_pass, stream, steps, warmup)

    def plan_of(interleave):
        o = new_outs("interleaved" if interleave else "in_order")
        plan = Plan(ctx)
        if not interleave:
            for (_si, wg, wu, wd, p0s, x, nw, s, _b), (y, res) in zip(layers, o):
                plan.add_mlp(wg, wu, wd, p0s, x, norm_w=nw, in_f=s.in_f, one_plus=s.one_plus,
                             mlp_out=y, res_out=res)
        else:
            tmp = [(torch.empty(l[1].nrows, dtype=torch.int16, device=dev),
                    torch.empty(l[1].nrows, dtype=torch.int32, device=dev)) for l in layers]

            def up(i):
                _si, wg, wu, _wd, p0s, x, nw, s, _b = layers[i]
                plan.add_site([wg, wu], [N.EPI_SILU32, N.EPI_MOVY_P32], p0s[:2], list(tmp[i]),
                              x, prologue=N.PRO_RMSNORM_DYNQ8, norm_w=nw, in_f=s.in_f,
                              one_plus=s.one_plus)

            def down(i):
                _si, _wg, _wu, wd, p0s, x, _nw, _s, _b = layers[i]
                plan.add_site_emul_res(wd, p0s[2], tmp[i][0], tmp[i][1], x, o[i][1],
                                       out=o[i][0])
            up(0)
            for i in range(1, len(layers)):
                up(i)
                down(i - 1)
            down(len(layers) - 1)
            plan._keep.append(tmp)
        plan.set_mode(N.PLAN_PERSISTENT)
        plan.set_fences(N.FENCE_AUTO)
        return plan

    res = {}
    for tag, inter in (("in_order", False), ("interleaved", True)):
        plan = plan_of(inter)
        fenced = plan.fenced()
        plan.run()
        ctx.sync()
        ms, _e, how = time_passes(ctx, plan.run, stream, steps, warmup)
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[tag] = {"ms_per_pass": round(ms, 4), "value": round(gbs, 1), "unit": "GB/s",
                    "pct_of_peak_hbm": round(100.0 * gbs / PEAK_HBM_GBS, 1), "timing": how,
                    "launches_per_pass": 1,
                    "waits": {"input": fenced.count(N.WAIT_INPUT),
                              "grid": fenced.count(N.WAIT_GRID)}}
        plan.close()
    same = all(torch.equal(a, b) for tag in ("in_order", "interleaved")
               for la, lb in zip(outs["launches"], outs[tag]) for a, b in zip(la, lb))
    gbs_l = nbytes / (ms_l * 1e-3) / 1e9
    si, wg, wu, wd, p0s, x, nw, s, _ = layers[0]
    y, r = outs["in_order"][0]
    keep = (si, p0s, x.cpu().numpy(), nw.cpu().numpy(), y.cpu().numpy(), r.cpu().numpy())
    io = res["in_order"]
    return {"layers": len(layers), "ms_per_pass": io["ms_per_pass"],
            "us_per_layer": round(io["ms_per_pass"] * 1e3 / len(layers), 2),
            "value": io["value"], "unit": "GB/s", "pct_of_peak_hbm": io["pct_of_peak_hbm"],
            "bytes_per_pass": nbytes,
            "kernel": "stream_kernel (persistent plan, fences from buffers)",
            "interleaved": res["interleaved"],
            "per_layer_launches": {"ms_per_pass": round(ms_l, 4),
                                   "ms_per_pass_eager": round(ms_l_eager, 4), "timing": how_l,
                                   "value": round(gbs_l, 1),
                                   "pct_of_peak_hbm": round(100.0 * gbs_l / PEAK_HBM_GBS, 1),
                                   "launches_per_layer": 2},
            "waits": io["waits"], "outputs_identical_across_the_three": bool(same),
            "chain": "RMSNorm->DYNQ8->gate SILU32 + up SHIFT32W (one site; EMUL32 formed "
                     "as stored); EMUL32->DYNQ8->down SHIFT32->residual ADD (one site)"}, keep


def head_leg(st, ctx, steps, warmup):
    """The 248,320-row LM head on its own (final RMSNorm -> DYNQ8 -> matvec),
    once with the AMAX32 argmax and once with TOPK-32 (y32 to a scratch
    vector, then the TOPK kernel), `steps` calls each."""
    import torch
    dev = torch.device("cuda", ctx.device)
    stream = torch.cuda.current_stream(dev)
    s = st.sites[-1]
    assert s.head
    w = st.weights[-1][0]
    x, nw = st.inputs[-1]
    res = torch.zeros(2, dtype=torch.int32, device=dev)
    tk = torch.zeros(66, dtype=torch.int32, device=dev)
    from fable5_llm_amd import _native as N
    from fable5_llm_amd.engine import Plan
    tkp = torch.zeros(66, dtype=torch.int32, device=dev)
    plan = Plan(ctx)
    plan.add_head_topk32(w, x, tkp, prologue=s.prologue, norm_w=nw, in_f=s.in_f,
                         one_plus=s.one_plus)
    plan.set_mode(N.PLAN_PERSISTENT)
    calls = {
        "argmax": lambda: ctx.head_argmax_async(w, x, res, prologue=s.prologue, norm_w=nw,
                                                in_f=s.in_f, one_plus=s.one_plus),
        "topk32": lambda: ctx.head_topk32_async(w, x, tk, prologue=s.prologue, norm_w=nw,
                                                in_f=s.in_f, one_plus=s.one_plus),
        "topk32_in_plan": plan.run,
    }
    out = {"rows": s.mats[0].nrows, "bytes": s.mats[0].bytes}
    for name, fn in calls.items():
        for _ in range(warmup):
            fn()
        ctx.sync()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            fn()
        e1.record(stream)
        ctx.sync()
        torch.cuda.synchronize(dev)
        us = e0.elapsed_time(e1) * 1e3 / steps
        out[name] = {"us_per_call": round(us, 2),
                     "value": round(s.mats[0].bytes / (us * 1e-6) / 1e9, 1), "unit": "GB/s"}
    out["topk32"]["how"] = "w4a8_head_topk32_async: the head's y32, then the TOPK-32 kernel"
    out["topk32_in_plan"]["how"] = ("a persistent plan of the head alone "
                                    "(w4a8_plan_add_head_topk32): one launch, the scan "
                                    "inside it, chunk by chunk as the rows are stored")
    keep = (res.cpu().numpy(), tk.cpu().numpy(), tkp.cpu().numpy())
    plan.close()
    return out, keep


def head_check(ys, keep):
    """The head leg's argmax and TOPK-32 against the oracle's head y32."""
    import numpy as np
    from oracle import law
    res, tk, tkp = keep
    y = ys[-1][0]
    vals, rows, count, ovf = law.topk32(y)
    ok = tuple(int(v) for v in res) == tuple(int(v) for v in law.amax32(y))
    for t in (tk, tkp):
        ok = ok and int(t[64]) == count and bool(t[65]) == ovf
        ok = ok and np.array_equal(t[:count], vals) and np.array_equal(t[32:32 + count], rows)
    return "bit-exact" if ok else "MISMATCH"


def ffn_check(st, keep):
    """Layer 0's FFN block against the oracle: law.py for RMSNorm, DYNQ8,
    SILU32, EMUL32 and the shifts, oracle/law_c.c for the matvecs."""
    import numpy as np
    from fable5_llm_amd.stream9b import sh_for_k
    from oracle import cfast, law
    si, p0s, x16, nw, y, res = keep
    s, d = st.sites[si], st.sites[si + 1]
    imgs = [np.frombuffer(w.download(), dtype=np.uint8) for w in
            (st.weights[si][0], st.weights[si][1], st.weights[si + 1][0])]
    mats = (s.mats[0], s.mats[1], d.mats[0])

    def mv(k, x):
        m = mats[k]
        x8, e_x = law.dyn_quant_i8(x)
        yy = cfast.matvec_y32_img(imgs[k], m.nrows, m.K, sh_for_k(m.K), x8, 0)
        return law.rs_s(yy.astype(np.int64), p0s[k] - e_x)
    xn = law.rmsnorm_fx(x16, nw, s.in_f, s.one_plus)
    g, u = mv(0, xn), mv(1, xn)
    sg = law.clip16(np.array([law.silu_q(int(np.clip(v, -(1 << 20), (1 << 20) - 1)))
                              for v in g], dtype=np.int64))
    prod = law.clip16(law.rshift_round(sg * law.clip32(u), 12))
    ref_y = law.clip16(mv(2, prod))
    ok = np.array_equal(y.astype(np.int64), ref_y) and np.array_equal(
        res.astype(np.int64), law.clip16(x16.astype(np.int64) + ref_y))
    return "bit-exact" if ok else "MISMATCH"


def batched_check(st, keep):
    """Every kept batched output against B oracle matvec_y32 calls."""
    import numpy as np
    from fable5_llm_amd.stream9b import sh_for_k
    from oracle import cfast
    bad = 0
    for B, si, mi, x8, y in keep:
        m = st.sites[si].mats[mi]
        img = np.frombuffer(st.weights[si][mi].download(), dtype=np.uint8)
        for b in range(B):
            ref = cfast.matvec_y32_img(img, m.nrows, m.K, sh_for_k(m.K), x8[b], 0)
            bad += int(not np.array_equal(ref, y[b]))
    return "bit-exact" if bad == 0 else f"MISMATCH in {bad} token rows"


def topk_step_leg(st, ctx, stream, args, ms_argmax):
    """The headline step with its LM head ending in TOPK-32 instead of the
    argmax (a sampling step): the same resident weights and inputs, one
    persistent launch whose TOPK-32 scan runs as the head's rows are
    stored.  Returns the stream (for the oracle comparison) and its figures."""
    from fable5_llm_amd import _native as N
    from fable5_llm_amd import stream9b
    stt = stream9b.Stream9B(ctx, seed=args.seed, mode=N.PLAN_PERSISTENT, fences=N.FENCE_AUTO,
                            weights_from=st, head_topk=True)
    ctx.sync()
    tm = time_steps(stt, ctx, stream, args.steps, args.warmup)
    gbs = stt.bytes / (tm["ms_per_step"] * 1e-3) / 1e9
    return stt, {"ms_per_step": round(tm["ms_per_step"], 4), "value": round(gbs, 1),
                 "unit": "GB/s", "pct_of_peak_hbm": round(100.0 * gbs / PEAK_HBM_GBS, 1),
                 "kernel_us": round(tm["kernel_ms"] * 1e3, 2),
                 "us_over_argmax_step": round((tm["ms_per_step"] - ms_argmax) * 1e3, 2),
                 "how": "the headline plan with w4a8_plan_add_head_topk32 as its head"}


def chained_leg(ctx, stream, args):
    """The decode step with its dependences: every site reads an earlier
    site's output (stream9b.chain_sources; the swiglu sites form
    EMUL32(gate, up) in their prologue), so every site after the first
    waits for the one before it.  Timed as one persistent launch (fences
    derived from the buffers: 128) and as a HIP graph of one launch per
    site.  Same shapes and bytes as the headline stream; its own weights
    (scales 2^U(-13, -7), so that the chain does not saturate)."""
    from fable5_llm_amd import _native as N
    from fable5_llm_amd import stream9b
    st = stream9b.Stream9B(ctx, seed=args.seed + 1, chain=True, mode=N.PLAN_PERSISTENT,
                           fences=N.FENCE_AUTO)
    ctx.sync()
    fenced = st.plan.fenced()
    out = {"fences": sum(1 for f in fenced if f != N.WAIT_NONE),
           "grid_wide_waits": fenced.count(N.WAIT_GRID),
           "stamped_input_waits": fenced.count(N.WAIT_INPUT),
           "bytes_per_step": st.bytes}
    for name, mode in (("persistent", N.PLAN_PERSISTENT), ("graph", N.PLAN_GRAPH)):
        st.plan.set_mode(mode)
        tm = time_steps(st, ctx, stream, args.steps, args.warmup)
        gbs = st.bytes / (tm["ms_per_step"] * 1e-3) / 1e9
        leg = {"ms_per_step": round(tm["ms_per_step"], 4), "value": round(gbs, 1),
               "unit": "GB/s", "pct_of_peak_hbm": round(100.0 * gbs / PEAK_HBM_GBS, 1),
               "warmup_steps_run": tm["warmup_steps_run"]}
        if name == "persistent":
            ach = st.bytes / (tm["kernel_ms"] * 1e-3) / 1e9
            leg["roofline"] = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS,
                               "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBS, 4),
                               "kernel": "stream_kernel",
                               "avg_launch_us": round(tm["kernel_ms"] * 1e3, 3)}
            out["end_hash"] = st.digest()
            # per site class, from workgroup 0's stamps (as for the headline)
            import numpy as np
            prof = np.median(np.array([st.profile() for _ in range(5)]), axis=0)
            leg["per_class"] = per_class(st, prof)
        else:
            leg["end_hash_equal"] = st.digest() == out["end_hash"]
        out[name] = leg
    st.plan.set_mode(N.PLAN_PERSISTENT)
    return st, out


def c0_leg(ctx, stream, args, copies=64):
    """C0 (one 4096 x 4096 W4A8 matvec: DYNQ8 of an N(0,1) Q8.7 vector with
    1 % outliers, MOVY int16 out) over `copies` distinct resident matrices,
    8,650,752 B each (553 MB in all, beyond the 256 MB Infinity Cache, so
    every launch reads cold weights), back to back: replayed as a HIP graph
    of one GEMV launch per matrix, and as one persistent launch of all of
    them.  Per-matrix kernel times are dispatch-recorded events around each
    launch of an eagerly submitted pass.  Every output is kept for the
    oracle check."""
    import numpy as np
    import torch
    from fable5_llm_amd import _native as N
    from fable5_llm_amd import stream9b as S
    from fable5_llm_amd.engine import Plan
    dev = torch.device("cuda", ctx.device)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed + 11)
    K = nrows = S.H
    m = S.Mat("c0", nrows, K, S.RS_F, N.EPI_MOVY_I16)
    x = S.synth_x16(gen, K, S.RS_F)
    plan = Plan(ctx)
    ws, outs = [], []
    for _ in range(copies):
        img = S.synth_image(gen, nrows, K)
        torch.cuda.synchronize(dev)
        ws.append(ctx.upload(img, nrows, K, S.sh_for_k(K)))
        outs.append(torch.zeros(nrows, dtype=torch.int16, device=dev))
        plan.add_site([ws[-1]], [m.epi], [m.p0(S.RS_F)], [outs[-1]], x, prologue=N.PRO_DYNQ8)
    ctx.sync()

    class _P:   # what time_steps needs of a stream
        pass
    st = _P()
    st.run, st.plan, st.profile = plan.run, plan, plan.profile
    out = {"matrix": "4096x4096", "copies": copies, "bytes_per_matrix": m.bytes,
           "bytes_resident": m.bytes * copies}
    for name, mode in (("graph", N.PLAN_GRAPH), ("persistent", N.PLAN_PERSISTENT)):
        plan.set_mode(mode)
        plan.set_fences(N.FENCE_AUTO)
        tm = time_steps(st, ctx, stream, max(10, args.steps), args.warmup)
        us = tm["ms_per_step"] * 1e3 / copies
        leg = {"us_per_matrix": round(us, 3), "value": round(m.bytes / (us * 1e-6) / 1e9, 1),
               "unit": "GB/s", "pct_of_peak_hbm": round(100 * m.bytes / (us * 1e-6) / 1e9 /
                                                        PEAK_HBM_GBS, 1)}
        if name == "graph":
            per = np.array([plan.profile() for _ in range(5)]).reshape(-1) * 1e3
            leg["kernel_us_p10_p50_p90"] = [round(float(np.percentile(per, q)), 3)
                                            for q in (10, 50, 90)]
            leg["kernel_value"] = round(float(m.bytes / (np.median(per) * 1e-6) / 1e9), 1)
            leg["note"] = ("one gemv_kernel launch per matrix in a HIP graph; us_per_matrix "
                           "includes the launch gaps, kernel_us_* are the launches alone")
        else:
            leg["note"] = "all copies in one stream_kernel launch (no site waits)"
            leg["site_trace_us"] = site_trace(plan)
        out[name] = leg
    ctx.sync()
    keep = (x.cpu().numpy(), [np.frombuffer(w.download(), dtype=np.uint8) for w in ws[:8]],
            [o.cpu().numpy() for o in outs[:8]], m.p0(S.RS_F))
    plan.close()
    for w in ws:
        w.free()
    return out, keep


def site_trace(plan, reps=5):
    """A persistent plan's per-site times from workgroup 0's wall-clock
    stamps (w4a8_plan_profile: the control wavefront stamps each site as it
    starts storing it; the intervals are scaled to the launch's event time),
    medians over `reps` launches: the first site's (launch start-up
    included), the last one's (the launch's tail) and the spread of the
    others."""
    import numpy as np
    us = np.median(np.array([plan.profile() for _ in range(reps)]), axis=0) * 1e3
    mid = us[1:-1]
    return {"first": round(float(us[0]), 3), "last": round(float(us[-1]), 3),
            "others_p10_p50_p90": [round(float(np.percentile(mid, q)), 3) for q in (10, 50, 90)],
            "sum": round(float(us.sum()), 2),
            "basis": "workgroup 0's per-site wall-clock stamps, scaled to the launch's event "
                     "time; medians over %d launches" % reps}


def c0_check(keep):
    """The C0 leg's first 8 outputs against the oracle."""
    import numpy as np
    from oracle import cfast, law
    x16, imgs, outs, p0 = keep
    x8, e = law.dyn_quant_i8(x16)
    bad = 0
    for img, o in zip(imgs, outs):
        y = cfast.matvec_y32_img(img, 4096, 4096, 7, x8, 0)
        bad += int(not np.array_equal(o.astype(np.int64),
                                      np.asarray(law.movy(y, p0 - e, law.MOVY_INT16), np.int64)))
    return "bit-exact" if bad == 0 else f"MISMATCH in {bad} matrices"


def read_ceiling_leg(ctx, gib=4, launches=20):
    """The measured HBM read ceiling: a plain read of `gib` GiB with the
    weight stream's 16-byte non-temporal loads (w4a8_read_ceiling), at a few
    grid sizes; the best median is reported."""
    import numpy as np
    import torch
    buf = torch.empty(gib << 30, dtype=torch.uint8, device=torch.device("cuda", ctx.device))
    best, by_grid = None, {}
    # one workgroup per CU (32 KB in flight per CU, the whole GPU sweeping
    # one 8 MB window) reads fastest on MI355X; more in flight, slower
    for per_cu in (1, 2, 4, 8, 16):
        ms, nbytes = ctx.read_ceiling(buf, launches, grid=per_cu * ctx.num_cu)
        ms, nbytes = ctx.read_ceiling(buf, launches, grid=per_cu * ctx.num_cu)   # warm
        gbs = nbytes / (float(np.median(ms)) * 1e-3) / 1e9
        by_grid[str(per_cu * ctx.num_cu)] = round(gbs, 1)
        if best is None or gbs > best["value"]:
            best = {"value": round(gbs, 1), "unit": "GB/s", "bytes": nbytes,
                    "grid": per_cu * ctx.num_cu, "pct_of_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 1),
                    "kernel": "read_kernel (16-byte non-temporal loads, grid-stride, "
                              "32 KB per workgroup in flight, XOR-folded)"}
    best["gbs_by_grid"] = by_grid
    del buf
    return best


def site_class(s):
    """The class of a stream site: its role in the layer and its shapes."""
    tail = s.name.split(".")[-1]
    if s.head:
        return "head"
    kind = "dn" if any(m.name.endswith("in_qkv") for m in s.mats) or tail == "dn_heads" else \
        "attn" if tail in ("ln1", "attn_heads") else "ffn"
    return {"ln1": f"{kind}_ln1", "dn_heads": "dn_heads", "attn_heads": "attn_heads",
            "ln2": "ffn_gate_up", "swiglu": "ffn_down"}[tail]


def per_class(st, ms_sites):
    """Per site class of the stream: sites, matrices (rows x K), bytes per
    site, and the median time per site over the class's sites (ms_sites:
    one time per site, ms)."""
    import numpy as np
    out = {}
    for si, s in enumerate(st.sites):
        c = out.setdefault(site_class(s), {"sites": 0, "matrices": [
            f"{m.name.split('.')[-1]} {m.nrows}x{m.K}" for m in s.mats],
            "bytes_per_site": sum(m.bytes for m in s.mats), "_us": []})
        c["sites"] += 1
        c["_us"].append(float(ms_sites[si]) * 1e3)
    for c in out.values():
        us = float(np.median(c.pop("_us")))
        c["us_per_site"] = round(us, 3)
        c["gbs"] = round(c["bytes_per_site"] / (us * 1e-6) / 1e9, 1)
        c["pct_of_peak_hbm"] = round(100.0 * c["gbs"] / PEAK_HBM_GBS, 1)
    return out


def class_leg(st, reps=5):
    """Time per site class of the headline step, two ways: in the persistent
    launch (workgroup 0's control wavefront stamps the wall clock as it
    starts each site's stores; the intervals, scaled to the launch's event
    time, are the per-site times -- sites overlap, so an interval is the
    time between consecutive sites' ends on that workgroup) and as one
    gemv_kernel launch per site (dispatch-recorded events around each
    launch, graph mode).  Medians over `reps` instrumented passes."""
    import numpy as np
    from fable5_llm_amd import _native as N
    out = {}
    for name, mode in (("persistent", N.PLAN_PERSISTENT), ("per_site_launch", N.PLAN_GRAPH)):
        st.plan.set_mode(mode)
        prof = np.median(np.array([st.profile() for _ in range(reps)]), axis=0)
        out[name] = per_class(st, prof)
    st.plan.set_mode(N.PLAN_PERSISTENT)
    out["basis"] = ("persistent: per-site intervals of workgroup 0's wall-clock stamps, scaled to "
                    "the launch's event time; per_site_launch: one gemv_kernel per site, "
                    "dispatch-recorded events; medians over 5 instrumented passes, then over "
                    "the class's sites")
    return out


def seeds_leg(st, ctx, stream, args, seeds, imgs, chain=False):
    """The step again on other seeded inputs (Stream9B.reseed: every site's
    own input and RMSNorm weights redrawn; the resident weights stay): per
    seed, the step time (at least --warmup untimed steps then until steady,
    then --steps timed), the end hash, and the oracle's bit-exact check of
    every output.  imgs: the stream's row images (downloaded once)."""
    from tests import stream_check as sc
    per = []
    for seed in seeds:
        st.reseed(seed)
        tm = time_steps(st, ctx, stream, args.steps, args.warmup)
        host = sc.host_inputs(st, imgs)
        ref, _ = sc.run_cpu_stream(st, host)
        bad = sc.compare(st, host, ref)
        per.append({"seed": seed, "ms_per_step": round(tm["ms_per_step"], 4),
                    "kernel_us": round(tm["kernel_ms"] * 1e3, 2),
                    "end_hash": st.digest()[:16],
                    "parity": "bit-exact" if not bad else f"MISMATCH {len(bad)}: {bad[:3]}"})
    return per


def spread_of(values):
    import numpy as np
    v = np.asarray(values, dtype=float)
    return {"min": round(float(v.min()), 4), "median": round(float(np.median(v)), 4),
            "max": round(float(v.max()), 4),
            "max_over_min": round(float(v.max() / v.min()), 4)}


def cpu_host_info():
    """The host the CPU baseline ran on: model, logical CPUs, the affinity
    set this process may use."""
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    aff = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else []
    ranges, start = [], None
    for i, c in enumerate(aff):
        if start is None:
            start = c
        if i + 1 == len(aff) or aff[i + 1] != c + 1:
            ranges.append(f"{start}-{c}" if c != start else f"{c}")
            start = None
    return {"cpu_model": model, "host_cpus": os.cpu_count(),
            "affinity": ",".join(ranges), "affinity_count": len(aff)}


def cpu_per_config(st, host):
    """CPU baselines per configuration, on the stream's own matrices: C0 one
    4096 x 4096 (layer 0's in_z), C1 the FFN set (layer 0's gate and up,
    12288 x 4096, and down, 4096 x 12288), C2 the 248,320-row head.  Each by
    the C oracle with OpenMP on every host core (repeated for >= 0.5 s) and
    by the numpy restatement on one thread (once)."""
    import numpy as np
    from fable5_llm_amd.stream9b import sh_for_k
    from oracle import cfast, law
    def find(name):
        for si, s in enumerate(st.sites):
            for mi, m in enumerate(s.mats):
                if m.name == name:
                    return m, host[si]["imgs"][mi]
        raise KeyError(name)
    rng = np.random.default_rng(5)
    rates = {}   # K -> [bytes, numpy seconds]
    cfgs = {"C0": [find("L0.in_z")], "C1": [find("L0.gate"), find("L0.up"), find("L0.down")],
            "C2": [find("lm_head")]}
    out = {}
    for c, mats in cfgs.items():
        xs = {m.K: rng.integers(-127, 128, m.K).astype(np.int8) for m, _ in mats}
        nbytes = sum(m.bytes for m, _ in mats)
        n, t = 0, 0.0
        while t < 0.5:
            t0 = time.perf_counter()
            for m, img in mats:
                cfast.matvec_y32_img(img, m.nrows, m.K, sh_for_k(m.K), xs[m.K], 0)
            t += time.perf_counter() - t0
            n += 1
        tn = 0.0
        for m, img in mats:
            t0 = time.perf_counter()
            law.matvec_y32_image(img.tobytes(), m.nrows, m.K, sh_for_k(m.K), xs[m.K])
            dt = time.perf_counter() - t0
            tn += dt
            by_k = rates.setdefault(m.K, [0, 0.0])
            by_k[0] += m.bytes
            by_k[1] += dt
        out[c] = {"bytes": nbytes,
                  "c_openmp": {"ms": round(t / n * 1e3, 3),
                               "gbs": round(nbytes * n / t / 1e9, 2), "cores": cfast.num_threads()},
                  "numpy_1thread": {"ms": round(tn * 1e3, 1), "gbs": round(nbytes / tn / 1e9, 4)}}
    # C3 by numpy on one thread, extrapolated: the stream's bytes at each K
    # over the rate measured above for that K (numpy's int64 law is linear in
    # rows for a given K)
    c3_s = 0.0
    stream_bytes = {}
    for s in st.sites:
        for m in s.mats:
            stream_bytes[m.K] = stream_bytes.get(m.K, 0) + m.bytes
    for K, b in stream_bytes.items():
        mb, mt = rates[K]
        c3_s += b * mt / mb
    out["C3_numpy_1thread_extrapolated"] = {
        "ms_per_step": round(c3_s * 1e3, 1), "gbs": round(st.bytes / c3_s / 1e9, 4),
        "basis": "; ".join(f"K={K}: {b:,} B of the stream at {rates[K][0] / rates[K][1] / 1e9:.4f} "
                           f"GB/s (numpy 1 thread over the {rates[K][0]:,} B of C0-C2 with that K)"
                           for K, b in sorted(stream_bytes.items()))}
    return out


def chain_check(st, imgs=None):
    """The chained stream's last run against the oracle run site after site
    (each site fed from the oracle's own output of its producer)."""
    from tests import stream_check as sc
    host = sc.host_inputs(st, imgs)
    ref, _ = sc.run_cpu_stream(st, host)
    bad = sc.compare(st, host, ref)
    return "bit-exact" if not bad else f"MISMATCH {len(bad)}: {bad[:5]}"


def cpu_baseline(st, min_seconds, keep=(), keep_ffn=None, keep_head=None, imgs=None):
    """Oracle leg: the C restatement over the full stream, repeated until
    `min_seconds` of matvec work; returns its rate and the parity check (of
    the stream and of the batched leg's kept outputs).  imgs: the stream's
    row images, if already downloaded."""
    import numpy as np
    from oracle import cfast
    from tests import stream_check as sc
    host = sc.host_inputs(st, imgs)
    ref, total = sc.run_cpu_stream(st, host)
    passes = 1
    while total < min_seconds:
        total += sc.time_cpu_matvecs(st, host, ref)
        passes += 1
    bad = sc.compare(st, host, ref)
    ys = [r["ys"] for r in ref]
    per_config = cpu_per_config(st, host)
    # single-threaded numpy restatement on one 4096 x 4096 matrix (sample)
    from oracle import law
    s0 = st.sites[1]
    img = host[1]["imgs"][0]
    x8, _ = sc.oracle_prologue(s0, host[1])
    t0 = time.perf_counter()
    law.matvec_y32_image(img.tobytes(), s0.mats[0].nrows, s0.mats[0].K, 7, x8)
    t_np = time.perf_counter() - t0
    return {
        "value": round(st.bytes * passes / total / 1e9, 3),
        "unit": "GB/s",
        "cores": cfast.num_threads(),
        "kind": "port",
        "sample": (f"{passes} full passes of the stream's 249 matvec_y32 "
                   f"(4,091,805,696 B each) by oracle/law_c.c with OpenMP, "
                   f"{total:.1f} s of matvec work"),
        "ms_per_step": round(total / passes * 1e3, 2),
        "numpy_1thread_gbs": round(img.size / t_np / 1e9, 4),
        "numpy_sample": "one 4096x4096 matvec_y32 by oracle/law.py (int64 numpy)",
        **cpu_host_info(),
        "numpy": np.__version__,
        "parity": "bit-exact" if not bad else f"MISMATCH {len(bad)}: {bad[:5]}",
        "batched_parity": batched_check(st, keep) if keep else None,
        "ffn_parity": ffn_check(st, keep_ffn) if keep_ffn else None,
        "head_parity": head_check(ys, keep_head) if keep_head else None,
        "per_config": per_config,
    }


def log(msg):
    """Progress to stderr (the JSON line alone goes to stdout)."""
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=60,
                    help="untimed steps first; the GPU needs about 40 steps of "
                         "continuous work to reach its steady clocks")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 1 GiB device copy (known bytes), the "
                         "reference point for rocprofv3 FETCH_SIZE/WRITE_SIZE")
    ap.add_argument("--mode", choices=["persistent", "cooperative", "graph"],
                    default="persistent",
                    help="one launch per step (plain, or through the cooperative "
                         "launch API), or one launch per site replayed as a HIP graph")
    ap.add_argument("--fences", choices=["all", "auto"], default="auto",
                    help="persistent mode: every site waits for all earlier ones, "
                         "or only where it shares a buffer with one")
    ap.add_argument("--no-ordered", action="store_true",
                    help="skip timing the same plan strictly in order (graph mode)")
    ap.add_argument("--no-c0", action="store_true",
                    help="skip the C0 leg (4096x4096 over 64 cold copies) and the read ceiling")
    ap.add_argument("--no-chain", action="store_true",
                    help="skip the chained decode step (every site reads an earlier "
                         "site's output)")
    ap.add_argument("--no-ffn", action="store_true",
                    help="skip the FFN-block leg (w4a8_mlp_async per layer) and the "
                         "LM-head leg (argmax and TOPK-32 alone)")
    ap.add_argument("--batch", default="8,32",
                    help="token counts B for the batched int8-MFMA leg over the FFN "
                         "matrices (comma-separated, each <= 64; empty: skip)")
    ap.add_argument("--seeds", type=int, default=4,
                    help="the headline and chained steps on this many input seeds in "
                         "all (--seed, then --seed + 100, + 200, ...), each checked "
                         "against the oracle; the spread of their step times is reported")
    ap.add_argument("--only-batched", action="store_true",
                    help="run the batched leg alone (for profiling it) and print its results")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} / WORLD_SIZE "
              f"{world} is not supported (the W4A8 path runs on one GPU; its "
              f"row-sharded multi-GPU design is described, not built)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    if args.copy_calibration:
        # one dispatch that reads and writes exactly 1 GiB
        src = torch.ones(1 << 28, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 4,
                          "copy_bytes_written": dst.numel() * 4}), flush=True)
        return
    from fable5_llm_amd import stream9b
    from fable5_llm_amd.engine import Context

    ctx = Context(0)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx.set_stream(stream)
    t_build = time.perf_counter()
    from fable5_llm_amd import _native as N
    mode = {"persistent": N.PLAN_PERSISTENT, "cooperative": N.PLAN_PERSISTENT_COOP,
            "graph": N.PLAN_GRAPH}[args.mode]
    persistent = mode != N.PLAN_GRAPH
    fences = N.FENCE_AUTO if args.fences == "auto" else N.FENCE_ALL
    log("building the stream")
    st = stream9b.Stream9B(ctx, seed=args.seed, mode=mode, fences=fences)
    ctx.sync()
    t_build = time.perf_counter() - t_build
    tot = stream9b.totals(st.sites)
    if args.only_batched:
        batches = [int(b) for b in args.batch.split(",") if b.strip()]
        log("batched leg alone")
        res, keep = batched_leg(st, ctx, batches, args.steps, args.warmup, args.seed)
        print(json.dumps({"batched": res, "batched_parity": batched_check(st, keep)},
                         default=_plain), flush=True)
        st.close()
        ctx.close()
        return

    import numpy as np
    log("timing the headline step")
    tm = time_steps(st, ctx, stream, args.steps, args.warmup)
    ms_step, ms_step_ev = tm["ms_per_step"], tm["ms_per_step_hip_events"]
    kern_ms, nlaunch = tm["kernel_ms"], tm["nlaunch"]
    achieved = st.bytes / (kern_ms * 1e-3) / 1e9
    kernel = "stream_kernel" if persistent else "gemv_kernel"
    # the step's end state after the timed runs, and after one more run over
    # cleared outputs: every output written again, identically
    end_hash = st.digest()
    st.clear_outputs()
    st.run()
    end_hash_rerun = st.digest()

    ordered = None
    if not args.no_ordered and persistent:
        log("timing the ordered (graph mode) step")
        # the same plan with every site after the previous one: graph mode
        st.plan.set_mode(N.PLAN_GRAPH)
        to = time_steps(st, ctx, stream, args.steps, 3)
        gbs_o = st.bytes / (to["ms_per_step"] * 1e-3) / 1e9
        ordered = {
            "mode": "graph", "ms_per_step": round(to["ms_per_step"], 4),
            "value": round(gbs_o, 1), "unit": "GB/s",
            "pct_of_peak_hbm": round(100.0 * gbs_o / PEAK_HBM_GBS, 1),
            "end_hash_equal": st.digest() == end_hash,
            "note": "the same independent-input plan with every site starting after "
                    "the previous one completes; one gemv_kernel launch per site"}
        st.plan.set_mode(mode)

    c0 = keep_c0 = None
    if not args.no_c0:
        log("C0 leg: 4096x4096 over 64 cold copies")
        c0, keep_c0 = c0_leg(ctx, stream, args)
        log("read ceiling")
        line_ceiling = read_ceiling_leg(ctx)
    log("step ending in TOPK-32")
    stt, topk_step = topk_step_leg(st, ctx, stream, args, ms_step)
    chained = stc = None
    if not args.no_chain:
        log("chained step")
        stc, chained = chained_leg(ctx, stream, args)

    line = {
        "metric": METRIC,
        "value": round(st.bytes / (ms_step * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "ms_per_step_hip_events": round(ms_step_ev, 4),
        "warmup_steps_run": tm["warmup_steps_run"],
        "warmup_rule": (f"at least --warmup steps, then batches of {STEADY_BATCH} until two "
                        f"consecutive batch means differ by < {STEADY_TOL:.0%} (at most "
                        f"{STEADY_MAX} steps); the roofline's launches follow the timed "
                        "steps with no idle gap"),
        "pct_of_peak_hbm": round(100.0 * st.bytes / (ms_step * 1e-3) / 1e9 / PEAK_HBM_GBS, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 x int8 -> int32/int64",
        "data": "synthetic (seeded int4 codes, log-uniform 2^-10..2^-4 scales, "
                "N(0,1) activations with 1% outliers at +-20)",
        "config": {
            "workload": "Qwen3.5-9B-shaped batch-1 decode weight stream: "
                        "32 layers (24 DeltaNet-style, 8 attention-style) at "
                        "hidden 4096 / FFN 12288 + 248,320-row LM head argmax",
            "matrices": tot["matrices"], "dynq8_sites": tot["sites"],
            "rmsnorm_sites": tot["rmsnorm_sites"], "bytes_per_step": st.bytes,
            "reference_chunks": 1370, "batch": 1,
            "end_hash": end_hash,
            "end_hash_rerun_equal": end_hash_rerun == end_hash,
            "end_hash_of": ("SHA-256 of every output, x8 export and e_x of the step and "
                            "the head's (index, value), in site order"),
            "fences": args.fences if persistent else "all",
            "launch": (("one launch per step, one workgroup per CU (" +
                        ("cooperative launch API" if args.mode == "cooperative" else
                         "plain launch") + "); " +
                       ("a site waits for earlier ones only where it shares a buffer "
                        "with them (the synthetic sites share none)"
                        if args.fences == "auto" else
                        "every site waits for all earlier ones (per-workgroup flags)"))
                       if persistent
                       else "HIP graph, one GEMV launch per site, in order"),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": pmc_traffic(kernel),
            "traffic_source": ("rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated, "
                               f"profiles/{kernel}_9b_stream_traffic.md"),
            "kernel": kernel,
            "launches_per_step": nlaunch,
            "avg_launch_us": round(kern_ms / nlaunch * 1e3, 3),
            "launch_us_p10_p50_p90": ([round(float(np.percentile(tm["launch_ms"], q)) * 1e3, 3)
                                       for q in (10, 50, 90)] if "launch_ms" in tm else None),
            "bytes_per_launch": round(st.bytes / nlaunch),
            "timing": ("median of --steps back-to-back launches, dispatch-recorded HIP "
                       "events, right after the timed steps" if persistent else
                       "one profiled pass, dispatch-recorded HIP events per launch"),
        },
        "reference_fpga": {
            "stream_ms": 54.408, "gbs": 75.2,
            "source": "BN_CENSUS.md:415-419 (chip testbench, 4 DDR4 channels)"},
        "build_s": round(t_build, 1),
    }
    if ordered:
        line["ordered"] = ordered
    line["topk_step"] = topk_step
    if c0:
        line["c0"] = c0
        line["read_ceiling"] = line_ceiling
        line["roofline"]["frac_of_read_ceiling"] = round(achieved / line_ceiling["value"], 4)
    if chained:
        # what each fence adds over the independent-input step, same mode
        if persistent:
            chained["persistent"]["us_per_fence_over_unfenced"] = round(
                (chained["persistent"]["ms_per_step"] - ms_step) * 1e3 / max(1, chained["fences"]), 3)
        line["chained"] = chained
    batches = [int(b) for b in args.batch.split(",") if b.strip()]
    keep = ()
    if batches:
        log("batched leg")
        line["batched"], keep = batched_leg(st, ctx, batches, min(args.steps, 50),
                                            max(3, args.warmup // 10), args.seed)
    keep_head = None
    if not args.no_ffn:
        log("head leg")
        line["head"], keep_head = head_leg(st, ctx, min(args.steps, 50),
                                           max(3, args.warmup // 10))
    keep_ffn = None
    if not args.no_ffn:
        log("ffn leg")
        line["ffn"], keep_ffn = ffn_leg(st, ctx, min(args.steps, 50),
                                        max(3, args.warmup // 10))
    log("per site class")
    line["per_class"] = class_leg(st)
    imgs = imgs_c = None
    if not args.no_cpu:
        from tests import stream_check as sc
        imgs = sc.images(st)
        log("cpu baseline and parity")
        line["cpu_baseline"] = cpu_baseline(st, args.cpu_seconds, keep, keep_ffn, keep_head,
                                            imgs=imgs)
        log("TOPK-32 step parity")
        topk_step["parity"] = chain_check(stt, imgs)
        if stc is not None:
            log("chained parity")
            imgs_c = sc.images(stc)
            chained["parity"] = chain_check(stc, imgs_c)
        if keep_c0 is not None:
            c0["parity"] = c0_check(keep_c0)
    if args.seeds > 1 and not args.no_cpu:
        others = [args.seed + 100 * i for i in range(1, args.seeds)]
        log(f"headline on seeds {others}")
        first = {"seed": args.seed, "ms_per_step": round(ms_step, 4),
                 "kernel_us": round(kern_ms * 1e3, 2), "end_hash": end_hash[:16],
                 "parity": line["cpu_baseline"]["parity"]}
        per = [first] + seeds_leg(st, ctx, stream, args, others, imgs)
        line["seeds"] = {"headline": per,
                         "ms_per_step_spread": spread_of([p["ms_per_step"] for p in per]),
                         "kernel_us_spread": spread_of([p["kernel_us"] for p in per]),
                         "basis": ("Stream9B.reseed(seed): every site's input and RMSNorm "
                                   "weights redrawn, the resident weights kept; each seed "
                                   "warmed until steady, --steps timed, every output checked "
                                   "against the oracle")}
        if stc is not None:
            log(f"chained step on seeds {others}")
            stc.plan.set_mode(N.PLAN_PERSISTENT)
            firstc = {"seed": args.seed + 1,
                      "ms_per_step": chained["persistent"]["ms_per_step"],
                      "kernel_us": chained["persistent"]["roofline"]["avg_launch_us"],
                      "end_hash": chained["end_hash"][:16], "parity": chained.get("parity")}
            perc = [firstc] + seeds_leg(stc, ctx, stream, args, [o + 1 for o in others], imgs_c)
            line["seeds"]["chained"] = perc
            line["seeds"]["chained_ms_per_step_spread"] = spread_of(
                [p["ms_per_step"] for p in perc])
    if stc is not None:
        stc.close()
    stt.close()
    st.close()
    ctx.close()
    print(json.dumps(line, default=_plain), flush=True)


if __name__ == "__main__":
    main()
