"""w4a8_head_topk32_noalloc_async, the head's TOPK-32 that allocates nothing
(its y32 and lists in the library's static per-GPU array), against
w4a8_head_topk32_async, the entry point that keeps them in the context's
buffer, and against the oracle: bit-exact, on two calls in a row, the second
with a smaller head, every output overwritten before each call; then a
graph capture of it, replayed with eager work between; and the refusal of a
head beyond the array's 2^18 rows."""
import numpy as np
import pytest
import torch

from fable5_llm_amd import _native as N
from oracle import cfast, law

pytestmark = pytest.mark.gpu


def _head(engine, rng, nrows, K):
    w4 = rng.integers(-8, 8, (nrows, K)).astype(np.int8)
    m = rng.integers(256, 16385, (nrows, K // 128)).astype(np.uint16)
    img, _ = law.pack_ddr_rows(w4, m)
    return img, engine.upload(img, nrows, K, law.sh_for_k(K))


def _oracle(img, nrows, K, x16, nw=None, in_f=0, one_plus=False):
    x = x16 if nw is None else law.rmsnorm_fx(x16, nw, in_f, one_plus)
    x8, _ = law.dyn_quant_i8(x)
    vals, rows, count, ovf = law.topk32(
        cfast.matvec_y32_img(img, nrows, K, law.sh_for_k(K), x8))
    return np.concatenate([vals, rows, [count, int(ovf)]]).astype(np.int32)


def _x16(rng, K):
    return np.clip(np.rint(rng.normal(0, 1, K) * 128), -32768, 32767).astype(np.int16)


def test_noalloc_matches_head_topk32_async(engine):
    rng = np.random.default_rng(2718)
    dev = torch.device("cuda", 0)
    # the largest head the array holds, then a smaller one with RMSNorm
    for nrows, K, rms in ((1 << 18, 512, False), (5000, 4096, True)):
        img, w = _head(engine, rng, nrows, K)
        try:
            x16 = _x16(rng, K)
            nw = rng.integers(-32768, 32768, K).astype(np.int16) if rms else None
            kw = {}
            if rms:
                kw = dict(prologue=N.PRO_RMSNORM_DYNQ8, norm_w=torch.from_numpy(nw).to(dev),
                          in_f=7, one_plus=True)
            xd = torch.from_numpy(x16).to(dev)
            a = torch.full((66,), -5, dtype=torch.int32, device=dev)
            b = torch.full((66,), -6, dtype=torch.int32, device=dev)
            torch.cuda.synchronize()
            engine.head_topk32_noalloc_async(w, xd, a, **kw)
            engine.sync()
            engine.head_topk32_async(w, xd, b, **kw)
            engine.sync()
            got, want = a.cpu().numpy(), b.cpu().numpy()
            ref = _oracle(img, nrows, K, x16, nw, 7, True)
            assert np.array_equal(got, want), (nrows, K)
            assert np.array_equal(got, ref), (nrows, K)
        finally:
            w.free()


def test_noalloc_graph_replays(engine):
    rng = np.random.default_rng(31415)
    dev = torch.device("cuda", 0)
    nrows, K = 20000, 2048
    img, w = _head(engine, rng, nrows, K)
    side = torch.cuda.Stream()
    try:
        xd = torch.from_numpy(_x16(rng, K)).to(dev)
        out = torch.zeros(66, dtype=torch.int32, device=dev)
        engine.head_topk32_noalloc_async(w, xd, out)     # eager before the capture
        engine.sync()
        g = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(g, stream=side):
                engine.set_stream(side)
                engine.head_topk32_noalloc_async(w, xd, out)
        finally:
            engine.set_stream(None)
        for k in range(3):
            x16 = _x16(rng, K)
            xd.copy_(torch.from_numpy(x16))
            want = _oracle(img, nrows, K, x16)
            out.fill_(-1)
            torch.cuda.synchronize()
            engine.head_topk32_noalloc_async(w, xd, out)  # eager between replays
            engine.sync()
            assert np.array_equal(out.cpu().numpy(), want), ("eager", k)
            out.fill_(-1)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy(), want), ("replay", k)
    finally:
        w.free()


def test_noalloc_refuses_beyond_its_array(engine):
    rng = np.random.default_rng(5)
    K = 128
    _, w = _head(engine, rng, (1 << 18) + 1, K)
    dev = torch.device("cuda", 0)
    try:
        xd = torch.zeros(K, dtype=torch.int16, device=dev)
        out = torch.zeros(66, dtype=torch.int32, device=dev)
        with pytest.raises(AssertionError, match="static scratch"):   # W4A8_E_RANGE
            engine.head_topk32_noalloc_async(w, xd, out)
    finally:
        w.free()
