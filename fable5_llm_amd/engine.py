"""Handle-level API over the C ABI: a Context owns one HIP stream on one
device; Weights are device-resident matrices repacked once from the
reference's row image (w4a8_ref.pack_ddr_rows layout).

Host-array methods (numpy in, numpy out) are synchronous; *_async methods
take torch tensors already on the device and enqueue on the context stream.
"""
import ctypes

import numpy as np

from . import _native as N

_c = ctypes.c_void_p


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def _dptr(t):
    """device pointer of a torch tensor (or None)"""
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _dev(t, need_bytes, name, required=True):
    """Check a device tensor handed to a kernel as a raw pointer: on the
    device, contiguous and at least need_bytes long (the C ABI cannot see a
    pointer's extent, so a short buffer would be written past).  None passes
    when the argument is optional."""
    if t is None:
        if required:
            raise ValueError(f"{name}: a device tensor is required")
        return
    if not getattr(t, "is_cuda", False):
        raise ValueError(f"{name}: must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")
    have = t.numel() * t.element_size()
    if have < need_bytes:
        raise ValueError(f"{name}: {have} bytes, the call touches {need_bytes}")


# bytes per output row of each epilogue
_EPI_BYTES = {N.EPI_Y32: 4, N.EPI_MOVY_I16: 2, N.EPI_MOVY_P32: 4, N.EPI_SILU32: 2,
              N.EPI_SHIFT_I64: 8}


def _x_bytes(prologue, K):
    return K if prologue == N.PRO_X8 else 2 * K


def wire_stride(K):
    ng = K // 128
    return (ng + (ng + 31) // 32) * 64


class Weights:
    """A W4A8 matrix resident in HBM in the engine's tile layout."""

    def __init__(self, ctx, handle, nrows, K, sh):
        self.ctx, self.h, self.nrows, self.K, self.sh = ctx, handle, nrows, K, sh
        dev = ctypes.c_int64()
        N.check(N.lib().w4a8_weights_info(handle, None, None, None,
                                           ctypes.byref(dev)))
        self.device_bytes = int(dev.value)

    @property
    def wire_bytes(self):
        return self.nrows * wire_stride(self.K)

    def download(self):
        """The row image back from the device (bytes)."""
        out = np.empty(self.wire_bytes, dtype=np.uint8)
        N.check(N.lib().w4a8_weights_download(self.ctx.h, self.h, _ptr(out)))
        return out.tobytes()

    def free(self):
        if self.h:
            N.lib().w4a8_weights_free(self.h)
            self.h = None

    def __del__(self):
        try:
            if self.h and self.ctx.h:
                self.free()
        except Exception:
            pass


class Context:
    def __init__(self, device=0):
        h = ctypes.c_void_p()
        N.check(N.lib().w4a8_ctx_create(device, ctypes.byref(h)), "ctx_create")
        self.h = h
        self.device = device
        cu, grid = ctypes.c_int32(), ctypes.c_int32()
        N.check(N.lib().w4a8_ctx_info(self.h, ctypes.byref(cu), ctypes.byref(grid)))
        self.num_cu, self.grid = int(cu.value), int(grid.value)

    def close(self):
        if self.h:
            N.lib().w4a8_ctx_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # ------------------------------------------------------------ control
    def set_stream(self, stream=None):
        """Run on a torch.cuda.Stream (or raw hipStream_t int); None = the
        context's own stream.  The null/legacy stream (handle 0) cannot be
        selected: pass a created stream."""
        s = None if stream is None else int(getattr(stream, "cuda_stream", stream))
        if stream is not None and s == 0:
            raise ValueError("the null stream cannot be selected; use a "
                             "torch.cuda.Stream() created for the engine")
        N.check(N.lib().w4a8_ctx_set_stream(self.h, ctypes.c_void_p(s)))

    def set_spin_limit(self, grid_polls=0, lds_polls=0):
        """Polls before the bounded waits of later persistent-plan and
        TOPK-32 launches give up (0: the defaults); a wait that gives up is
        reported as a RuntimeError at the next sync."""
        N.check(N.lib().w4a8_ctx_set_spin_limit(self.h, int(grid_polls), int(lds_polls)))

    def set_grid(self, grid):
        N.check(N.lib().w4a8_ctx_set_grid(self.h, int(grid)))

    def sync(self):
        N.check(N.lib().w4a8_ctx_sync(self.h), "sync")

    def tables(self):
        r = np.empty(512, dtype=np.int32)
        s = np.empty(257, dtype=np.int32)
        N.check(N.lib().w4a8_tables(self.h, _ptr(r), _ptr(s)))
        return r, s

    def read_ceiling(self, buf, n, grid=0):
        """Kernel ms of each of n launches reading the device tensor `buf`
        once (16-byte non-temporal loads): the measured HBM read ceiling."""
        _dev(buf, 16, "buf")
        nbytes = (buf.numel() * buf.element_size()) // 16 * 16
        ms = np.zeros(n, dtype=np.float32)
        N.check(N.lib().w4a8_read_ceiling(self.h, _dptr(buf), nbytes, int(grid), int(n),
                                          _ptr(ms)), "read_ceiling")
        return ms, nbytes

    # ------------------------------------------------------------ weights
    def upload(self, img, nrows, K, sh):
        """img: row image (bytes / uint8 array on the host, or a uint8 torch
        tensor on the device)."""
        h = ctypes.c_void_p()
        if hasattr(img, "data_ptr"):
            assert img.numel() == nrows * wire_stride(K), "image size"
            N.check(N.lib().w4a8_weights_upload_async(
                self.h, _dptr(img), nrows, K, sh, ctypes.byref(h)), "upload")
        else:
            a = np.frombuffer(img, dtype=np.uint8) if isinstance(img, (bytes, bytearray)) \
                else np.ascontiguousarray(img, dtype=np.uint8).reshape(-1)
            assert a.size == nrows * wire_stride(K), \
                f"image is {a.size}B, expected {nrows}*{wire_stride(K)}"
            N.check(N.lib().w4a8_weights_upload(self.h, _ptr(a), nrows, K, sh,
                                                 ctypes.byref(h)), "upload")
        return Weights(self, h, nrows, K, sh)

    # -------------------------------------------------- elementwise (host)
    def rshift_round(self, v, s):
        a = np.ascontiguousarray(np.asarray(v, dtype=np.int64).reshape(-1))
        out = np.empty_like(a)
        N.check(N.lib().w4a8_rshift_round(self.h, _ptr(a), a.size, int(s), _ptr(out)))
        return out.reshape(np.shape(v))

    def dynq8(self, x16):
        x = np.ascontiguousarray(np.asarray(x16, dtype=np.int16).reshape(-1))
        n = x.size
        pad = (-n) % 8
        if pad:   # zeros never change max|x|, so padding is exact
            x = np.concatenate([x, np.zeros(pad, np.int16)])
        x8 = np.empty(x.size, dtype=np.int8)
        e = ctypes.c_int32()
        N.check(N.lib().w4a8_dynq8(self.h, _ptr(x), x.size, _ptr(x8), ctypes.byref(e)),
                "dyn_quant_i8")
        return x8[:n], int(e.value)

    def rmsnorm(self, x16, w_q14, in_f, one_plus):
        x = np.ascontiguousarray(np.asarray(x16, dtype=np.int16).reshape(-1))
        w = np.ascontiguousarray(np.asarray(w_q14, dtype=np.int16).reshape(-1))
        assert w.size == x.size, "weight length"
        out = np.empty(x.size, dtype=np.int16)
        N.check(N.lib().w4a8_rmsnorm(self.h, _ptr(x), _ptr(w), x.size, int(in_f),
                                     1 if one_plus else 0, _ptr(out)), "rmsnorm_fx")
        return out

    def movy(self, y32, shift, mode):
        y = np.ascontiguousarray(np.asarray(y32, dtype=np.int32).reshape(-1))
        out = np.empty(y.size, dtype=np.int16 if mode == N.MOVY_INT16 else np.int32)
        N.check(N.lib().w4a8_movy(self.h, _ptr(y), y.size, int(shift), int(mode),
                                  _ptr(out)), "movy")
        return out

    def movy_async(self, d_y32, n, shift, mode, d_out):
        """MOVY on device tensors: n int32 -> int16 (INT16) or int32 (PAIRS32)."""
        _dev(d_y32, 4 * n, "movy y32")
        _dev(d_out, (2 if mode == N.MOVY_INT16 else 4) * n, "movy out")
        N.check(N.lib().w4a8_movy_async(self.h, _dptr(d_y32), int(n), int(shift), int(mode),
                                        _dptr(d_out)), "movy_async")

    def movx_async(self, d_src, n, d_x8):
        """MOVX's data move on device buffers: n int8 values held in int16
        words -> the x window (tail to a 4-byte word zeroed)."""
        _dev(d_src, 2 * n, "movx source")
        _dev(d_x8, (n + 3) // 4 * 4, "movx x window")
        N.check(N.lib().w4a8_movx_async(self.h, _dptr(d_src), int(n), _dptr(d_x8)),
                "movx_async")

    def alu(self, op, y32, p0, b=None):
        y = np.ascontiguousarray(np.asarray(y32, dtype=np.int32).reshape(-1))
        bb = None if b is None else np.ascontiguousarray(np.asarray(b, dtype=np.int16))
        out = np.empty(y.size, dtype=np.int32 if op == N.ALU_SHIFT32W else np.int16)
        N.check(N.lib().w4a8_alu(self.h, int(op), _ptr(y),
                                 None if bb is None else _ptr(bb), y.size, int(p0),
                                 _ptr(out)), f"alu op {op}")
        return out

    # ------------------------------------------------------- matvec (host)
    def matvec_y32(self, w, x8):
        x = np.ascontiguousarray(np.asarray(x8, dtype=np.int8))
        assert x.size == w.K, "x8 length"
        y = np.empty(w.nrows, dtype=np.int32)
        N.check(N.lib().w4a8_matvec_y32(self.h, w.h, _ptr(x), _ptr(y)), "matvec_y32")
        return y

    def matvec_fused(self, w, x, prologue=N.PRO_X8, epilogue=N.EPI_Y32, p0=0,
                     e_x=0, norm_w=None, in_f=0, one_plus=False):
        """Returns (out, x8, e_x, xn) -- xn only for the RMSNorm prologue."""
        xdt = np.int8 if prologue == N.PRO_X8 else np.int16
        xa = np.ascontiguousarray(np.asarray(x, dtype=xdt))
        assert xa.size == w.K, "x length"
        nw = None
        if prologue == N.PRO_RMSNORM_DYNQ8:
            nw = np.ascontiguousarray(np.asarray(norm_w, dtype=np.int16))
            assert nw.size == w.K
        odt = {N.EPI_Y32: np.int32, N.EPI_MOVY_I16: np.int16, N.EPI_MOVY_P32: np.int32,
               N.EPI_SILU32: np.int16, N.EPI_SHIFT_I64: np.int64}[epilogue]
        out = np.empty(w.nrows, dtype=odt)
        x8 = np.empty(w.K, dtype=np.int8)
        xn = np.empty(w.K, dtype=np.int16)
        ex = ctypes.c_int32(int(e_x))
        N.check(N.lib().w4a8_matvec_fused(
            self.h, w.h, int(prologue), _ptr(xa), None if nw is None else _ptr(nw),
            int(in_f), 1 if one_plus else 0, int(epilogue), int(p0), _ptr(out),
            _ptr(x8), ctypes.byref(ex), _ptr(xn)), "matvec")
        return out, x8, int(ex.value), (xn if prologue == N.PRO_RMSNORM_DYNQ8 else None)

    def head_argmax(self, w, x, prologue=N.PRO_X8, norm_w=None, in_f=0,
                    one_plus=False):
        xdt = np.int8 if prologue == N.PRO_X8 else np.int16
        xa = np.ascontiguousarray(np.asarray(x, dtype=xdt))
        assert xa.size == w.K
        nw = None if norm_w is None else np.ascontiguousarray(np.asarray(norm_w, np.int16))
        idx, val = ctypes.c_int32(), ctypes.c_int32()
        N.check(N.lib().w4a8_head_argmax(
            self.h, w.h, int(prologue), _ptr(xa), None if nw is None else _ptr(nw),
            int(in_f), 1 if one_plus else 0, ctypes.byref(idx), ctypes.byref(val)),
            "head_argmax")
        return int(idx.value), int(val.value)

    def topk32(self, y32):
        """TOPK-32 of an int32 vector (one fresh scan): (vals, rows, count,
        overflow), vals / rows int64[count]."""
        y = np.ascontiguousarray(np.asarray(y32, dtype=np.int32).reshape(-1))
        vals, rows = np.zeros(32, np.int32), np.zeros(32, np.int32)
        cnt, ovf = ctypes.c_int32(), ctypes.c_int32()
        N.check(N.lib().w4a8_topk32(self.h, _ptr(y), y.size, _ptr(vals), _ptr(rows),
                                    ctypes.byref(cnt), ctypes.byref(ovf)), "topk32")
        n = int(cnt.value)
        return vals[:n].astype(np.int64), rows[:n].astype(np.int64), n, bool(ovf.value)

    def head_topk32(self, w, x, prologue=N.PRO_X8, norm_w=None, in_f=0, one_plus=False):
        """The head's matvec, then TOPK-32 of its raw y32."""
        xa = np.ascontiguousarray(x, dtype=np.int8 if prologue == N.PRO_X8 else np.int16)
        nw = None if norm_w is None else np.ascontiguousarray(np.asarray(norm_w, np.int16))
        vals, rows = np.zeros(32, np.int32), np.zeros(32, np.int32)
        cnt, ovf = ctypes.c_int32(), ctypes.c_int32()
        N.check(N.lib().w4a8_head_topk32(
            self.h, w.h, int(prologue), _ptr(xa), None if nw is None else _ptr(nw),
            int(in_f), 1 if one_plus else 0, _ptr(vals), _ptr(rows), ctypes.byref(cnt),
            ctypes.byref(ovf)), "head_topk32")
        n = int(cnt.value)
        return vals[:n].astype(np.int64), rows[:n].astype(np.int64), n, bool(ovf.value)

    def head_topk32_async(self, w, x, out, prologue=N.PRO_DYNQ8, e_x=0, norm_w=None,
                          in_f=0, one_plus=False):
        _dev(x, _x_bytes(prologue, w.K), "x")
        _dev(norm_w, 2 * w.K, "norm_w", required=False)
        _dev(out, 66 * 4, "out")
        N.check(N.lib().w4a8_head_topk32_async(
            self.h, w.h, int(prologue), _dptr(x), _dptr(norm_w), int(in_f),
            1 if one_plus else 0, int(e_x), _dptr(out)), "head_topk32")

    def head_topk32_noalloc_async(self, w, x, out, prologue=N.PRO_DYNQ8, e_x=0, norm_w=None,
                                  in_f=0, one_plus=False):
        """head_topk32_async without any device allocation: the y32 and the
        lists live in the library's static per-GPU array (heads of at most
        2^18 rows); calls that overlap on one GPU race."""
        _dev(x, _x_bytes(prologue, w.K), "x")
        _dev(norm_w, 2 * w.K, "norm_w", required=False)
        _dev(out, 66 * 4, "out")
        N.check(N.lib().w4a8_head_topk32_noalloc_async(
            self.h, w.h, int(prologue), _dptr(x), _dptr(norm_w), int(in_f),
            1 if one_plus else 0, int(e_x), _dptr(out)), "head_topk32_noalloc")

    def matmul_y32(self, w, x8):
        x = np.ascontiguousarray(np.asarray(x8, dtype=np.int8))
        assert x.ndim == 2 and x.shape[1] == w.K
        y = np.empty((x.shape[0], w.nrows), dtype=np.int32)
        N.check(N.lib().w4a8_matmul_y32(self.h, w.h, _ptr(x), x.shape[0], _ptr(y)),
                "matmul_y32")
        return y

    # ------------------------------------------------------ device (async)
    def site_async(self, weights, epilogues, p0s, outs, x, prologue=N.PRO_DYNQ8,
                   e_x=0, norm_w=None, in_f=0, one_plus=False, x8_out=None,
                   e_x_out=None, xn_out=None):
        n = len(weights)
        if not (n == len(epilogues) == len(p0s) == len(outs)):
            raise ValueError("site: one epilogue, p0 and output per matrix")
        K = weights[0].K
        for w, e, o in zip(weights, epilogues, outs):
            _dev(o, _EPI_BYTES.get(int(e), 8) * w.nrows, "site output")
        _dev(x, _x_bytes(prologue, K), "x")
        _dev(norm_w, 2 * K, "norm_w", required=False)
        _dev(x8_out, K, "x8_out", required=False)
        _dev(e_x_out, 4, "e_x_out", required=False)
        _dev(xn_out, 2 * K, "xn_out", required=False)
        wa = (ctypes.c_void_p * n)(*[w.h.value for w in weights])
        oa = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
        ea = np.ascontiguousarray(epilogues, dtype=np.int32)
        pa = np.ascontiguousarray(p0s, dtype=np.int32)
        N.check(N.lib().w4a8_site_async(
            self.h, n, wa, _ptr(ea), _ptr(pa), oa, int(prologue), _dptr(x),
            _dptr(norm_w), int(in_f), 1 if one_plus else 0, int(e_x), _dptr(x8_out),
            _dptr(e_x_out), _dptr(xn_out)), "site")

    def head_argmax_async(self, w, x, result, prologue=N.PRO_DYNQ8, e_x=0,
                          norm_w=None, in_f=0, one_plus=False):
        _dev(x, _x_bytes(prologue, w.K), "x")
        _dev(norm_w, 2 * w.K, "norm_w", required=False)
        _dev(result, 8, "result")
        N.check(N.lib().w4a8_head_argmax_async(
            self.h, w.h, int(prologue), _dptr(x), _dptr(norm_w), int(in_f),
            1 if one_plus else 0, int(e_x), _dptr(result)), "head_argmax")

    def matmul_async(self, w, x8, y32):
        B = x8.shape[0]
        _dev(x8, B * w.K, "x8")
        _dev(y32, 4 * B * w.nrows, "y32")
        N.check(N.lib().w4a8_matmul_y32_async(self.h, w.h, _dptr(x8), x8.shape[0],
                                              _dptr(y32)), "matmul")

    def matmul_multi_async(self, weights, x8s, y32s):
        """Several matrices for the same B tokens in one launch (device
        tensors x8s[i] [B][K_i], y32s[i] [B][nrows_i])."""
        n = len(weights)
        if not n == len(x8s) == len(y32s):
            raise ValueError("matmul_multi: one x8 and one y32 per matrix")
        B = x8s[0].shape[0]
        for w, x, y in zip(weights, x8s, y32s):
            if x.shape[0] != B or y.shape[0] != B:
                raise ValueError("matmul_multi: every x8 and y32 holds the same B tokens")
            _dev(x, B * w.K, "x8")
            _dev(y, 4 * B * w.nrows, "y32")
        wa = (ctypes.c_void_p * n)(*[w.h.value for w in weights])
        xa = (ctypes.c_void_p * n)(*[x.data_ptr() for x in x8s])
        ya = (ctypes.c_void_p * n)(*[y.data_ptr() for y in y32s])
        N.check(N.lib().w4a8_matmul_y32_multi_async(self.h, n, wa, xa, B, ya), "matmul_multi")

    def mlp_async(self, gate, up, down, p0s, x16, norm_w=None, in_f=0, one_plus=False,
                  mlp_out=None, res_out=None):
        """The SwiGLU block on device tensors (w4a8_mlp_async): optional
        RMSNorm, gate / up, EMUL32, down; mlp_out = int16[H] block output,
        res_out = clip16(x16 + mlp_out) (may be x16 itself)."""
        pg, pu, pd = (int(p) for p in p0s)
        H = gate.K
        _dev(x16, 2 * H, "x16")
        _dev(norm_w, 2 * H, "norm_w", required=False)
        _dev(mlp_out, 2 * H, "mlp_out", required=False)
        _dev(res_out, 2 * H, "res_out", required=False)
        N.check(N.lib().w4a8_mlp_async(
            self.h, gate.h, up.h, down.h, pg, pu, pd, _dptr(x16), _dptr(norm_w),
            int(in_f), 1 if one_plus else 0, _dptr(mlp_out), _dptr(res_out)), "mlp")


_DEFAULT = None


def default_context():
    """Process-wide context on device 0, for the reference-named functions."""
    global _DEFAULT
    if _DEFAULT is None or _DEFAULT.h is None:
        _DEFAULT = Context(0)
    return _DEFAULT


class Plan:
    """A fixed sequence of sites (matrices sharing one input vector) and LM
    heads, replayed as one HIP graph with the site order kept.  Holds
    references to every device tensor it was given."""

    def __init__(self, ctx):
        self.ctx = ctx
        h = ctypes.c_void_p()
        N.check(N.lib().w4a8_plan_create(ctx.h, ctypes.byref(h)), "plan_create")
        self.h = h
        self._keep = []
        self.bytes = 0        # algorithmic weight bytes per replay
        self.nsites = 0
        self.nmats = 0

    def add_site(self, weights, epilogues, p0s, outs, x, prologue=N.PRO_DYNQ8,
                 e_x=0, norm_w=None, in_f=0, one_plus=False, x8_out=None,
                 e_x_out=None, xn_out=None):
        n = len(weights)
        if not (n == len(epilogues) == len(p0s) == len(outs)):
            raise ValueError("site: one epilogue, p0 and output per matrix")
        K = weights[0].K
        for w, e, o in zip(weights, epilogues, outs):
            _dev(o, _EPI_BYTES.get(int(e), 8) * w.nrows, "site output")
        _dev(x, _x_bytes(prologue, K), "x")
        _dev(norm_w, 2 * K, "norm_w", required=False)
        _dev(x8_out, K, "x8_out", required=False)
        _dev(e_x_out, 4, "e_x_out", required=False)
        _dev(xn_out, 2 * K, "xn_out", required=False)
        wa = (ctypes.c_void_p * n)(*[w.h.value for w in weights])
        oa = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
        ea = np.ascontiguousarray(epilogues, dtype=np.int32)
        pa = np.ascontiguousarray(p0s, dtype=np.int32)
        N.check(N.lib().w4a8_plan_add_site(
            self.h, n, wa, _ptr(ea), _ptr(pa), oa, int(prologue), _dptr(x),
            _dptr(norm_w), int(in_f), 1 if one_plus else 0, int(e_x),
            _dptr(x8_out), _dptr(e_x_out), _dptr(xn_out)), "plan_add_site")
        self._keep += [weights, outs, x, norm_w, x8_out, e_x_out, xn_out]
        self.bytes += sum(w.wire_bytes for w in weights)
        self.nsites += 1
        self.nmats += n

    def add_site_emul(self, weights, epilogues, p0s, outs, x, x2, x8_out=None,
                      e_x_out=None):
        """The SwiGLU product site: DYNQ8(EMUL32(x2, x; 12)) with x the
        gate's SILU32 output (int16) and x2 the up projection's (int32),
        then the site's matrices (the down projection)."""
        n = len(weights)
        if not (n == len(epilogues) == len(p0s) == len(outs)):
            raise ValueError("site: one epilogue, p0 and output per matrix")
        K = weights[0].K
        for w, e, o in zip(weights, epilogues, outs):
            _dev(o, _EPI_BYTES.get(int(e), 8) * w.nrows, "site output")
        _dev(x, 2 * K, "x")
        _dev(x2, 4 * K, "x2")
        _dev(x8_out, K, "x8_out", required=False)
        _dev(e_x_out, 4, "e_x_out", required=False)
        wa = (ctypes.c_void_p * n)(*[w.h.value for w in weights])
        oa = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
        ea = np.ascontiguousarray(epilogues, dtype=np.int32)
        pa = np.ascontiguousarray(p0s, dtype=np.int32)
        N.check(N.lib().w4a8_plan_add_site_emul(
            self.h, n, wa, _ptr(ea), _ptr(pa), oa, _dptr(x), _dptr(x2),
            _dptr(x8_out), _dptr(e_x_out)), "plan_add_site_emul")
        self._keep += [weights, outs, x, x2, x8_out, e_x_out]
        self.bytes += sum(w.wire_bytes for w in weights)
        self.nsites += 1
        self.nmats += n

    def add_site_emul_res(self, down, p0, x, x2, res, res_out, out=None):
        """The SwiGLU product site with the block's residual ADD: down over
        DYNQ8(EMUL32(x2, x; 12)), MOVY int16 at p0 into out (optional) and
        clip16(res + that) into res_out."""
        H = down.nrows
        _dev(x, 2 * down.K, "x")
        _dev(x2, 4 * down.K, "x2")
        _dev(res, 2 * H, "res")
        _dev(res_out, 2 * H, "res_out")
        _dev(out, 2 * H, "out", required=False)
        N.check(N.lib().w4a8_plan_add_site_emul_res(
            self.h, down.h, int(p0), _dptr(out), _dptr(x), _dptr(x2), _dptr(res),
            _dptr(res_out)), "plan_add_site_emul_res")
        self._keep += [down, x, x2, res, res_out, out]
        self.bytes += down.wire_bytes
        self.nsites += 1
        self.nmats += 1

    def add_mlp(self, gate, up, down, p0s, x16, norm_w=None, in_f=0, one_plus=False,
                mlp_out=None, res_out=None):
        """A layer's FFN block as two sites (the arguments of
        Context.mlp_async); its temporaries belong to the plan."""
        pg, pu, pd = (int(p) for p in p0s)
        H = gate.K
        _dev(x16, 2 * H, "x16")
        _dev(norm_w, 2 * H, "norm_w", required=False)
        _dev(mlp_out, 2 * H, "mlp_out", required=False)
        _dev(res_out, 2 * H, "res_out", required=False)
        N.check(N.lib().w4a8_plan_add_mlp(
            self.h, gate.h, up.h, down.h, pg, pu, pd, _dptr(x16), _dptr(norm_w), int(in_f),
            1 if one_plus else 0, _dptr(mlp_out), _dptr(res_out)), "plan_add_mlp")
        self._keep += [gate, up, down, x16, norm_w, mlp_out, res_out]
        self.bytes += gate.wire_bytes + up.wire_bytes + down.wire_bytes
        self.nsites += 2
        self.nmats += 3

    def add_head(self, w, x, result, prologue=N.PRO_DYNQ8, e_x=0, norm_w=None,
                 in_f=0, one_plus=False):
        _dev(x, _x_bytes(prologue, w.K), "x")
        _dev(norm_w, 2 * w.K, "norm_w", required=False)
        _dev(result, 8, "result")
        N.check(N.lib().w4a8_plan_add_head(
            self.h, w.h, int(prologue), _dptr(x), _dptr(norm_w), int(in_f),
            1 if one_plus else 0, int(e_x), _dptr(result)), "plan_add_head")
        self._keep += [w, x, result, norm_w]
        self.bytes += w.wire_bytes
        self.nsites += 1
        self.nmats += 1

    def add_head_topk32(self, w, x, out, prologue=N.PRO_DYNQ8, e_x=0, norm_w=None,
                        in_f=0, one_plus=False):
        """The LM head ending in TOPK-32 (docs/SEQ_ISA.md B8): out (66 int32)
        gets vals[32], rows[32], count, overflow.  One per plan, its last
        step in a persistent plan, where the scan runs in the same launch."""
        _dev(x, _x_bytes(prologue, w.K), "x")
        _dev(norm_w, 2 * w.K, "norm_w", required=False)
        _dev(out, 66 * 4, "out")
        N.check(N.lib().w4a8_plan_add_head_topk32(
            self.h, w.h, int(prologue), _dptr(x), _dptr(norm_w), int(in_f),
            1 if one_plus else 0, int(e_x), _dptr(out)), "plan_add_head_topk32")
        self._keep += [w, x, out, norm_w]
        self.bytes += w.wire_bytes
        self.nsites += 1
        self.nmats += 1

    def set_mode(self, mode):
        N.check(N.lib().w4a8_plan_set_mode(self.h, int(mode)), "plan_set_mode")

    def set_fences(self, fences):
        """Persistent mode: FENCE_ALL (every site waits for all earlier ones)
        or FENCE_AUTO (only where a site shares a buffer with an earlier
        one); results are the same either way."""
        N.check(N.lib().w4a8_plan_set_fences(self.h, int(fences)), "plan_set_fences")

    def fenced(self):
        """Per site, how a persistent replay orders it (under the current
        fence mode): N.WAIT_NONE, N.WAIT_GRID (every earlier site on every
        workgroup) or N.WAIT_INPUT (the one earlier output it reads, through
        that output's stamped words)."""
        f = np.zeros(self.nsites, dtype=np.int32)
        N.check(N.lib().w4a8_plan_fences(self.h, self.nsites, _ptr(f)), "plan_fences")
        return [int(v) for v in f]

    def run(self):
        N.check(N.lib().w4a8_plan_run(self.h), "plan_run")

    def profile(self):
        """Per-step GEMV kernel times in ms (one eager, instrumented pass)."""
        ms = np.zeros(self.nsites, dtype=np.float32)
        N.check(N.lib().w4a8_plan_profile(self.h, self.nsites, _ptr(ms)), "plan_profile")
        return ms

    def time_launches(self, n):
        """Kernel ms of each of n back-to-back replays of a persistent plan
        (dispatch-recorded events)."""
        ms = np.zeros(n, dtype=np.float32)
        N.check(N.lib().w4a8_plan_time_launches(self.h, n, _ptr(ms)), "plan_time_launches")
        return ms

    def close(self):
        if self.h:
            N.lib().w4a8_plan_destroy(self.h)
            self.h = None


class MatmulPlan:
    """Up to 128 matrices for the same B tokens run as ONE batched int8-MFMA
    launch per run (device tensors x8 [B][K], y32 [B][nrows] per matrix).
    The first run after an add writes the plan's device table; run it once
    before capturing it into a graph.  Holds references to its tensors."""

    def __init__(self, ctx, B):
        self.ctx, self.B = ctx, int(B)
        h = ctypes.c_void_p()
        N.check(N.lib().w4a8_mplan_create(ctx.h, self.B, ctypes.byref(h)), "mplan_create")
        self.h = h
        self._keep = []
        self.bytes = 0        # algorithmic weight bytes per run
        self.nmats = 0

    def add(self, w, x8, y32):
        if x8.shape[0] != self.B or y32.shape[0] != self.B:
            raise ValueError(f"matmul plan: x8 and y32 hold the plan's {self.B} tokens")
        _dev(x8, self.B * w.K, "x8")
        _dev(y32, 4 * self.B * w.nrows, "y32")
        N.check(N.lib().w4a8_mplan_add(self.h, w.h, _dptr(x8), _dptr(y32)), "mplan_add")
        self._keep += [w, x8, y32]
        self.bytes += w.wire_bytes
        self.nmats += 1

    def run(self):
        N.check(N.lib().w4a8_mplan_run(self.h), "mplan_run")

    def close(self):
        if self.h:
            N.lib().w4a8_mplan_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()
