"""ctypes binding of libfable5_w4a8.so (the C ABI in include/fable5_w4a8.h).

There is no CPU fallback: if the HIP library is missing this module raises,
and every compute call goes through the HIP kernels.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfable5_w4a8.so")

OK = 0
E_SHAPE, E_ENVELOPE, E_ACC_OVF, E_Y32_OVF, E_HIP, E_ARG, E_RANGE = \
    -1, -2, -3, -4, -5, -6, -7

PRO_X8, PRO_DYNQ8, PRO_RMSNORM_DYNQ8, PRO_EMUL_DYNQ8 = 0, 1, 2, 3
EPI_Y32, EPI_MOVY_I16, EPI_MOVY_P32, EPI_SILU32, EPI_SHIFT_I64 = 0, 1, 2, 3, 4
ALU_SHIFT32, ALU_SILU32, ALU_EMUL32, ALU_SHIFT32W = 1, 6, 8, 9
MOVY_PAIRS32, MOVY_INT16 = 0, 1
PLAN_GRAPH, PLAN_PERSISTENT, PLAN_PERSISTENT_COOP = 0, 1, 2
FENCE_ALL, FENCE_AUTO = 0, 1
WAIT_NONE, WAIT_GRID, WAIT_INPUT = 0, 1, 2   # w4a8_plan_fences

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_PP = ctypes.POINTER(ctypes.c_void_p)

# name -> argtypes (every entry point returns int except the two char* ones)
SIGNATURES = {
    "w4a8_ctx_create": [_I32, ctypes.POINTER(_P)],
    "w4a8_ctx_destroy": [_P],
    "w4a8_ctx_set_stream": [_P, _P],
    "w4a8_ctx_sync": [_P],
    "w4a8_ctx_info": [_P, _P, _P],
    "w4a8_ctx_set_grid": [_P, _I32],
    "w4a8_ctx_set_spin_limit": [_P, ctypes.c_uint32, ctypes.c_uint32],
    "w4a8_tables": [_P, _P, _P],
    "w4a8_read_ceiling": [_P, _P, _I64, _I32, _I32, _P],
    "w4a8_weights_upload": [_P, _P, _I64, _I32, _I32, ctypes.POINTER(_P)],
    "w4a8_weights_upload_async": [_P, _P, _I64, _I32, _I32, ctypes.POINTER(_P)],
    "w4a8_weights_download": [_P, _P, _P],
    "w4a8_weights_info": [_P, _P, _P, _P, _P],
    "w4a8_weights_free": [_P],
    "w4a8_rshift_round": [_P, _P, _I64, _I32, _P],
    "w4a8_dynq8": [_P, _P, _I32, _P, _P],
    "w4a8_rmsnorm": [_P, _P, _P, _I32, _I32, _I32, _P],
    "w4a8_movy": [_P, _P, _I64, _I32, _I32, _P],
    "w4a8_movy_async": [_P, _P, _I64, _I32, _I32, _P],
    "w4a8_movx_async": [_P, _P, _I64, _P],
    "w4a8_alu": [_P, _I32, _P, _P, _I64, _I32, _P],
    "w4a8_matvec_y32": [_P, _P, _P, _P],
    "w4a8_matvec_fused": [_P, _P, _I32, _P, _P, _I32, _I32, _I32, _I32, _P, _P,
                          _P, _P],
    "w4a8_head_argmax": [_P, _P, _I32, _P, _P, _I32, _I32, _P, _P],
    "w4a8_matmul_y32": [_P, _P, _P, _I32, _P],
    "w4a8_matvec_fused_async": [_P, _P, _I32, _P, _P, _I32, _I32, _I32, _I32,
                                _I32, _P, _P, _P, _P],
    "w4a8_site_async": [_P, _I32, _PP, _P, _P, _PP, _I32, _P, _P, _I32, _I32,
                        _I32, _P, _P, _P],
    "w4a8_head_argmax_async": [_P, _P, _I32, _P, _P, _I32, _I32, _I32, _P],
    "w4a8_matmul_y32_async": [_P, _P, _P, _I32, _P],
    "w4a8_matmul_y32_multi_async": [_P, _I32, _P, _P, _I32, _P],
    "w4a8_mplan_create": [_P, _I32, ctypes.POINTER(_P)],
    "w4a8_mplan_add": [_P, _P, _P, _P],
    "w4a8_mplan_run": [_P],
    "w4a8_mplan_destroy": [_P],
    "w4a8_topk32": [_P, _P, _I64, _P, _P, _P, _P],
    "w4a8_head_topk32": [_P, _P, _I32, _P, _P, _I32, _I32, _P, _P, _P, _P],
    "w4a8_head_topk32_async": [_P, _P, _I32, _P, _P, _I32, _I32, _I32, _P],
    "w4a8_head_topk32_noalloc_async": [_P, _P, _I32, _P, _P, _I32, _I32, _I32, _P],
    "w4a8_mlp_async": [_P, _P, _P, _P, _I32, _I32, _I32, _P, _P, _I32, _I32, _P, _P],
    "w4a8_plan_create": [_P, ctypes.POINTER(_P)],
    "w4a8_plan_add_site": [_P, _I32, _PP, _P, _P, _PP, _I32, _P, _P, _I32, _I32,
                           _I32, _P, _P, _P],
    "w4a8_plan_add_site_emul": [_P, _I32, _PP, _P, _P, _PP, _P, _P, _P, _P],
    "w4a8_plan_add_site_emul_res": [_P, _P, _I32, _P, _P, _P, _P, _P],
    "w4a8_plan_add_mlp": [_P, _P, _P, _P, _I32, _I32, _I32, _P, _P, _I32, _I32, _P, _P],
    "w4a8_plan_add_head": [_P, _P, _I32, _P, _P, _I32, _I32, _I32, _P],
    "w4a8_plan_add_head_topk32": [_P, _P, _I32, _P, _P, _I32, _I32, _I32, _P],
    "w4a8_plan_set_mode": [_P, _I32],
    "w4a8_plan_set_fences": [_P, _I32],
    "w4a8_plan_fences": [_P, _I32, _P],
    "w4a8_plan_run": [_P],
    "w4a8_plan_profile": [_P, _I32, _P],
    "w4a8_plan_time_launches": [_P, _I32, _P],
    "w4a8_plan_destroy": [_P],
}
STRING_FUNCS = ("w4a8_version", "w4a8_last_error")

_LIB = None


def lib():
    """Load the HIP engine; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        # One HIP runtime per process.  PyTorch-ROCm ships its own
        # libamdhip64 (soname libamdhip64.so.7) and loads it by the
        # unversioned name; loaded first, it also satisfies this library's
        # libamdhip64.so.7 dependency, so torch tensors, streams and this
        # engine share one runtime.  Loaded the other way round, torch
        # would bring up a second runtime that sees no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: the W4A8 engine is a HIP library "
                "with no CPU fallback; build it with "
                "`python -m fable5_llm_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = ctypes.c_int
        for name in STRING_FUNCS:
            f = getattr(L, name)
            f.argtypes = []
            f.restype = ctypes.c_char_p
        _LIB = L
    return _LIB


def last_error():
    return lib().w4a8_last_error().decode("utf-8", "replace")


def check(rc, what=""):
    """Map a status code to the reference's exception classes: the law's
    own conditions are AssertionErrors (w4a8_ref.py asserts), bad
    arguments ValueError, device failures RuntimeError."""
    if rc == OK:
        return
    msg = last_error()
    if what:
        msg = f"{what}: {msg}"
    if rc in (E_SHAPE, E_ENVELOPE, E_ACC_OVF, E_Y32_OVF, E_RANGE):
        raise AssertionError(msg)
    if rc == E_ARG:
        raise ValueError(msg)
    raise RuntimeError(msg)
