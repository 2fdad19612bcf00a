"""The C-ABI library builds for gfx950, loads, and exports every entry point
include/fable5_w4a8.h declares (no GPU needed: nothing is computed)."""
import ctypes
import os
import re

import pytest

from fable5_llm_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "fable5_w4a8.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(w4a8_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(_native.LIB_PATH)
    names = header_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_header():
    names = set(header_functions())
    bound = set(_native.SIGNATURES) | set(_native.STRING_FUNCS)
    assert names == bound, (names - bound, bound - names)


def test_version_string():
    assert b"gfx950" in _native.lib().w4a8_version()


def test_library_holds_gfx950_code():
    data = open(_native.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def test_status_codes_match_header():
    text = open(os.path.join(ROOT, "include", "fable5_w4a8.h")).read()
    codes = dict((k, int(v)) for k, v in
                 re.findall(r"#define W4A8_(E_[A-Z0-9_]+)\s+\((-\d+)\)", text))
    for k, v in codes.items():
        assert getattr(_native, k) == v, k


def test_single_hip_runtime_in_process():
    """Loading the engine maps exactly one HIP and one HSA runtime (torch's,
    when torch is installed), so torch tensors/streams are valid handles."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r)\n"
            "from fable5_llm_amd import _native; _native.lib()\n"
            "m = open('/proc/self/maps').read().splitlines()\n"
            "print(len(set(l.split()[-1] for l in m if 'libamdhip64' in l)),"
            " len(set(l.split()[-1] for l in m if 'libhsa-runtime64' in l)))" % ROOT)
    out = subprocess.run([sys.executable, "-c", code], capture_output=True,
                         text=True, timeout=120).stdout.split()
    assert out == ["1", "1"], out


def test_device_wrappers_refuse_short_buffers():
    # the wrappers check device tensors before a raw pointer reaches C (no
    # GPU needed: the checks run first, and CPU tensors are refused)
    import torch
    from fable5_llm_amd import engine as E
    with pytest.raises(ValueError, match="required"):
        E._dev(None, 4, "x")
    E._dev(None, 4, "x", required=False)
    with pytest.raises(ValueError, match="device tensor"):
        E._dev(torch.zeros(4, dtype=torch.int32), 16, "x")
