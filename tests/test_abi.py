"""The C-ABI library loads and exports every entry point include/vlrf_hip.h
declares; argument errors are reported without a device.  No GPU compute."""
import ctypes as C
import os
import re

import pytest

import vlrf_amd as V
from vlrf_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vlrf_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vlrf_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared()
    assert len(names) >= 40
    lib = C.CDLL(_lib.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_only_binds_declared_symbols():
    assert set(_lib._SIGS) <= set(declared())


def test_host_helpers_reject_bad_sizes():
    import numpy as np
    x = np.zeros(33, np.float32)
    out = np.zeros(64, np.uint8)
    assert V.lib().vlrf_quantize_q8_0(x.ctypes.data, out.ctypes.data, 33) == _lib.ERR_ARG
    assert V.lib().vlrf_dequantize(out.ctypes.data, 5, x.ctypes.data, 32) == _lib.ERR_ARG


def test_init_without_a_device_reports_nodev():
    if V.lib().vlrf_hip_device_count() > 0:
        pytest.skip("a GPU is visible: covered by the gpu tests")
    h = C.c_void_p()
    rc = V.lib().vlrf_hip_init(0, C.byref(h))
    assert rc in (_lib.ERR_NODEV, _lib.ERR_RUNTIME)
    assert h.value is None
    assert _lib.last_error()
