"""CPU checks of the native boundary: the built libraries load and export every
function that include/*.h declares (no device calls)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    src = open(os.path.join(ROOT, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(cpi_[a-z0-9_]+)\s*\(", src)))


def exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True, text=True, check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if l.strip()}


@pytest.mark.parametrize("header,lib", [("cpi_hip.h", "libcpi_hip.so"), ("cpi_engine.h", "libcpi_engine.so")])
def test_exports_match_header(header, lib):
    path = os.path.join(ROOT, "cpi_amd", lib)
    if not os.path.exists(path):
        pytest.skip(f"{lib} not built")
    names = declared(header)
    assert len(names) > 5
    missing = [n for n in names if n not in exported(path)]
    assert not missing, missing
    ctypes.CDLL(path)  # loads without a GPU


def test_python_binding_covers_header():
    from cpi_amd import _lib
    names = declared("cpi_hip.h")
    assert set(names) == set(_lib.declared_symbols())


def test_host_helpers_without_gpu():
    from cpi_amd import _lib
    import numpy as np
    L = _lib.lib()
    order = np.zeros((8 + 2) * 64, np.int32)
    assert L.cpi_hip_qkv_row_order(8, 1, 64, order.ctypes.data_as(ctypes.POINTER(ctypes.c_int))) == 0
    assert sorted(order) == list(range(order.size))
    # rope tables follow theta^(-2d/hd)
    c = np.zeros((4, 32), np.float32)
    s = np.zeros_like(c)
    assert L.cpi_rope_tables(4, 64, 10000.0, c.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p)) == 0
    ang = 3 * 10000.0 ** (-2 * np.arange(32) / 64)
    np.testing.assert_allclose(c[3], np.cos(ang), atol=1e-6)
    assert L.cpi_hip_swiglu_row_order(6, order.ctypes.data_as(ctypes.POINTER(ctypes.c_int))) != 0  # 6 % 4
