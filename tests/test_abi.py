"""The C-ABI library (infer_amd/libiq.so) loads, exports every symbol that
include/iq.h declares, keeps iq_view byte-compatible with the reference's
gpu::QuantView (kernels/ops/ops.cuh:166-172), and rejects bad arguments on the
host before touching a device (no compute calls: runs without a GPU)."""
import ctypes
import os
import re

import pytest

from infer_amd import ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "iq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(iq_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_are_exported():
    L = ops.lib()
    names = declared_functions()
    assert "iq_gemv" in names and "iq_quantize" in names
    for n in names:
        assert hasattr(L, n), n
    # the Python mirror binds exactly what the header declares
    assert set(names) == set(ops.SIGNATURES)


def test_view_layout_matches_quantview():
    assert ctypes.sizeof(ops.IqView) == 56
    assert ops.IqView.rows.offset == 8
    assert ops.IqView.q.offset == 32
    assert ops.IqView.zeros.offset == 48


def _view(kind=0, rows=64, cols=128, groups=None, q=1, s=1, z=1):
    return ops.IqView(kind, rows, cols, (cols + 127) // 128 if groups is None else groups,
                      q, s, z if kind == 1 else None)


def test_error_codes_without_device():
    L = ops.lib()
    E = {"kind": -1, "shape": -2, "null": -3}
    v = _view(kind=7)
    assert L.iq_gemv(1, ctypes.byref(v), None, 1, 128, 64, 1, None) == E["kind"]
    v = _view()
    assert L.iq_gemv(1, ctypes.byref(v), None, 1, 129, 64, 1, None) == E["shape"]   # in != cols
    assert L.iq_gemv(1, ctypes.byref(v), None, 0, 128, 64, 1, None) == E["shape"]   # B < 1
    assert L.iq_gemv(1, ctypes.byref(v), None, 33, 128, 64, 1, None) == E["shape"]  # B > 32
    assert L.iq_gemv(None, ctypes.byref(v), None, 1, 128, 64, 1, None) == E["null"]
    assert L.iq_gemv(1, None, None, 1, 128, 64, 1, None) == E["null"]
    bad = _view(groups=2)
    assert L.iq_gemm(1, ctypes.byref(bad), None, 40, 128, 64, 1, None) == E["shape"]
    odd = _view(kind=1, cols=129)
    assert L.iq_gemm(1, ctypes.byref(odd), None, 40, 129, 64, 1, None) == E["shape"]
    noz = ops.IqView(1, 64, 128, 1, 1, 1, None)
    assert L.iq_linear(1, ctypes.byref(noz), None, 4, 128, 64, 1, None) == E["null"]
    assert L.iq_quantize(1, 4, 3, 1, 1, 1, 1, None) == E["shape"]   # int4 odd cols
    assert L.iq_quantize(1, 4, 4, 2, 1, 1, 1, None) == E["kind"]
    assert L.iq_quantize(1, 4, 4, 1, 1, 1, None, None) == E["null"]
    assert L.iq_embedding(ctypes.byref(v), 1, 0, 128, 1, None) == E["shape"]
    for code in (0, -1, -2, -3, -4, -5, -6, -99):
        assert L.iq_error_string(code)


def test_python_mirror_raises_on_missing_library(monkeypatch):
    monkeypatch.setattr(ops, "_lib", None)
    monkeypatch.setattr(ops, "LIB_PATH", "/nonexistent/libiq.so")
    with pytest.raises(RuntimeError):
        ops.lib()
