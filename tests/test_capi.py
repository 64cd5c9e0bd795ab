"""The C ABI library loads and exports exactly what include/m3x.h declares (CPU: no kernel is launched)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "m3x.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(int|long|size_t)\s+(m3x_\w+)\s*\(([^)]*)\)\s*;", text):
        args = [a.strip() for a in m.group(3).split(",") if a.strip() and a.strip() != "void"]
        decls[m.group(2)] = len(args)
    return decls


def test_header_declares_entry_points():
    d = _declared()
    assert len(d) >= 20 and "m3x_decode_attn" in d and "m3x_linear" in d


def test_library_exports_every_declared_symbol():
    from m3x import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} not built (run __graft_entry__.build())")
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(raw, name), name


def test_binding_matches_header():
    from m3x import _lib
    d = _declared()
    assert set(_lib.SIGNATURES) == set(d)
    for name, (_, args) in _lib.SIGNATURES.items():
        assert len(args) == d[name], (name, len(args), d[name])


def test_library_loads_and_reports_abi():
    from m3x import _lib
    L = _lib.lib()
    assert L.m3x_version() == _lib.ABI_VERSION


def test_workspace_queries_are_host_only():
    from m3x import ops
    # attention partials: rows x kv heads x splits x (m[2], l[2], pad[4], o[2][128]) fp32
    assert ops.decode_attn_workspace(224, 8, 4096, 1024) == 224 * 8 * 4 * 264 * 4
    assert ops.decode_attn_workspace(0, 8, 4096, 1024) == 0


def test_packed_weight_size_query_is_host_only():
    from m3x._lib import lib
    L = lib()
    assert L.m3x_packed_weight_elems(2049, 1024) == 2064 * 1024  # rows padded to a multiple of 16
    assert L.m3x_packed_weight_elems(16, 32) == 512
    assert L.m3x_packed_weight_elems(16, 48) == -1  # K must be a multiple of 32
