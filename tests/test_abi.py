"""The C ABI library: builds, loads, and exports every symbol include/mimo_moe.h declares (CPU only)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mimo_moe.h")


def declared_symbols():
    text = open(HEADER).read()
    decl = r"^(?:int|size_t|const char\*)\s+(mimo_[a-z0-9_]+)\s*\("
    return sorted(set(re.findall(decl, text, flags=re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("mimo_moe_decode", "mimo_moe_prefill", "mimo_router", "mimo_group_routes", "mimo_quantize_mxfp4"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    from mimo_stream import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libmimo_moe.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for s in declared_symbols():
        assert hasattr(lib, s), s
    assert set(declared_symbols()) == set(_lib.SIGNATURES), "ctypes signatures must cover the header exactly"
    assert _lib.load().mimo_abi_version() == _lib.ABI_VERSION


def test_workspace_size_queries_need_no_gpu():
    from mimo_stream import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libmimo_moe.so not built")
    lib = _lib.load()
    assert lib.mimo_moe_decode_workspace_size(1, 256, 8, 4096, 2048) > 0
    assert lib.mimo_moe_prefill_workspace_size(2048, 8, 256, 4096, 2048) > 2048 * 8 * 4096 * 2


def test_argument_errors_are_reported_without_a_gpu():
    from mimo_stream import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libmimo_moe.so not built")
    lib = _lib.load()
    # null pointers and bad shapes are rejected on the host before any HIP call
    assert lib.mimo_quantize_mxfp4(None, 1, 32, None, None, None) == _lib.ERR_ARG
    assert "null" in lib.mimo_last_error().decode()
    with pytest.raises(ValueError):
        _lib.check(lib.mimo_router_select(None, None, 1, 8, 2, 1.0, None, None, None), "router_select")
