"""CPU: the C-ABI library loads and exports every entry point include/loki_moe.h declares (no compute calls)."""
import ctypes
import os
import re

import loki_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "loki_moe.h")
REF_NAMES = ["fl_init", "fl_attn", "fl_wide_init", "fl_wide_moe", "fl_wide_mark", "fl_wide_wait", "fl_wide_finish",
             "fl_moe_outs", "fl_wide_outs", "fl_wide_skip", "fl_spec", "fl_sketch", "fl_fetch", "fl_moe", "fl_skip",
             "fl_h2d", "fl_wait_event", "fl_gpu_ms"]   # the 18 functions of the reference's src/fused_layer.h


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(fl_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_reference_surface():
    d = declared()
    for n in REF_NAMES:
        assert n in d, n


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(loki_amd.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_list_matches_header():
    assert sorted(set(loki_amd.ABI_SYMBOLS)) == declared()


def test_struct_layouts_match_reference():
    # FLW: 18 pointers + 2 ints; FLOut: 11 pointers (src/fused_layer.h:12-21)
    P = ctypes.sizeof(ctypes.c_void_p)
    assert ctypes.sizeof(loki_amd.FLW) == 18 * P + 8
    assert ctypes.sizeof(loki_amd.FLOut) == 11 * P
    assert ctypes.sizeof(loki_amd.FLMoeLayer) == 8 * P + 16


def test_no_cpu_fallback(monkeypatch):
    # the product path fails loudly without the built library
    monkeypatch.setattr(loki_amd, "LIB_PATH", "/nonexistent/libloki_moe.so")
    monkeypatch.setattr(loki_amd, "_lib", None)
    try:
        loki_amd.lib()
    except loki_amd.LokiError as e:
        assert "not built" in str(e)
    else:
        raise AssertionError("lib() must raise when the library is missing")
