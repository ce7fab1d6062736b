"""The C-ABI backend library on a host without a GPU: libnewt_hip.so loads,
exports every entry point include/newt_hip.h declares, reports its error
strings, and hipRTC compiles for gfx950 (compilation needs no device). No
kernel is launched here; launches are covered by the gpu-marked tests."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "newt_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(newt_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("newt_rtc_compile", "newt_module_load", "newt_module_get_function",
              "newt_launch", "newt_launch_packed", "newt_error_string", "newt_last_error"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    from newt_amd.runtime import hip
    L = hip.lib()
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert not missing, f"libnewt_hip.so lacks {missing}"
    assert L.newt_abi_version() == 1


def test_error_strings():
    from newt_amd.runtime import hip
    L = hip.lib()
    assert L.newt_error_string(0) is not None
    assert b"hipRTC" in L.newt_error_string(10001) or L.newt_error_string(10001)
    assert L.newt_error_string(10002)


def test_rtc_compiles_for_gfx950_without_device():
    from newt_amd.runtime import hip
    src = 'extern "C" __global__ void k(float* p) { p[threadIdx.x] = 1.0f; }'
    code = hip.compile_hip(src, "k")
    assert code[:4] == b"\x7fELF"
    assert hip.rtc_version() > 0


def test_rtc_error_carries_log():
    from newt_amd.runtime import hip
    with pytest.raises(hip.HIPRTCError, match="error"):
        hip.compile_hip('extern "C" __global__ void k() { undeclared_thing(); }', "k")


def test_null_handles_rejected():
    from newt_amd.runtime import hip
    L = hip.lib()
    f = ctypes.c_void_p()
    assert L.newt_module_get_function(None, b"k", ctypes.byref(f)) != 0
    assert L.newt_function_set_max_lds(None, 1024) != 0
