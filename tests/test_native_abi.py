"""The C-ABI library loads on a machine without a GPU and exports every entry point
include/vmrt.h declares (no device calls are made here)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vmrt.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vmrt_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_runtime_surface():
    names = declared_functions()
    for required in ("vmrt_create", "vmrt_load", "vmrt_execute", "vmrt_enqueue", "vmrt_alloc", "vmrt_free",
                     "vmrt_h2d", "vmrt_d2h", "vmrt_unload", "vmrt_destroy"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from pjrt_amd import find_runtime_library
    try:
        path = find_runtime_library()
    except FileNotFoundError:
        pytest.skip("libvmrt.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    lib.vmrt_version.restype = ctypes.c_char_p
    assert b"gfx950" in lib.vmrt_version()


def test_python_binding_covers_the_header():
    from pjrt_amd import runtime
    assert sorted(runtime.SIGNATURES) == declared_functions()


def test_binding_loads_without_a_device():
    from pjrt_amd import runtime
    try:
        lib = runtime.load_library()
    except FileNotFoundError:
        pytest.skip("libvmrt.so not built")
    assert lib.vmrt_version()
