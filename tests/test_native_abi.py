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


class _FakeLib:
    """Records native calls; stands in for libvmrt.so to test the host-side
    ownership rules without a device."""

    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        def fn(*args):
            self.calls.append(name)
            return 0
        return fn


def _fake_runtime():
    import weakref
    from pjrt_amd import runtime
    rt = object.__new__(runtime.Runtime)
    rt._lib = _FakeLib()
    rt._h = 1234
    rt._programs = weakref.WeakSet()
    lp = object.__new__(runtime.LoadedProgram)
    lp.rt, lp._h = rt, 5678
    rt._programs.add(lp)
    return rt, lp


def test_closing_the_runtime_closes_its_programs_first():
    rt, lp = _fake_runtime()
    rt.close()
    assert rt._lib.calls == ["vmrt_unload", "vmrt_destroy"]
    lp.close()                        # already unloaded: no second native call
    del lp
    assert rt._lib.calls == ["vmrt_unload", "vmrt_destroy"]


def test_program_of_a_closed_runtime_makes_no_native_call():
    from pjrt_amd import runtime
    rt, lp = _fake_runtime()
    rt._programs.discard(lp)          # a program the runtime no longer tracks
    rt.close()
    assert rt._lib.calls == ["vmrt_destroy"]
    lp.close()
    with pytest.raises(runtime.VmrtError):
        lp.status()
    buf = runtime.DeviceBuffer(rt, 42, 16)
    buf.free()
    assert rt._lib.calls == ["vmrt_destroy"] and buf.ptr == 0


def test_plugin_library_exports_the_declared_entry_point():
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "pjrt_amd.h")).read(), flags=re.S)
    names = set(re.findall(r"\b(GetPjrtApi)\s*\(", text))
    path = os.path.join(ROOT, "pjrt-ocl_amd", "python", "pjrt_amd", "libpjrt_amd.so")
    if not os.path.isfile(path):
        pytest.skip("libpjrt_amd.so not built")
    lib = ctypes.CDLL(path)
    assert names == {"GetPjrtApi"} and all(hasattr(lib, n) for n in names)
