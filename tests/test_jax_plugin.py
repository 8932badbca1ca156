"""JAX discovery of the plugin, without jax: the packaging metadata names the
hook, the namespace module reaches it, and ``pjrt_amd.initialize()`` registers
what the reference's hook registers (python/pjrt_ocl/__init__.py:85-112;
pyproject.toml:20-21) -- checked against a stand-in ``jax._src.xla_bridge``
that records the call."""
import ctypes
import importlib
import importlib.metadata
import logging
import os
import pkgutil
import sys
import types

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "pjrt-ocl_amd", "python")


class _XlaBridge(types.ModuleType):
    """What initialize() touches of jax._src.xla_bridge: the factory table and
    register_plugin (keyword arguments as jax defines them)."""

    def __init__(self):
        super().__init__("jax._src.xla_bridge")
        self._backend_factories = {}
        self.calls = []

    def register_plugin(self, plugin_name, *, priority=400, library_path=None, options=None):
        self.calls.append(dict(name=plugin_name, priority=priority, library_path=library_path, options=options))
        self._backend_factories[plugin_name] = object()


@pytest.fixture
def xla_bridge(monkeypatch):
    xb = _XlaBridge()
    jax = types.ModuleType("jax")
    src = types.ModuleType("jax._src")
    jax._src = src
    src.xla_bridge = xb
    monkeypatch.setitem(sys.modules, "jax", jax)
    monkeypatch.setitem(sys.modules, "jax._src", src)
    monkeypatch.setitem(sys.modules, "jax._src.xla_bridge", xb)
    return xb


def _plugin_built():
    import pjrt_amd
    try:
        return pjrt_amd.find_plugin_library()
    except FileNotFoundError:
        pytest.skip("libpjrt_amd.so not built (run __graft_entry__.build())")


def _check_registration(xb):
    import pjrt_amd
    assert len(xb.calls) == 1, xb.calls
    c = xb.calls[0]
    assert c["name"] == "mi355x" == pjrt_amd.PLATFORM
    assert c["priority"] == 500
    lib = c["library_path"]
    assert os.path.isabs(lib) and os.path.isfile(lib)
    assert hasattr(ctypes.CDLL(lib), "GetPjrtApi")
    opts = c["options"]
    assert set(opts) == {"python_exe", "lower_service"}
    assert opts["python_exe"] == sys.executable and os.path.isfile(opts["python_exe"])
    assert os.path.isfile(opts["lower_service"]) and opts["lower_service"].endswith("lower_service.py")


def test_initialize_registers_the_platform(xla_bridge, monkeypatch):
    _plugin_built()
    monkeypatch.delenv("PJRT_AMD_PLUGIN_PATH", raising=False)
    import pjrt_amd
    pjrt_amd.initialize()
    _check_registration(xla_bridge)
    pjrt_amd.initialize()            # already registered: no second registration
    assert len(xla_bridge.calls) == 1


def test_missing_library_registers_nothing_and_warns(xla_bridge, monkeypatch, caplog, capsys, tmp_path):
    import pjrt_amd
    monkeypatch.setenv("PJRT_AMD_PLUGIN_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setenv("JAX_PLATFORMS", "cpu")
    with caplog.at_level(logging.WARNING, logger="pjrt_amd"):
        pjrt_amd.initialize()
    assert xla_bridge.calls == []
    assert any("not registered" in r.getMessage() for r in caplog.records)
    # asked for explicitly, the reason goes to stderr (the reference's visible message)
    monkeypatch.setenv("JAX_PLATFORMS", "mi355x")
    pjrt_amd.initialize()
    assert xla_bridge.calls == []
    assert "cannot register the 'mi355x' backend" in capsys.readouterr().err


def test_entry_point_in_the_packaging():
    """pyproject.toml declares the jax_plugins entry point, its package mapping
    ships the module and both native libraries, and the entry point -- loaded
    the way jax loads the group's entries -- gives the module whose
    initialize() jax calls."""
    tomli = pytest.importorskip("tomli")
    with open(os.path.join(ROOT, "pyproject.toml"), "rb") as f:
        meta = tomli.load(f)
    eps = meta["project"]["entry-points"]["jax_plugins"]
    assert eps == {"mi355x": "pjrt_amd"}
    st = meta["tool"]["setuptools"]
    src = os.path.join(ROOT, st["package-dir"][""])
    assert os.path.samefile(src, PKG_DIR)
    for pkg in st["packages"]:
        assert os.path.isfile(os.path.join(src, *pkg.split("."), "__init__.py")), pkg
    assert sorted(meta["tool"]["setuptools"]["package-data"]["pjrt_amd"]) == ["libpjrt_amd.so", "libvmrt.so"]
    ep = importlib.metadata.EntryPoint(name="mi355x", value=eps["mi355x"], group="jax_plugins")
    mod = ep.load()
    assert mod.__name__ == "pjrt_amd" and callable(mod.initialize)


def test_namespace_discovery_runs_initialize(xla_bridge, monkeypatch):
    """jax's other route: every module of the jax_plugins namespace package is
    imported and its initialize() called."""
    _plugin_built()
    monkeypatch.delenv("PJRT_AMD_PLUGIN_PATH", raising=False)
    monkeypatch.syspath_prepend(PKG_DIR)
    for m in [m for m in sys.modules if m == "jax_plugins" or m.startswith("jax_plugins.")]:
        monkeypatch.delitem(sys.modules, m)
    import jax_plugins
    assert not hasattr(jax_plugins, "__file__") or jax_plugins.__file__ is None   # a namespace package
    names = [n for _, n, _ in pkgutil.iter_modules(jax_plugins.__path__, jax_plugins.__name__ + ".")]
    assert "jax_plugins.pjrt_amd" in names
    for n in names:
        mod = importlib.import_module(n)
        if hasattr(mod, "initialize"):
            mod.initialize()
    _check_registration(xla_bridge)
