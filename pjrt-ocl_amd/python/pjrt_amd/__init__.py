"""pjrt_amd: MI355X-native megakernel VM behind the pjrt-ocl plugin surface.

Layers (each mirrors a reference component; paths are into the reference tree):

* ``vmprogram``  VMProgram v3 bytecode reader/writer
                 (python/pjrt_ocl/lowering.py:207-331, scheduler.py:226-248)
* ``graph``      instruction-selection builder for tensor programs
                 (python/pjrt_ocl/ops/*.py encodings)
* ``scheduler``  tasks -> barrier phases -> per-lane entry streams
                 (python/pjrt_ocl/scheduler.py)
* ``runtime``    ctypes binding of ``libvmrt.so``, the HIP runtime that owns device
                 buffers, the arena and the persistent-kernel launch
                 (pjrt_plugin/src/runtime.{h,cc})

JAX discovery (``initialize``) follows python/pjrt_ocl/__init__.py:85-112: it
registers the PJRT plugin library under the platform name ``mi355x`` when both the
library and jax are present, and otherwise does nothing.
"""
from __future__ import annotations

import logging
import os
import sys

logger = logging.getLogger(__name__)

PLATFORM = "mi355x"
PLUGIN_PATH_ENV = "PJRT_AMD_PLUGIN_PATH"
RUNTIME_PATH_ENV = "PJRT_AMD_VMRT_PATH"

_HERE = os.path.dirname(os.path.abspath(__file__))


def find_runtime_library() -> str:
    """Absolute path of libvmrt.so: $PJRT_AMD_VMRT_PATH, else next to this file."""
    env = os.environ.get(RUNTIME_PATH_ENV)
    if env:
        if not os.path.isfile(env):
            raise FileNotFoundError(f"{RUNTIME_PATH_ENV}={env!r} is set but that file does not exist")
        return os.path.abspath(env)
    path = os.path.join(_HERE, "libvmrt.so")
    if os.path.isfile(path):
        return path
    raise FileNotFoundError(
        "libvmrt.so not found next to the pjrt_amd package; build it with "
        "`make -C pjrt-ocl_amd/csrc` (or __graft_entry__.build()), or set "
        f"{RUNTIME_PATH_ENV}")


def find_plugin_library() -> str:
    """Absolute path of the PJRT plugin library (libpjrt_amd.so), or raise
    FileNotFoundError.  Search order: $PJRT_AMD_PLUGIN_PATH, next to this file."""
    env = os.environ.get(PLUGIN_PATH_ENV)
    if env:
        if not os.path.isfile(env):
            raise FileNotFoundError(f"{PLUGIN_PATH_ENV}={env!r} is set but that file does not exist")
        return os.path.abspath(env)
    path = os.path.join(_HERE, "libpjrt_amd.so")
    if os.path.isfile(path):
        return path
    raise FileNotFoundError(f"PJRT plugin library not found (searched ${PLUGIN_PATH_ENV}, {path})")


def lower_service_path() -> str:
    """Absolute path of the lowering-service script the plugin executes."""
    return os.path.join(_HERE, "lower_service.py")


def initialize() -> None:
    """jax_plugins hook: register the ``mi355x`` PJRT platform with jax."""
    try:
        library_path = find_plugin_library()
    except FileNotFoundError as e:
        if PLATFORM in os.environ.get("JAX_PLATFORMS", ""):
            sys.stderr.write(f"\npjrt_amd: cannot register the '{PLATFORM}' backend:\n{e}\n\n")
        else:
            logger.warning("pjrt_amd: '%s' backend not registered: %s", PLATFORM, e)
        return
    try:
        from jax._src import xla_bridge as xb
    except ImportError:
        logger.warning("pjrt_amd: jax is not importable; '%s' not registered", PLATFORM)
        return
    if PLATFORM in xb._backend_factories:
        return
    options = {"python_exe": sys.executable, "lower_service": lower_service_path()}
    xb.register_plugin(PLATFORM, priority=500, library_path=library_path, options=options)
