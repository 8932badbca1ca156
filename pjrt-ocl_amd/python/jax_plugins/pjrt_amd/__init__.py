"""jax_plugins namespace hook of the MI355X PJRT plugin.

jax imports every module under the ``jax_plugins`` namespace package at start-up
and calls its ``initialize()``; this one hands over to ``pjrt_amd.initialize``,
which registers platform ``mi355x`` (python/pjrt_ocl/__init__.py:85-112 is the
reference's hook).  An installed package reaches the same function through the
``jax_plugins`` entry point instead.
"""
from pjrt_amd import initialize  # noqa: F401
