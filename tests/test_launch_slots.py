"""Per-launch status bookkeeping of the runtime, on the CPU: the slot pool and
status decoding of pjrt-ocl_amd/csrc/launch_slots.h, built with g++ and driven
by tests/launch_slots_check.cpp (the GPU side -- the status epilogue kernel and
vmrt_submit -- is tested in test_gpu_vm.py)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_launch_slots_bookkeeping(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "launch_slots_check"
    subprocess.run([cxx, "-O1", "-std=c++17", "-Wall", "-Werror", "-fsanitize=address,undefined",
                    "-I", os.path.join(ROOT, "pjrt-ocl_amd", "csrc"),
                    os.path.join(ROOT, "tests", "launch_slots_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, timeout=120)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr
