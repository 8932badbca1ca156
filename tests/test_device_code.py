"""Checks on the device code object this repository builds (gfx950 assembly of our
own sources, read with the ROCm LLVM tools).

A function larger than the 128 KiB reach of a short branch gets long branches
(s_getpc_b64 / s_add / s_setpc_b64 through an SGPR pair).  In a leaf called from
the kernel the compiler once took s[30:31] for them, the pair that holds the
return address, without saving it: after such a branch the leaf's return jumped
to a stale address and the GPU faulted.  No function may use that pair for
anything but its return."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "pjrt-ocl_amd", "python", "pjrt_amd", "libvmrt.so")
LLVM = "/opt/rocm/llvm/bin"
TOOLS = [os.path.join(LLVM, t) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")]


def _disassembly(tmp_path):
    if not os.path.exists(LIB):
        pytest.skip("libvmrt.so is not built")
    if not all(os.path.exists(t) for t in TOOLS) and not shutil.which("llvm-objdump"):
        pytest.skip("ROCm LLVM tools not found")
    fat, co = tmp_path / "fatbin", tmp_path / "gfx950.co"
    subprocess.run([TOOLS[0], f"--dump-section=.hip_fatbin={fat}", LIB], check=True)
    subprocess.run([TOOLS[1], "--unbundle", "--type=o", f"--input={fat}",
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={co}"], check=True)
    return subprocess.run([TOOLS[2], "-d", str(co)], check=True, capture_output=True, text=True).stdout


def test_no_long_branch_through_the_return_address(tmp_path):
    fn, bad, seen = None, {}, 0
    for line in _disassembly(tmp_path).splitlines():
        s = line.strip()
        if s.endswith(">:") and "<" in s:
            fn = s[s.index("<") + 1:-2]
            seen += 1
        elif s.startswith("s_getpc_b64 s[30:31]"):
            bad[fn] = bad.get(fn, 0) + 1
    assert seen > 10, "no functions found in the device code object"
    assert not bad, f"long branches through the return address pair s[30:31]: {bad}"
