"""The workspace ownership rules of the C ABI (xor-net_amd/csrc/xtern_workspace.h)
on the CPU with a fake allocator: several host threads on one stream never
share a buffer, growth retires the old buffer instead of freeing it, nothing
is allocated while a stream is captured, release frees every buffer once.
Built twice: AddressSanitizer + UBSan, and ThreadSanitizer."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "cpp", "test_workspace.cpp")
GXX = shutil.which("g++")


@pytest.mark.skipif(GXX is None, reason="g++ not available")
@pytest.mark.parametrize("san", ["address,undefined", "thread"])
def test_workspace_table(tmp_path, san):
    exe = str(tmp_path / "test_workspace")
    cmd = [GXX, "-std=c++17", "-O1", "-g", "-pthread", "-include", "cstring",
           f"-fsanitize={san}", "-fno-sanitize-recover=all", SRC, "-o", exe]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    run = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, (run.stdout + run.stderr)[-3000:]
    assert "workspace ok" in run.stdout
