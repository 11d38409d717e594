"""Host parsers under AddressSanitizer / UndefinedBehaviorSanitizer: builds
tests/cpp/fuzz_host_parsers.cpp with the host-only library sources
(xtern_layout.cpp, xtern_container.cpp) and runs its mutation fuzzer over
XorSparse row blobs, the XORSPARE1 container reader, the dense repacks and
the HF destripe.  CPU only."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "cpp", "fuzz_host_parsers.cpp")
BIN = os.path.join(HERE, "cpp", "fuzz_host_parsers")
HIPCC = "/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else shutil.which("hipcc")


@pytest.mark.skipif(HIPCC is None, reason="hipcc not available")
def test_host_parsers_under_sanitizers():
    csrc = os.path.join(ROOT, "xor-net_amd", "csrc")
    cmd = [HIPCC, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-gpu-sanitize", "-fno-sanitize-recover=all",
           SRC, os.path.join(csrc, "xtern_layout.cpp"), os.path.join(csrc, "xtern_container.cpp"),
           "-o", BIN]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    run = subprocess.run([BIN, "2000"], capture_output=True, text=True, timeout=300, env=env)
    assert run.returncode == 0, (run.stdout + run.stderr)[-3000:]
    assert "fuzz ok" in run.stdout
