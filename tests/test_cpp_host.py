"""Runs the C++ host-API test program (tests/cpp/test_host_api.cpp, built by
__graft_entry__.build()): its codec tests on the CPU, everything on the GPU."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(__file__), "cpp", "test_host_api")


def _run(args):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built; run __graft_entry__.build()")
    r = subprocess.run([BIN] + args, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr


def test_cpp_codecs_cpu():
    _run(["--cpu"])


@pytest.mark.gpu
def test_cpp_host_api_gpu():
    _run([])
