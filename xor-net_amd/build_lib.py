"""Build libxtern.so (HIP, gfx950) in-tree with hipcc.

Invoked by __graft_entry__.build(); also runnable directly:
    python xor-net_amd/build_lib.py
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "xtern", "libxtern.so")

SOURCES = ["xtern_kernels.hip", "xtern_sstack.hip", "xtern_gstream.hip", "xtern_xs.hip",
           "xtern_api.cpp", "xtern_layout.cpp", "xtern_container.cpp"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Wall",
    # Packed FP32 instructions are kept out of the device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


ROOT = os.path.dirname(HERE)
CPP_TEST_SRC = os.path.join(ROOT, "tests", "cpp", "test_host_api.cpp")
CPP_TEST_BIN = os.path.join(ROOT, "tests", "cpp", "test_host_api")


def build_cpp_tests(verbose=False):
    """The C++ host-API test program (links libxtern.so, rpath in-tree)."""
    cmd = [hipcc(), "-std=c++17", "-O2", "-Wall", CPP_TEST_SRC,
           "-L" + os.path.dirname(OUT), "-lxtern",
           "-Wl,-rpath,$ORIGIN/../../xor-net_amd/xtern", "-o", CPP_TEST_BIN]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc (C++ tests) failed:\n" + res.stderr)
    return CPP_TEST_BIN


DIAG_SRC = os.path.join(CSRC, "xtern_diag.hip")
DIAG_OUT = os.path.join(HERE, "xtern", "libxtern_diag.so")


def build_diag(verbose=False):
    """libxtern_diag.so: the measurement kernels of bench.py --peaks (streaming
    read, MFMA loop, empty launch); not part of the product ABI."""
    cmd = [hipcc()] + HIPCC_FLAGS + [DIAG_SRC, "-o", DIAG_OUT]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc (diag) failed:\n" + res.stderr)
    return DIAG_OUT


def build(verbose=False):
    """One object per source, compiled in parallel, then one link."""
    from concurrent.futures import ThreadPoolExecutor
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]

    def compile_one(src):
        obj = os.path.join(objdir, os.path.splitext(src)[0] + ".o")
        cmd = [hipcc()] + flags + ["-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        return obj, subprocess.run(cmd, capture_output=True, text=True)

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 6)) as ex:
        results = list(ex.map(compile_one, SOURCES))
    for obj, res in results:
        if res.returncode != 0:
            raise RuntimeError("hipcc failed:\n" + res.stderr)
        errs = [l for l in res.stderr.splitlines()
                if "packed-fp32-ops" not in l and "warning: unknown target feature" not in l]
        if verbose and errs:
            print("\n".join(errs))
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC"] + [o for o, _ in results] + ["-o", OUT]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc (link) failed:\n" + res.stderr)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-q" not in sys.argv))
    print(build_cpp_tests(verbose="-q" not in sys.argv))
    print(build_diag(verbose="-q" not in sys.argv))
