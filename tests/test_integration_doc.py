"""INTEGRATION.md's Rust recipe must stay in step with the library it binds:
the build.rs source list equals the sources build_lib compiles, every
`extern "C"` fn is declared in include/xtern.h with the same number of
arguments, every `XT_*` constant carries the header's value, and the
`XtStackOp` mirror has the header struct's fields in order."""
import os
import re

import build_lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DOC = open(os.path.join(ROOT, "INTEGRATION.md")).read()
HDR = open(os.path.join(ROOT, "include", "xtern.h")).read()


def _strip_c_comments(s):
    s = re.sub(r"/\*.*?\*/", " ", s, flags=re.S)
    return re.sub(r"//[^\n]*", " ", s)


HDR_CODE = _strip_c_comments(HDR)


def _top_level_args(argstr):
    argstr = argstr.strip()
    if argstr in ("", "void"):
        return 0
    depth, n = 0, 1
    for ch in argstr:
        if ch in "([<":
            depth += 1
        elif ch in ")]>":
            depth -= 1
        elif ch == "," and depth == 0:
            n += 1
    return n


def _header_functions():
    out = {}
    for m in re.finditer(r"\b(xt_\w+)\s*\(([^;{]*?)\)\s*;", HDR_CODE, flags=re.S):
        out[m.group(1)] = _top_level_args(m.group(2))
    return out


def _header_consts():
    return {m.group(1): int(m.group(2))
            for m in re.finditer(r"\b(XT_\w+)\s*=\s*(-?\d+)", HDR_CODE)}


def _rust_blocks():
    return re.findall(r"```rust\n(.*?)```", DOC, flags=re.S)


def test_build_rs_compiles_every_library_source():
    build_rs = [b for b in _rust_blocks() if "fn main()" in b and "hipcc" in b]
    assert len(build_rs) == 1
    listed = re.findall(r'"xtern/csrc/([\w.]+)"', build_rs[0])
    assert len(listed) == len(set(listed))
    assert sorted(listed) == sorted(build_lib.SOURCES)
    # the device flags the library is built with are the ones the recipe uses
    for flag in ("--offload-arch=gfx950", "-ffp-contract=off", "-packed-fp32-ops"):
        assert flag in build_rs[0]


def test_extern_fns_exist_in_header_with_same_arity():
    hfns = _header_functions()
    ffi = "\n".join(b for b in _rust_blocks() if 'extern "C"' in b)
    fns = re.findall(r"pub fn (xt_\w+)\s*\((.*?)\)\s*(?:->[^;]*)?;", ffi, flags=re.S)
    assert len(fns) >= 25
    for name, args in fns:
        assert name in hfns, f"{name} is bound in INTEGRATION.md but not declared in xtern.h"
        assert _top_level_args(args) == hfns[name], name


def test_rust_consts_match_header():
    hc = _header_consts()
    consts = re.findall(r"pub const (XT_\w+): c_int = (-?\d+);", DOC)
    assert consts
    for name, val in consts:
        assert name in hc, name
        assert int(val) == hc[name], name
    # every format the header offers is bindable from Rust
    fmts = re.search(r"enum\s*\{\s*(XT_PACK4[^}]*)\}", HDR_CODE).group(1)
    for name in re.findall(r"(XT_\w+)\s*=", fmts):
        assert name in dict(consts), f"{name} missing from the Rust constants"


def test_stack_op_struct_mirror():
    c = re.search(r"typedef struct xt_stack_op \{(.*?)\}", HDR_CODE, flags=re.S).group(1)
    cfields = re.findall(r"(\w+)\s*(?:\[\d+\])?\s*;", c)
    r = re.search(r"pub struct XtStackOp \{(.*?)\}", DOC, flags=re.S).group(1)
    rfields = re.findall(r"pub (\w+):", r)
    assert cfields == rfields
