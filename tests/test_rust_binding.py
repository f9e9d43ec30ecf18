"""The Rust binding (rust/mlxq-sys, not compiled in this image: no cargo)
declares every entry point of include/mlxq.h with the header's argument
count, so a maintainer's build links and calls the same C ABI the tests use."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def c_functions():
    text = open(os.path.join(ROOT, "include", "mlxq.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(mlxq_\w+)\s*\(([^)]*)\)\s*;", text):
        args = [a for a in m.group(2).split(",") if a.strip() and a.strip() != "void"]
        out[m.group(1)] = len(args)
    return out


def rust_functions():
    text = open(os.path.join(ROOT, "rust", "mlxq-sys", "src", "lib.rs")).read()
    block = text[text.index('extern "C" {'):]
    block = block[: block.index("\n    }\n")]
    out = {}
    for m in re.finditer(r"pub fn (mlxq_\w+)\s*\(([^)]*)\)", block, flags=re.S):
        args = [a for a in m.group(2).split(",") if a.strip()]
        out[m.group(1)] = len(args)
    return out


def test_every_header_function_is_bound_with_its_arity():
    c, r = c_functions(), rust_functions()
    assert len(c) >= 18
    assert set(c) == set(r), (set(c) ^ set(r))
    for name, n in c.items():
        assert r[name] == n, (name, n, r[name])
