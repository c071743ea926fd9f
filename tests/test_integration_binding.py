"""The Rust binding that INTEGRATION.md gives a maintainer, checked against the C header
on the CPU: the return codes keep the crate's three-way error split
(src/error.rs:11-29: InvalidArgument / Runtime / Internal), and every extern function
the binding declares exists in include/krea2_w8a8.h with the same number of
parameters."""

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _read(name):
    with open(os.path.join(ROOT, name)) as f:
        return f.read()


def _rust_blocks():
    return re.findall(r"```rust\n(.*?)```", _read("INTEGRATION.md"), re.S)


def _header_codes():
    codes = {}
    for name, value, comment in re.findall(r"#define (K2W8_\w+) \(?(-?\d+)\)?\s*(?:/\*(.*?)\*/)?",
                                           _read("include/krea2_w8a8.h")):
        codes[name] = (int(value), comment.strip())
    return codes


def test_the_return_codes_keep_the_crates_error_split():
    codes = _header_codes()
    assert codes["K2W8_OK"][0] == 0
    # the header names the crate variant each code stands for
    want = {"K2W8_INVALID_ARGUMENT": "InvalidArgument", "K2W8_RUNTIME": "Runtime", "K2W8_INTERNAL": "Internal"}
    for name, variant in want.items():
        assert variant in codes[name][1], (name, codes[name])
    check = next(b for b in _rust_blocks() if "fn check(" in b)
    arms = dict(re.findall(r"^\s*(-?\d+|_)\s*=>\s*crate::Error::(\w+)", check, re.M))
    assert arms[str(codes["K2W8_INVALID_ARGUMENT"][0])] == "InvalidArgument"
    assert arms[str(codes["K2W8_RUNTIME"][0])] == "Runtime"
    # a HIP failure is the machine's, carried as the runtime's own error type
    assert re.search(r"-3\s*=>\s*crate::Error::Runtime\(hrx::Error::\w+\(msg\)\)", check)
    # whatever is left (K2W8_INTERNAL) is a host bug
    internal = str(codes["K2W8_INTERNAL"][0])
    assert arms.get(internal, arms.get("_")) == "Internal"
    # every code the header defines besides OK has an arm
    for name in want:
        assert str(codes[name][0]) in arms or arms.get("_") == want[name], name


def _c_prototypes():
    text = re.sub(r"/\*.*?\*/", "", _read("include/krea2_w8a8.h"), flags=re.S)
    protos = {}
    for name, params in re.findall(r"\b(k2w8_\w+)\s*\(([^;{]*?)\)\s*;", text):
        params = params.strip()
        protos[name] = 0 if params in ("", "void") else params.count(",") + 1
    return protos


def test_every_bound_function_matches_a_header_prototype():
    protos = _c_prototypes()
    bound = {}
    for block in _rust_blocks():
        for name, params in re.findall(r"fn (k2w8_\w+)\s*\((.*?)\)\s*(?:->|;)", block, re.S):
            params = params.strip()
            bound[name] = 0 if not params else params.rstrip(",").count(",") + 1
    assert len(bound) >= 20
    for name, n in bound.items():
        assert name in protos, f"{name} is bound in INTEGRATION.md but not declared in the header"
        assert protos[name] == n, f"{name}: {n} parameters in the binding, {protos[name]} in the header"
