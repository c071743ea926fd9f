"""Reads the gfx950 code objects that the build put into libkrea2_w8a8.so.

Test infrastructure: the kernels' resource metadata (scratch, spills, registers, LDS)
and their disassembly, taken from the library this repository builds, so that CPU
tests can hold invariants of the device code that no host-side run exercises.
"""

from __future__ import annotations

import functools
import hashlib
import os
import re
import struct
import subprocess
import tempfile

import yaml

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "krea2-hrx_amd", "libkrea2_w8a8.so")
LLVM = "/opt/rocm/llvm/bin"
_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def code_objects(path: str = LIB) -> list[bytes]:
    """The gfx950 ELF images of every offload bundle in the library's .hip_fatbin."""
    data = open(path, "rb").read()
    out, i = [], 0
    while True:
        i = data.find(_MAGIC, i)
        if i < 0:
            return out
        (count,) = struct.unpack_from("<Q", data, i + len(_MAGIC))
        p = i + len(_MAGIC) + 8
        for _ in range(count):
            off, size, tlen = struct.unpack_from("<QQQ", data, p)
            triple = data[p + 24:p + 24 + tlen]
            p += 24 + tlen
            if b"gfx950" in triple and size:
                out.append(data[i + off:i + off + size])
        i += len(_MAGIC)


def _tool(args: list[str], image: bytes) -> str:
    with tempfile.NamedTemporaryFile(suffix=".co") as f:
        f.write(image)
        f.flush()
        return subprocess.run([os.path.join(LLVM, args[0]), *args[1:], f.name], check=True,
                              capture_output=True, text=True).stdout


@functools.lru_cache(maxsize=None)
def kernels(path: str = LIB) -> list[dict]:
    """AMDGPU metadata of every kernel (the `amdhsa.kernels` entries), with `.image`
    set to the index of its code object in code_objects()."""
    out = []
    for n, image in enumerate(code_objects(path)):
        notes = _tool(["llvm-readelf", "--notes"], image)
        start = notes.index("---")
        end = notes.index("\n...", start)
        meta = yaml.safe_load(notes[start:end])
        for k in meta["amdhsa.kernels"]:
            k[".image"] = n
            out.append(k)
    return out


@functools.lru_cache(maxsize=None)
def disassembly(image_index: int, path: str = LIB) -> dict[str, list[str]]:
    """Instruction lines of each function symbol of one code object, by symbol name."""
    text = _tool(["llvm-objdump", "-d", "--no-show-raw-insn", "--no-leading-addr"],
                 code_objects(path)[image_index])
    funcs: dict[str, list[str]] = {}
    cur = None
    for line in text.splitlines():
        if line.endswith(">:") and "<" in line:
            cur = line[line.index("<") + 1:-2]
            funcs[cur] = []
        elif cur is not None and line.strip():
            funcs[cur].append(line.strip())
    return funcs


def fingerprints(path: str = LIB) -> dict[str, str]:
    """A hash of each function's instructions (the disassembly without addresses and
    encodings), by symbol name: equal hashes mean the same machine code, wherever the
    linker placed it."""
    out = {}
    for n in range(len(code_objects(path))):
        for name, lines in disassembly(n, path).items():
            text = "\n".join(re.sub(r"\s*//.*", "", line).strip() for line in lines)
            out[name] = hashlib.sha256(text.encode()).hexdigest()[:16]
    return out
