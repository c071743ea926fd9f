"""The checkpoint reader and upload plan (k2w8_checkpoint.cpp) on malformed input,
on the CPU: the reader's source is compiled with AddressSanitizer and
UndefinedBehaviorSanitizer into tests/fuzz/checkpoint_fuzz.cpp's driver, which runs
open -> tensor lookups -> plan -> span queries on byte-level mutations of a valid
synthetic checkpoint and on valid-JSON headers with adversarial values (offsets past
the data, negative or huge numbers, shapes that disagree with the bytes, wrong dtypes,
missing and duplicated tensors). A memory error or undefined behaviour aborts the
driver; every variant must instead be accepted or refused with an error code."""

import json
import os
import random
import shutil
import struct
import subprocess

import numpy as np
import pytest

from ckpt_fixture import block_tensors, write_safetensors

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
ROCM = "/opt/rocm"


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if shutil.which("g++") is None or not os.path.exists(os.path.join(ROCM, "include", "hip")):
        pytest.skip("needs g++ and the ROCm headers")
    out = tmp_path_factory.mktemp("fuzz") / "checkpoint_fuzz"
    cmd = ["g++", "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{ROOT}/include",
           os.path.join(HERE, "fuzz", "checkpoint_fuzz.cpp"),
           os.path.join(ROOT, "krea2-hrx_amd", "csrc", "k2w8_checkpoint.cpp"),
           f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and "sanitize" in r.stderr:
        pytest.skip("no sanitizer runtime")
    assert r.returncode == 0, r.stderr[-2000:]
    return str(out)


@pytest.fixture(scope="module")
def base(tmp_path_factory):
    path = tmp_path_factory.mktemp("base") / "base.safetensors"
    write_safetensors(path, block_tensors(np.random.default_rng(1), layers=1, hidden=256, kv=64, inter=512))
    return path


def run(driver, args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([driver] + args, capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    return r.stdout


def test_the_valid_checkpoint_opens_and_plans(driver, base):
    assert "opened 1 planned 1" in run(driver, ["--files", str(base)])


def test_byte_mutations_never_corrupt_memory(driver, base, tmp_path):
    out = run(driver, ["--mutate", str(base), "6000", "12345", str(tmp_path / "m.safetensors")])
    assert out.startswith("mutations 6000")


def test_adversarial_headers_never_corrupt_memory(driver, base, tmp_path):
    raw = open(base, "rb").read()
    hlen = struct.unpack("<Q", raw[:8])[0]
    header = json.loads(raw[8:8 + hlen])
    data = raw[8 + hlen:]
    names = [k for k in header if k != "__metadata__"]
    values = [0, 1, -1, 2**31 - 1, 2**31, 2**32, 2**53, 2**63 - 1, -2**63, 10**30, 3.5, "7", None, [], {}]
    rnd = random.Random(7)
    files = []
    for i in range(1500):
        h = json.loads(json.dumps(header))
        name = rnd.choice(names)
        e = h[name]
        payload = data
        kind = rnd.randrange(12)
        if kind == 0:
            e["data_offsets"] = [rnd.choice(values), rnd.choice(values)]
        elif kind == 1:
            e["data_offsets"] = [rnd.choice(values)]
        elif kind == 2:
            e["shape"] = [rnd.choice(values) for _ in range(rnd.randrange(0, 10))]
        elif kind == 3:
            e["dtype"] = rnd.choice(["I8", "F32", "BF16", "F16", "F64", "U8", "", 5, None])
        elif kind == 4:
            del h[name]
        elif kind == 5:
            h[name.replace("blocks.0", "blocks." + str(rnd.choice(values)))] = e
        elif kind == 6:
            lo, hi = e["data_offsets"]
            e["data_offsets"] = [lo, hi + rnd.choice([-1, 1, 4096, 10**9])]
        elif kind == 7:
            h[name] = rnd.choice(values)
        elif kind == 8:
            h["__metadata__"] = rnd.choice([{"format": "pt"}, 5, [], {"a": {"b": 1}}])
        elif kind == 9:
            e["shape"] = [s * rnd.choice([2, 0]) for s in e["shape"]]
        elif kind == 10:
            payload = data[:rnd.randrange(len(data))]
        else:
            h["blocks.1.attn.wq.weight"] = e
        text = json.dumps(h).encode()
        path = tmp_path / f"{i:04d}.safetensors"
        with open(path, "wb") as f:
            f.write(struct.pack("<Q", len(text)))
            f.write(text)
            f.write(payload)
        files.append(str(path))
    out = run(driver, ["--files"] + files)
    assert out.startswith("files 1500")
