"""The C ABI's validation on the CPU, under AddressSanitizer and UndefinedBehaviorSanitizer:
every GEMM, prepare, one-call linear and block entry point is driven with edge and random
arguments (tests/fuzz/abi_validation.cpp), with the kernel launchers replaced by stubs
that check the preconditions the kernels rely on. Accepted calls must meet them all;
rejected ones must return an error code, with no sanitizer report either way."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
ROCM = "/opt/rocm"


def test_accepted_calls_meet_the_launchers_preconditions(tmp_path):
    if shutil.which("g++") is None or not os.path.exists(os.path.join(ROCM, "include", "hip")):
        pytest.skip("needs g++ and the ROCm headers")
    exe = tmp_path / "abi_validation"
    cmd = ["g++", "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{ROOT}/include",
           f"-I{ROOT}/krea2-hrx_amd/csrc", os.path.join(HERE, "fuzz", "abi_validation.cpp"),
           os.path.join(ROOT, "krea2-hrx_amd", "csrc", "k2w8_api.cpp"),
           os.path.join(ROOT, "krea2-hrx_amd", "csrc", "k2w8_block.cpp"),
           f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0 and "sanitize" in r.stderr:
        pytest.skip("no sanitizer runtime")
    assert r.returncode == 0, r.stderr[-2000:]
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600,
                       env=dict(os.environ, UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1"))
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    counts = dict(part.rsplit(" ", 1) for part in r.stdout.strip().split(", "))
    assert int(counts["gemm launches"]) > 1000 and int(counts["prepare launches"]) > 1000
    assert int(counts["other launches"]) > 100 and int(counts["blocks accepted"]) > 1000
    assert counts["violations"] == "0"
