"""Which kernels of this build are the machine code a GPU run has passed.

tests/golden/kernel_manifest.json holds the instruction fingerprints of two earlier
builds (tests/golden/kernel_manifest.py wrote them): the one the driver's end-of-round
GPU tests passed, and the one the builder's last full GPU suite passed. A kernel of
this build whose fingerprint equals one of theirs is the same machine code, so those
runs' results hold for it. Every kernel of the default path must be such a kernel;
only the opt-in paths changed or added since (the one-launch prepare -> GEMM with its
barrier reset, and the backward-K tile GEMMs) may be new."""

import json
import os
import re
import subprocess

import pytest

import codeobj

HERE = os.path.dirname(os.path.abspath(__file__))
MANIFEST = os.path.join(HERE, "golden", "kernel_manifest.json")

# Opt-in paths whose machine code no GPU run has passed yet.
NOT_YET_RUN = re.compile(r"_ZN4k2w85fused|_ZN4k2w84gemm20gemm_kernel_backward")


@pytest.fixture(scope="module")
def manifest():
    with open(MANIFEST) as f:
        data = json.load(f)
    out = subprocess.run(["/opt/rocm/bin/hipcc", "--version"], capture_output=True, text=True).stdout
    if data["compiler"] not in out:
        pytest.skip("another compiler: fingerprints of its machine code are not comparable")
    return data


def classify(manifest):
    now = codeobj.fingerprints()
    kernels = {k[".name"] for k in codeobj.kernels()}
    builds = manifest["builds"]
    out = {}
    for name in kernels:
        h = now[name]
        out[name] = ("driver" if builds["driver"]["kernels"].get(name) == h
                     else "builder" if builds["builder"]["kernels"].get(name) == h else None)
    return out


def test_every_default_path_kernel_is_machine_code_a_gpu_run_passed(manifest):
    cls = classify(manifest)
    unrun = sorted(k for k, c in cls.items() if c is None)
    assert [k for k in unrun if not NOT_YET_RUN.search(k)] == []
    # the hot path's kernels: the tile GEMMs, the prepares, the few-token kernel
    for family in ("gemm11gemm_kernel", "prepare_kernel", "skinny13stream_kernel", "splitk13reduce_kernel"):
        members = [k for k in cls if family in k]
        assert members and all(cls[k] for k in members), family


def test_the_attention_step_is_the_driver_verified_machine_code(manifest):
    cls = classify(manifest)
    for family in ("attn16attention_kernel", "attn18rope_qknorm_kernel", "attn18v_transpose_kernel",
                   "transport_kernel"):
        members = [k for k in cls if family in k]
        assert members and all(cls[k] == "driver" for k in members), family
