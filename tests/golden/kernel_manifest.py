"""Writes the machine-code fingerprints of a built libkrea2_w8a8.so into
tests/golden/kernel_manifest.json under a label, for test_kernel_manifest.py.

A label names a build whose kernels a GPU run passed: the fingerprints say which
kernels of a later build are the same machine code. To record an earlier commit:

    git worktree add /tmp/build <commit>
    make -C /tmp/build/krea2-hrx_amd
    python tests/golden/kernel_manifest.py /tmp/build/krea2-hrx_amd/libkrea2_w8a8.so \\
        <label> --commit <commit> --run "<which GPU run passed it>"
"""

import argparse
import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import codeobj  # noqa: E402

MANIFEST = os.path.join(HERE, "kernel_manifest.json")


def compiler() -> str:
    out = subprocess.run(["/opt/rocm/bin/hipcc", "--version"], capture_output=True, text=True).stdout
    return next((line.strip() for line in out.splitlines() if "clang version" in line), "unknown")


def main():
    p = argparse.ArgumentParser()
    p.add_argument("lib")
    p.add_argument("label")
    p.add_argument("--commit", required=True)
    p.add_argument("--run", required=True)
    a = p.parse_args()
    data = {}
    if os.path.exists(MANIFEST):
        with open(MANIFEST) as f:
            data = json.load(f)
    data["compiler"] = compiler()
    data.setdefault("builds", {})[a.label] = {
        "commit": a.commit, "gpu_run": a.run, "kernels": codeobj.fingerprints(a.lib)}
    with open(MANIFEST, "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
