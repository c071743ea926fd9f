"""bench.py's contract on the CPU: it measures one GPU and says so for any other count,
and its CPU baseline (the oracle on the host's cores) reports the fields the bench line
carries, on a small budget."""

import importlib.util
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_bench():
    spec = importlib.util.spec_from_file_location("bench", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_cpu_baseline_reports_its_sample_cores_and_single_thread_figure():
    bench = load_bench()
    out = bench.cpu_baseline(4096, 256, 256, 256, 0.2)
    assert out["kind"] == "port" and out["unit"] == "TOPS" and out["value"] > 0
    assert out["cores"] >= 1 and "tokens" in out["sample"]
    single = out["single_thread"]
    assert single["cores"] == 1 and single["value"] > 0
    # the multi-threaded figure is not below the single-threaded one by much (same code)
    assert out["value"] > 0.5 * single["value"]


def test_kernel_choices_name_every_benchmarked_shape():
    import sys
    sys.path.insert(0, os.path.join(ROOT, "krea2-hrx_amd"))
    import krea2_w8a8 as k2

    bench = load_bench()
    out = bench.kernel_choices(k2, 256)
    assert out["cus"] == 256 and len(out) == 1 + 9 + 15
    assert out["configs[1] QKV"] == "tile 256x192"
    assert out["configs[4] down M=256"] == "split-k 128x128 x6 slices"
    assert out["configs[4] qkv M=1"] == "few-token"


def test_roofline_traffic_names_its_source():
    # roofline.traffic is read from a committed rocprofv3 profile, not measured in the
    # run: the bench line says which file, launch and build it comes from.
    bench = load_bench()
    src = bench.traffic_source()
    assert src["measured_in_this_run"] is False
    assert os.path.exists(os.path.join(ROOT, src["file"])) and src["file"].startswith("profiles/")
    assert "gemm_kernel<256, 192" in src["launch"] and src["build"]
    assert all("rocprofv3 --pmc" in c for c in src["commands"])
    assert bench.measured_traffic() > 0
