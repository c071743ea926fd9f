"""Which kernel each BASELINE shape runs (k2w8_gemm_choose, the rule launch_gemm
applies), on the CPU. The expected choices are the kernels the GPU kernel traces show
for these shapes (profiles/gemm_i8_mid_m_counters.md for config 5,
profiles/block_linears_4544_kernel_trace.md for the block, the QKV and north-star
traces), so a change of the rule that moves a measured shape to another kernel shows
up here."""

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "krea2-hrx_amd")


@pytest.fixture(scope="module")
def k2():
    if not os.path.exists(os.path.join(LIBDIR, "libkrea2_w8a8.so")):
        subprocess.run(["make", "-s", "-C", LIBDIR], check=True)
    import krea2_w8a8

    return krea2_w8a8


CASES = [
    # (what, m, k, n, epilogue, expected)
    ("configs[1] QKV", 4096, 3072, 9216, "plain", {"kernel": "tile", "tile": (256, 192), "stages": 2}),
    ("north star", 4096, 3072, 12288, "plain", {"kernel": "tile", "tile": (256, 256), "stages": 2}),
    ("configs[0] bias", 4096, 3072, 3072, "bias", {"kernel": "tile", "tile": (256, 192), "stages": 2}),
    ("block qkvg", 4544, 3072, 9216, "plain", {"kernel": "tile", "tile": (256, 256), "stages": 2}),
    ("block wo", 4544, 3072, 3072, "resid", {"kernel": "tile", "tile": (256, 256), "stages": 2}),
    ("block gate|up", 4544, 3072, 24576, "swiglu", {"kernel": "tile", "tile": (256, 256), "stages": 2}),
    ("block down", 4544, 12288, 3072, "resid", {"kernel": "tile", "tile": (256, 256), "stages": 2}),
    ("config 5 QKV, 1 token", 1, 2560, 4096, "plain", {"kernel": "few-token"}),
    ("config 5 QKV, 77", 77, 2560, 4096, "plain", {"kernel": "few-token"}),
    ("config 5 up, 77", 77, 2560, 19456, "swiglu", {"kernel": "tile", "tile": (128, 64), "stages": 3}),
    ("config 5 down, 77", 77, 9728, 2560, "resid",
     {"kernel": "split-k", "tile": (128, 128), "stages": 3, "splits": 11, "split_steps": 7}),
    ("config 5 QKV, 256", 256, 2560, 4096, "plain", {"kernel": "tile", "tile": (64, 64), "stages": 4}),
    ("config 5 up, 256", 256, 2560, 19456, "swiglu", {"kernel": "tile", "tile": (256, 128), "stages": 3}),
    ("config 5 down, 256", 256, 9728, 2560, "resid",
     {"kernel": "split-k", "tile": (128, 128), "stages": 3, "splits": 6, "split_steps": 13}),
    ("config 5 QKV, 512", 512, 2560, 4096, "plain", {"kernel": "tile", "tile": (128, 64), "stages": 3}),
    ("config 5 up, 512", 512, 2560, 19456, "swiglu", {"kernel": "tile", "tile": (256, 256), "stages": 2}),
    ("config 5 down, 512", 512, 9728, 2560, "resid",
     {"kernel": "split-k", "tile": (128, 128), "stages": 3, "splits": 3, "split_steps": 26}),
    ("a mostly idle last round", 2000, 256, 9216, "plain",
     {"kernel": "tile+tail", "tile": (256, 256), "stages": 2, "n_big": 8192}),
]


@pytest.mark.parametrize("what,m,k,n,epilogue,expected", CASES, ids=[c[0] for c in CASES])
def test_baseline_shapes_run_the_measured_kernels(k2, what, m, k, n, epilogue, expected):
    got = k2.gemm_choose(m, cfg=k2.GemmConfig(k_size=k, n_size=n, k_stride=k), epilogue=epilogue)
    assert got == expected


def test_split_k_needs_room_for_two_slices(k2):
    cfg = k2.GemmConfig(k_size=9728, n_size=2560, k_stride=9728)
    # the M=256 down projection splits in the library's workspace and in the 16 MiB
    # static scratch of the allocation-free entry point, not in 1 MiB
    assert k2.gemm_choose(256, cfg=cfg, epilogue="resid")["kernel"] == "split-k"
    assert k2.gemm_choose(256, cfg=cfg, epilogue="resid", workspace_bytes=16 << 20)["kernel"] == "split-k"
    no_room = k2.gemm_choose(256, cfg=cfg, epilogue="resid", workspace_bytes=1 << 20)
    assert no_room == {"kernel": "tile", "tile": (64, 64), "stages": 4}


def test_every_split_fits_the_static_scratch_on_256_cus(k2):
    # The allocation-free entry point's promise: on 256 CUs, two int32 slices of every
    # shape the split rule picks fit its 16 MiB.
    for m in range(33, 2049, 7):
        for n in range(128, 32769, 640):
            for k in (1024, 4224, 9728, 16384, 65536):
                got = k2.gemm_choose(m, cfg=k2.GemmConfig(k_size=k, n_size=n, k_stride=k), epilogue="plain",
                                     workspace_bytes=1 << 40)
                if got["kernel"] == "split-k":
                    assert 2 * m * n * 4 <= 16 << 20, (m, n, k)


def test_the_allocation_free_refusal_is_the_choice_rule(k2):
    # gemm_i8_noalloc's 16 MiB scratch is fixed: on a device with more CUs the split
    # rule can pick a shape whose two int32 slices do not fit, and the entry point
    # refuses it (INVALID_ARGUMENT) instead of running 64x64 tiles. 512 CUs, M=1024,
    # N=2560, K=9728: 160 128x128 tiles split, and 2 x 1024 x 2560 x 4 = 20 MiB > 16 MiB.
    cfg = k2.GemmConfig(k_size=9728, n_size=2560, k_stride=9728)
    fixed = dict(cus=512, workspace_bytes=16 << 20)
    assert k2.gemm_choose(1024, cfg=cfg, epilogue="resid", **fixed, workspace_required=True) == {"kernel": "refused"}
    # the same fixed size without the requirement falls back to 64x64 tiles
    assert k2.gemm_choose(1024, cfg=cfg, epilogue="resid", **fixed)["tile"] == (64, 64)
    # with room for two slices the required workspace splits as usual
    roomy = dict(cus=512, workspace_bytes=32 << 20)
    assert k2.gemm_choose(1024, cfg=cfg, epilogue="resid", **roomy, workspace_required=True)["kernel"] == "split-k"
    # a shape that does not split is never refused
    wide = k2.GemmConfig(k_size=3072, n_size=9216, k_stride=3072)
    assert k2.gemm_choose(4096, cfg=wide, **fixed, workspace_required=True)["kernel"] in ("tile", "tile+tail")


def test_a_captured_call_without_a_workspace_runs_64x64_tiles(k2):
    # Inside a stream capture with no registered or installed workspace the library has
    # none: the M=256 down projection then runs 64x64 tiles, not split K.
    cfg = k2.GemmConfig(k_size=9728, n_size=2560, k_stride=9728)
    assert k2.gemm_choose(256, cfg=cfg, epilogue="resid", workspace_bytes=0) == {
        "kernel": "tile", "tile": (64, 64), "stages": 4}


def test_the_choice_depends_on_the_cu_count(k2):
    cfg = k2.GemmConfig(k_size=3072, n_size=9216, k_stride=3072)
    assert k2.gemm_choose(4096, cfg=cfg, cus=256)["tile"] == (256, 192)
    # 304 CUs: 576 256x256 tiles are 1.9 rounds, 768 256x192 ones 2.5
    assert k2.gemm_choose(4096, cfg=cfg, cus=304)["tile"] == (256, 256)


def test_bad_arguments_are_refused(k2):
    cfg = k2.GemmConfig(k_size=3072, n_size=9216, k_stride=3072)
    for kwargs in (dict(cus=0), dict(cus=5000), dict(workspace_bytes=-1)):
        with pytest.raises(k2.InvalidArgument):
            k2.gemm_choose(4096, cfg=cfg, **kwargs)
    with pytest.raises(k2.InvalidArgument):
        k2.gemm_choose(0, cfg=cfg)
    with pytest.raises(k2.InvalidArgument):
        k2.gemm_choose(4096, cfg=k2.GemmConfig(k_size=3000, n_size=9216, k_stride=3072))


def test_the_one_launch_rule_admits_whole_rounds_of_256x192_tiles(tmp_path):
    # k2w8_linear_{norm,plain}_i8's one-launch form (K2W8_LINEAR_ONE_LAUNCH=1) runs only
    # where every workgroup is resident with one per CU: whole rounds of 256x192 tiles.
    import shutil
    if shutil.which("g++") is None:
        pytest.skip("needs g++")
    exe = tmp_path / "one_launch_rule"
    src = os.path.join(ROOT, "tests", "fuzz", "one_launch_rule.cpp")
    subprocess.run(["g++", "-O1", "-std=c++17", f"-I{LIBDIR}/csrc", src, "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert int(r.stdout.split()[-1]) > 0
