"""GPU parity of the INT8 GEMM family: int32 accumulators bit-exact with a brute-force
integer dot, and every epilogue bit-exact with the CPU oracle on the same accumulators
(the reference's tolerance, tests/quantized.rs:277, is checked as well)."""

import os

import numpy as np
import pytest
import torch

import oracle
from gpu_common import (bf16_bits, bf16_value, channel_scales, dev, f16_bits, host, int8_weights,
                        k2, sync)

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def cfg(k, n, stride):
    return k2.GemmConfig(k_size=k, n_size=n, k_stride=stride, m_group=4)


def gpu_acc(a, w, m, n, k, stride):
    acc = torch.empty((m, n), dtype=torch.int32, device="cuda")
    k2.gemm_i8_acc(dev(a), dev(w), acc, cfg=cfg(k, n, stride), m=m)
    sync()
    return host(acc)


def gpu_epilogue(mode, a, w, ws, a_scale, m, n, k, stride, gate=None, prior=None, bias=None):
    c = cfg(k, n, stride)
    A, W, WS, AS = dev(a), dev(w), dev(ws), dev(a_scale)
    if mode == "plain":
        out = torch.full((m, n), 7, dtype=torch.int16, device="cuda").view(torch.float16)
        k2.gemm_i8(A, W, WS, AS, out, cfg=c, m=m)
    elif mode == "bias":
        out = torch.empty((m, n), dtype=torch.float16, device="cuda")
        k2.gemm_i8_bias(A, W, WS, AS, dev(bias, torch.float16), out, cfg=c, m=m)
    elif mode in ("resid", "resid_wide"):
        out = dev(prior.reshape(m, n), torch.bfloat16)
        fn = k2.gemm_i8_resid if mode == "resid" else k2.gemm_i8_resid_256x256
        fn(A, W, WS, AS, out, dev(gate), cfg=c, m=m)
    else:
        out = torch.empty((m, n // 2), dtype=torch.float16, device="cuda")
        k2.gemm_i8_swiglu(A, W, WS, AS, out, cfg=c, m=m)
    sync()
    return host(out)


GOLDEN_CASES = [
    "gemm_plain_17x128x128_pad0", "gemm_plain_257x384x256_pad128",
    "gemm_resid_17x128x128_pad0", "gemm_resid_257x384x256_pad128",
    "gemm_swiglu_17x128x128_pad0", "gemm_swiglu_257x384x256_pad128",
    "gemm_resid_wide_17x128x256_pad0", "gemm_resid_wide_257x384x512_pad128",
]


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_reference_integer_cases_are_exact(name):
    g = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    m, k, n, stride = (int(g[x]) for x in ("m", "k", "n", "stride"))
    acc = gpu_acc(g["a"], g["w"], m, n, k, stride)
    assert np.array_equal(acc, g["dot"])
    if "_swiglu" in name:
        out = gpu_epilogue("swiglu", g["a"], g["w"], g["ws"], g["a_scale"], m, n, k, stride)
        ref = oracle.epilogue_swiglu(g["dot"], g["ws"], g["a_scale"])
        val = out.view(np.float16).astype(np.float64)
    elif "_resid" in name:
        mode = "resid_wide" if "_wide" in name else "resid"
        out = gpu_epilogue(mode, g["a"], g["w"], g["ws"], g["a_scale"], m, n, k, stride,
                           gate=g["gates"], prior=g["residual"])
        ref = oracle.epilogue_resid(g["dot"], g["ws"], g["a_scale"], g["gates"], g["residual"])
        val = bf16_value(out).astype(np.float64)
    else:
        out = gpu_epilogue("plain", g["a"], g["w"], g["ws"], g["a_scale"], m, n, k, stride)
        ref = oracle.epilogue_plain(g["dot"], g["ws"], g["a_scale"])
        val = out.view(np.float16).astype(np.float64)
    assert np.array_equal(out, ref)
    want = g["want"].astype(np.float64)
    assert np.all(np.abs(val - want) <= 2e-3 + 4e-3 * np.abs(want))


SHAPES = [
    # (m, k, n, pad): ghost rows, one and many tiles on both axes, both tile widths
    (1, 128, 128, 0),
    (17, 256, 384, 64),
    (255, 384, 256, 0),
    (256, 512, 512, 128),
    (257, 640, 1024, 0),
    (1000, 3072, 768, 0),
    (513, 2560, 4096, 0),
    (2000, 256, 8192, 64),  # >= 256 tiles of 256x256: the wide-tile kernel
    # whole rounds of 256x256 tiles, then the last columns as one round of 128x128
    (2000, 256, 9216, 64),
    # one round of 256x256 tiles where 256x128 would take two
    (300, 256, 19456, 0),
    # 256x192 tiles where they take less time than 256x256 (rounds x width), including
    # a SwiGLU output whose 32-row gate|up groups the 192-wide tiles keep whole
    (4096, 256, 9216, 0),
    (4096, 128, 3072, 64),
    (2304, 128, 24576, 0),
    # one round of 256x128 tiles over more than half the CUs: the three-stage kernel
    (200, 1024, 19456, 64),
    # split K over 128x128 tiles (fewer than half the CUs get a tile; or 64x64 tiles
    # would fill the chip but K is long)
    (320, 4224, 4096, 0),
    (256, 9728, 2560, 0),
    (129, 2560, 4096, 64),
    (300, 1024, 512, 0),
    # few-token kernel: K ranges that leave a wave one 128-byte step or none; 8-row
    # (N/16 below the CU count) and 16-row workgroups; 8 staged token rows (M <= 8) and
    # one or two 16-token blocks; row strides that are not whole cache lines
    (2, 384, 256, 0),
    (16, 2560, 512, 0),
    (8, 9728, 256, 64),
    (9, 256, 4096, 0),
    (24, 512, 4096, 64),
    (32, 1024, 1024, 0),
    (33, 640, 384, 64),
    (64, 9728, 256, 0),
    (77, 2560, 512, 0),
    # the streaming kernel past 32 tokens (short K, grid resident at once): two token
    # groups of 64 and 36
    (100, 1024, 4096, 64),
    # the epilogue stages its output in a stage buffer free at the end of the K loop:
    # stage 1 after a single K step, stage (steps - 2) mod stages after more; one, two
    # and three steps on the 64x64 tiles of two K groups, the 128x64 tiles (three
    # stages), the three-stage 256x128 tiles and the two-stage 256x256 tiles
    (256, 128, 4096, 0),
    (256, 256, 4096, 64),
    (512, 128, 4096, 0),
    (512, 384, 4096, 64),
    (200, 128, 19456, 0),
    (200, 384, 19456, 0),
    (2000, 384, 8192, 0),
    # the largest K (65536): 128 K steps per wave in the few-token kernel; split K over
    # 128 slices in the tile kernels
    (3, 65536, 512, 0),
    (64, 65536, 256, 0),
]


@pytest.mark.parametrize("m,k,n,pad", SHAPES)
def test_accumulators_and_every_epilogue_are_exact(m, k, n, pad):
    rng = np.random.default_rng(m * 7 + k + n)
    stride = k + pad
    a = int8_weights(rng, m, k, stride)
    w = int8_weights(rng, n, k, stride)
    a[0, :k] = 127           # the largest-magnitude dots
    w[0, :k] = -127
    ws = channel_scales(rng, n)
    a_scale = rng.uniform(1e-3, 3e-2, m).astype(np.float32)
    acc = gpu_acc(a, w, m, n, k, stride)
    ref_acc = oracle.gemm_i32(a, w, m, n, k, stride)
    assert np.array_equal(acc, ref_acc)
    assert np.array_equal(gpu_epilogue("plain", a, w, ws, a_scale, m, n, k, stride),
                          oracle.epilogue_plain(ref_acc, ws, a_scale))
    bias = f16_bits(rng.standard_normal(n) * 0.02)
    assert np.array_equal(gpu_epilogue("bias", a, w, ws, a_scale, m, n, k, stride, bias=bias),
                          oracle.epilogue_bias(ref_acc, ws, a_scale, bias))
    gate = rng.uniform(0.5, 1.5, n).astype(np.float32)
    prior = bf16_bits(rng.standard_normal(m * n))
    for mode in ("resid", "resid_wide"):
        got = gpu_epilogue(mode, a, w, ws, a_scale, m, n, k, stride, gate=gate, prior=prior)
        assert np.array_equal(got, oracle.epilogue_resid(ref_acc, ws, a_scale, gate, prior))
    assert np.array_equal(gpu_epilogue("swiglu", a, w, ws, a_scale, m, n, k, stride),
                          oracle.epilogue_swiglu(ref_acc, ws, a_scale))


def test_rows_past_m_are_never_written():
    rng = np.random.default_rng(11)
    m, k, n = 300, 256, 256
    a = int8_weights(rng, 512, k)  # the buffer holds more rows than m
    w = int8_weights(rng, n, k)
    out = torch.full((512, n), 0x5A5A, dtype=torch.int16, device="cuda")
    k2.gemm_i8(dev(a), dev(w), dev(channel_scales(rng, n)), dev(np.ones(512, np.float32)),
               out.view(torch.float16), cfg=cfg(k, n, k), m=m)
    sync()
    assert np.all(host(out)[m:] == 0x5A5A)


@pytest.mark.parametrize("n", [12288, 9216])
def test_north_star_shape_checksums_and_sampled_rows(n):
    # M=4096, K=3072 with N=12288 (the north star, 256x256 tiles) and N=9216 (the QKV
    # GEMM of the bench step, 256x192 tiles): full-size row and column checksums of the
    # int32 accumulators (size-independent identities) plus exact rows against the
    # oracle.
    rng = np.random.default_rng(12)
    m, k = 4096, 3072
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    A, W = dev(a), dev(w)
    acc = torch.empty((m, n), dtype=torch.int32, device="cuda")
    k2.gemm_i8_acc(A, W, acc, cfg=cfg(k, n, k), m=m)
    col = W.to(torch.int64).sum(0)                      # [k]
    row_check = (A.to(torch.int64) * col).sum(1)        # [m]
    assert torch.equal(acc.to(torch.int64).sum(1), row_check)
    arow = A.to(torch.int64).sum(0)                     # [k]
    col_check = (W.to(torch.int64) * arow).sum(1)       # [n]
    assert torch.equal(acc.to(torch.int64).sum(0), col_check)
    rows = np.sort(rng.choice(m, 24, replace=False))
    got = host(acc)[rows]
    ref = oracle.gemm_i32(a[rows], w, len(rows), n, k, k)
    assert np.array_equal(got, ref)
    ws = channel_scales(rng, n)
    a_scale = rng.uniform(1e-3, 3e-2, m).astype(np.float32)
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    k2.gemm_i8(A, W, dev(ws), dev(a_scale), out, cfg=cfg(k, n, k), m=m)
    sync()
    assert np.array_equal(host(out)[rows], oracle.epilogue_plain(ref, ws, a_scale[rows]))


@pytest.mark.parametrize("inputs", [6144, 16384])
def test_convrot_known_answer_through_prepare_and_gemm(inputs):
    # src/training/quantized.rs:187-224: exact bf16 base projection.
    g = np.load(os.path.join(GOLDEN, f"convrot_kat_{inputs}.npz"))
    tokens, outputs = int(g["tokens"]), int(g["outputs"])
    h = dev(g["h"].reshape(tokens, inputs), torch.float16)
    q = torch.empty((tokens, inputs), dtype=torch.int8, device="cuda")
    s = torch.empty(tokens, dtype=torch.float32, device="cuda")
    k2.prepare_plain_i8(h, q, s, width=inputs, out_stride=inputs)
    out = torch.empty((tokens, outputs), dtype=torch.float16, device="cuda")
    k2.gemm_i8(q, dev(g["weights"]), dev(g["scales"]), s, out, cfg=cfg(inputs, outputs, inputs))
    sync()
    want = oracle.f16_bits(bf16_value(g["base_bf16"]))
    assert np.array_equal(host(out), want)


@pytest.mark.parametrize("m", [64, 5])
def test_swiglu_reads_the_sixteen_row_interleave(m):
    # Gate rows of group j are rows 32j..32j+15 and up rows 32j+16..32j+31
    # (src/checkpoint/plan.rs:193-208): permuting the interleave must change the output
    # exactly as the oracle says. m=5 runs the few-token kernel, whose workgroups each
    # take half a group (8 gate rows and their 8 up rows).
    rng = np.random.default_rng(13)
    k, n = 256, 256
    a = int8_weights(rng, m, k)
    w = int8_weights(rng, n, k)
    ws = channel_scales(rng, n)
    sc = rng.uniform(1e-3, 3e-2, m).astype(np.float32)
    base = gpu_epilogue("swiglu", a, w, ws, sc, m, n, k, k)
    swapped = w.reshape(n // 32, 2, 16, k)[:, ::-1].reshape(n, k).copy()
    ws_swapped = ws.reshape(n // 32, 2, 16)[:, ::-1].reshape(n).copy()
    other = gpu_epilogue("swiglu", a, swapped, ws_swapped, sc, m, n, k, k)
    ref_acc = oracle.gemm_i32(a, swapped, m, n, k, k)
    assert np.array_equal(other, oracle.epilogue_swiglu(ref_acc, ws_swapped, sc))
    assert not np.array_equal(base, other)


def test_split_k_calls_on_two_streams_keep_their_own_workspace():
    # (256, 9728, 2560) splits K: its int32 partial sums go to a workspace per stream.
    # Two streams running such calls at the same time must each get their own results.
    rng = np.random.default_rng(21)
    m, k, n = 256, 9728, 2560
    w = int8_weights(rng, n, k)
    ws = channel_scales(rng, n)
    inputs = [int8_weights(rng, m, k) for _ in range(2)]
    a_scale = rng.uniform(1e-3, 3e-2, m).astype(np.float32)
    want = [oracle.epilogue_plain(oracle.gemm_i32(a, w, m, n, k, k), ws, a_scale) for a in inputs]
    W, WS, AS = dev(w), dev(ws), dev(a_scale)
    A = [dev(a) for a in inputs]
    outs = [torch.empty((m, n), dtype=torch.float16, device="cuda") for _ in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for _ in range(4):  # interleaved launches, so the two streams' kernels overlap
        for i in range(2):
            with torch.cuda.stream(streams[i]):
                k2.gemm_i8(A[i], W, WS, AS, outs[i], cfg=cfg(k, n, k), m=m)
    torch.cuda.synchronize()
    for i in range(2):
        assert np.array_equal(host(outs[i]), want[i]), i
