"""Pins the CPU oracle (oracle/w8a8_oracle.c) before it is trusted as the GPU checker.

Every check here is independent of the oracle's own formulas: the reference tests'
known answers and tolerances (fixtures from tests/golden/make_golden.py), library
conversions (numpy binary16, torch bfloat16, numpy exp), brute-force integer dots,
and invariants of the Hadamard rotation.
"""

import os

import numpy as np
import pytest
import torch

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
H4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]])


def golden(name):
    return np.load(os.path.join(GOLDEN, name))


def bf16_value(bits):
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def close(actual, expected, abs_tol, rel_tol):
    """tests/common/mod.rs:7-15: every element finite and within abs + rel*|expected|."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert actual.shape == expected.shape
    assert np.all(np.isfinite(actual))
    bad = np.abs(actual - expected) > abs_tol + rel_tol * np.abs(expected)
    assert not bad.any(), f"{bad.sum()} elements out of tolerance, first at {np.argwhere(bad)[0]}"


@pytest.mark.parametrize("width", [2048, 6144, 16384])
def test_plain_prepare_matches_the_reference_known_answers_bit_for_bit(width):
    # tests/quantized.rs:514-569: zero, normal and subnormal rows, padding untouched.
    g = golden(f"plain_kat_{width}.npz")
    stride = int(g["stride"])
    q = np.full((3, stride), -91, np.int8)  # 0xa5
    q, s = oracle.prepare_plain(g["h"], width, stride, q=q)
    assert np.array_equal(s.view(np.uint32), g["scales"].view(np.uint32))
    assert np.array_equal(q[:, :width], g["codes"])
    assert np.all(q[:, width:] == -91)


@pytest.mark.parametrize("kind", ["norm", "gated", "plain"])
def test_prepares_match_the_kronecker_hadamard_within_the_reference_tolerance(kind):
    # tests/quantized.rs:476-510: scale within 0.2 %, codes within +-1 with < 2 % mismatches,
    # pad bytes untouched.
    g = golden(f"kronecker_{kind}.npz")
    tokens, width, stride = int(g["tokens"]), int(g["width"]), int(g["stride"])
    q = np.full((tokens, stride), -91, np.int8)
    if kind == "norm":
        q, s = oracle.prepare_norm(g["norm_input"], g["norm"], g["modulation"], g["shift"], width,
                                   stride, 1e-5, q=q)
    elif kind == "gated":
        q, s = oracle.prepare_gated(g["half_input"], g["gate"], width, stride,
                                    int(g["gate_stride"]), q=q)
    else:
        q, s = oracle.prepare_plain(g["half_input"], width, stride, q=q)
    rotated, scale = g["rotated"], g["scale"]
    assert np.all(np.abs(s - scale) <= scale * 0.002 + 1e-30)
    want = np.clip(np.rint(rotated / scale[:, None]), -127, 127).astype(np.int32)
    code = q[:, :width].astype(np.int32)
    assert np.all(np.abs(code - want) <= 1)
    assert (code != want).mean() < 0.02
    assert np.all(q[:, width:] == -91)


def test_rotation_is_the_regular_hadamard_in_every_prepare():
    # A one-hot row at position j rotates to column j of H4(x)H4(x)H4(x)H4 / 16: every
    # entry is +-1/16, so every code is +-127 with the matrix's sign. Catches a wrong
    # stage order, sign or stride in any of the three prepares.
    width = 512
    hmat = np.ones((256, 256), np.int64)
    ii, jj = np.meshgrid(np.arange(256), np.arange(256), indexing="ij")
    for _ in range(4):
        hmat *= H4[ii % 4, jj % 4]
        ii, jj = ii // 4, jj // 4
    tokens = 256
    onehot = np.zeros((tokens, width), np.float32)
    onehot[np.arange(tokens), 256 + np.arange(tokens)] = 1.0  # second group of each row
    f16 = onehot.astype(np.float16).view(np.uint16)
    expect = np.zeros((tokens, width), np.int64)
    expect[:, 256:] = 127 * hmat.T  # row t: column t of H
    q, s = oracle.prepare_plain(f16, width, width)
    assert np.array_equal(q.astype(np.int64), expect)
    assert np.allclose(s, (1 / 16) / 127)
    # gated: sigmoid(30) rounds to 1 in bf16, so the formed row is the one-hot row
    gate = np.full((tokens, width), 30.0, np.float32).astype(np.float16).view(np.uint16)
    q, s = oracle.prepare_gated(f16, gate, width, width, width)
    assert np.array_equal(q.astype(np.int64), expect)
    # norm: rms of a one-hot row of width 512 is 1/sqrt(512): the formed row is one-hot
    bf = (onehot.view(np.uint32) >> 16).astype(np.uint16)
    zeros = np.zeros(width, np.float32)
    q, s = oracle.prepare_norm(bf, zeros, zeros, zeros, width, width, 0.0)
    assert np.array_equal(q.astype(np.int64), expect)


@pytest.mark.parametrize("name", [
    "gemm_plain_17x128x128_pad0", "gemm_plain_257x384x256_pad128",
    "gemm_resid_17x128x128_pad0", "gemm_resid_257x384x256_pad128",
    "gemm_swiglu_17x128x128_pad0", "gemm_swiglu_257x384x256_pad128",
    "gemm_resid_wide_17x128x256_pad0", "gemm_resid_wide_257x384x512_pad128",
])
def test_gemm_and_epilogues_match_the_reference_integer_test(name):
    # tests/quantized.rs:171-280: exact int32 dots; outputs within abs 2e-3 + rel 4e-3 and
    # on the bf16 grid.
    g = golden(f"{name}.npz")
    m, k, n, stride = (int(g[x]) for x in ("m", "k", "n", "stride"))
    acc = oracle.gemm_i32(g["a"], g["w"], m, n, k, stride)
    assert np.array_equal(acc, g["dot"])
    if "_resid" in name:
        out = bf16_value(oracle.epilogue_resid(acc, g["ws"], g["a_scale"], g["gates"],
                                               g["residual"]))
    elif "_swiglu" in name:
        out = oracle.epilogue_swiglu(acc, g["ws"], g["a_scale"]).view(np.float16).astype(np.float32)
    else:
        out = oracle.epilogue_plain(acc, g["ws"], g["a_scale"]).view(np.float16).astype(np.float32)
    assert np.array_equal(bf16_value(oracle.bf16_bits(out)), out)
    close(out, g["want"], 2e-3, 4e-3)


@pytest.mark.parametrize("inputs", [6144, 16384])
def test_plain_prepare_gemm_and_epilogue_match_the_convrot_known_answer(inputs):
    # src/training/quantized.rs:187-224: assert_eq! on bf16((dot as f32 * ws) * scale).
    g = golden(f"convrot_kat_{inputs}.npz")
    tokens, outputs = int(g["tokens"]), int(g["outputs"])
    q, s = oracle.prepare_plain(g["h"], inputs, inputs)
    acc = oracle.gemm_i32(q, g["weights"], tokens, outputs, inputs, inputs)
    out = oracle.epilogue_plain(acc, g["scales"], s)
    want = oracle.f16_bits(bf16_value(g["base_bf16"]))
    assert np.array_equal(out, want)


def test_gemm_dot_is_the_brute_force_integer_dot_at_the_extremes():
    rng = np.random.default_rng(7)
    m, n, k, stride = 5, 7, 384, 448
    a = rng.integers(-127, 128, (m, stride), dtype=np.int8)
    w = rng.integers(-127, 128, (n, stride), dtype=np.int8)
    a[0, :k] = 127
    w[0, :k] = -127
    acc = oracle.gemm_i32(a, w, m, n, k, stride)
    want = a[:, :k].astype(np.int64) @ w[:, :k].astype(np.int64).T
    assert np.array_equal(acc, want)
    assert acc[0, 0] == -127 * 127 * k


def test_f16_rounding_is_numpy_binary16():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 4_000_000, dtype=np.uint64).astype(np.uint32)
    edges = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x477FF000, 0x477FEFFF, 0x477FE000,
                      0x38800000, 0x387FFFFF, 0x33000000, 0x33000001, 0x32FFFFFF, 0x33800000,
                      0x7F7FFFFF], np.uint32)
    x = np.concatenate([bits, edges]).view(np.float32)
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f16_bits(x), want)


def test_bf16_rounding_is_torch_bfloat16():
    rng = np.random.default_rng(2)
    bits = rng.integers(0, 2**32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.bf16_bits(x), want)


def test_exp_is_within_two_ulp_of_the_true_exponential():
    x = np.linspace(-87.0, 88.7, 3_000_001).astype(np.float32)
    y = oracle.expf(x).astype(np.float64)
    true = np.exp(x.astype(np.float64))
    ulp = np.spacing(true.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(y - true) / ulp) <= 2.0
    assert np.all(np.diff(y) >= 0)  # monotone
    special = oracle.expf(np.array([0.0, -0.0, np.inf, -np.inf, 89.0, -110.0], np.float32))
    assert special[0] == 1.0 and special[1] == 1.0
    assert np.isposinf(special[2]) and special[3] == 0.0
    assert np.isposinf(special[4]) and special[5] == 0.0
    assert np.isnan(oracle.expf(np.array([np.nan], np.float32))[0])


def test_norm_sum_of_squares_is_the_row_energy():
    rng = np.random.default_rng(3)
    for width in (256, 2048, 3072, 6144, 12288):
        x = rng.standard_normal(width).astype(np.float32)
        bits = (x.view(np.uint32) >> 16).astype(np.uint16)  # truncation: any bf16 row will do
        xv = bf16_value(bits).astype(np.float64)
        got = oracle.norm_sum_squares(bits)
        assert abs(got - np.sum(xv * xv)) <= 1e-5 * np.sum(xv * xv)


def test_quantiser_scale_is_amax_over_127_and_codes_saturate():
    # A row whose rotated amax is known: all entries +1 in a 256-group rotate to
    # 16 * e_0-ish patterns; check the scale formula s = max(amax*16,1e-30)/127 (f32) and
    # that every code is in [-127, 127].
    rng = np.random.default_rng(4)
    h = (rng.standard_normal((16, 1024)) * 3).astype(np.float16)
    q, s = oracle.prepare_plain(h.view(np.uint16), 1024, 1024)
    assert q.min() >= -127 and q.max() <= 127
    assert np.all(np.abs(q).max(axis=1) == 127)
    z = np.zeros((2, 512), np.float16)
    q, s = oracle.prepare_plain(z.view(np.uint16), 512, 512)
    assert np.all(q == 0)
    assert np.all(s == np.float32(np.float32(1e-30) / np.float32(127.0)))


def _bias_case(seed, m=37, n=96, k=256):
    rng = np.random.default_rng(seed)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    w = rng.integers(-127, 128, (n, k), dtype=np.int8)
    ws = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    s = rng.uniform(1e-3, 5e-2, m).astype(np.float32)
    bias = (rng.standard_normal(n) * 0.02).astype(np.float16)
    acc = a.astype(np.int64) @ w.astype(np.int64).T  # brute-force dot, not the oracle's
    return acc.astype(np.int32), ws, s, bias


def test_bias_epilogue_with_a_zero_bias_is_the_plain_epilogue():
    # The bias epilogue adds one f32 term before the bf16 rounding: with a -0.0 bias
    # (x + -0 == x for every x, +0 included) it must equal the plain epilogue bit for bit,
    # whose formula the reference's ConvRot known answer pins.
    acc, ws, s, bias = _bias_case(11)
    neg_zero = np.full(bias.shape, 0x8000, np.uint16)
    assert np.array_equal(oracle.epilogue_bias(acc, ws, s, neg_zero),
                          oracle.epilogue_plain(acc, ws, s))
    pos_zero = np.zeros(bias.shape, np.uint16)
    assert np.array_equal(oracle.epilogue_bias(acc, ws, s, pos_zero),
                          oracle.epilogue_plain(acc, ws, s))


def test_bias_epilogue_of_a_zero_accumulator_is_the_rounded_bias():
    # acc = 0 leaves exactly the bias: out = f16(bf16(bias)), with bf16 rounding by torch
    # and f16 by numpy (independent of the oracle's conversions).
    _, ws, s, bias = _bias_case(12)
    acc = np.zeros((s.size, ws.size), np.int32)
    out = oracle.epilogue_bias(acc, ws, s, bias.view(np.uint16))
    want = torch.from_numpy(bias.astype(np.float32)).to(torch.bfloat16).float().numpy()
    want = np.broadcast_to(want.astype(np.float16).view(np.uint16), out.shape)
    assert np.array_equal(out, want)


def test_bias_epilogue_is_within_one_bf16_ulp_of_the_exact_value():
    # Closed form in f64: v = acc * ws * as + bias. The f32 evaluation rounds twice before
    # the bf16 rounding, so the stored value is within one bf16 ulp of bf16(v) (and the
    # store is on the bf16 grid); a dropped or mis-signed bias term is off by far more.
    acc, ws, s, bias = _bias_case(13)
    out = oracle.epilogue_bias(acc, ws, s, bias.view(np.uint16)).view(np.float16).astype(np.float64)
    v = acc.astype(np.float64) * ws.astype(np.float64)[None, :] * s.astype(np.float64)[:, None]
    v += bias.astype(np.float64)[None, :]
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -30))) - 7)
    # three f32 roundings before the bf16 one: each within 2^-24 of its operands' size
    f32_err = 4 * 2.0 ** -24 * (np.abs(v - bias.astype(np.float64)[None, :]) +
                                np.abs(bias.astype(np.float64))[None, :])
    assert np.all(np.abs(out - v) <= ulp + f32_err)
    assert np.array_equal(bf16_value(oracle.bf16_bits(out.astype(np.float32))), out.astype(np.float32))
    # the bias matters at this scale: dropping it moves many outputs by more than an ulp
    no_bias = v - bias.astype(np.float64)[None, :]
    assert (np.abs(out - no_bias) > 2 * ulp).mean() > 0.1


def test_fused_cpu_gemm_is_the_integer_gemm_then_the_plain_epilogue():
    # ora_gemm_i8 (the fused CPU baseline) against the separately pinned parts, at a
    # padded row stride and a ragged token count.
    rng = np.random.default_rng(14)
    m, n, k, stride = 45, 160, 384, 448
    a = rng.integers(-127, 128, (m, stride), dtype=np.int8)
    w = rng.integers(-127, 128, (n, stride), dtype=np.int8)
    ws = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    s = rng.uniform(1e-3, 5e-2, m).astype(np.float32)
    want = oracle.epilogue_plain(oracle.gemm_i32(a, w, m, n, k, stride), ws, s)
    for threads in (1, 0):
        assert np.array_equal(oracle.gemm_i8(a, w, m, n, k, stride, ws, s, threads=threads), want)
