"""GPU parity of the activation prepares against the reference tests and the CPU oracle.

int8 codes and f32 scales must be bit-exact with the oracle; padding bytes past the
row width must be untouched (tests/quantized.rs:501-505, 566)."""

import os

import numpy as np
import pytest
import torch

import oracle
from gpu_common import (PAD, activations, bf16_bits, dev, f16_bits, host, k2, sync)

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def run_plain(h_bits, tokens, width, stride):
    h = dev(h_bits.reshape(tokens, width), torch.float16)
    q = torch.full((tokens, stride), PAD, dtype=torch.int8, device="cuda")
    s = torch.zeros(tokens, dtype=torch.float32, device="cuda")
    k2.prepare_plain_i8(h, q, s, width=width, out_stride=stride)
    sync()
    return host(q), host(s)


def run_norm(h_bits, ns, ms, sh, tokens, width, stride, eps):
    h = dev(h_bits.reshape(tokens, width), torch.bfloat16)
    q = torch.full((tokens, stride), PAD, dtype=torch.int8, device="cuda")
    s = torch.zeros(tokens, dtype=torch.float32, device="cuda")
    k2.prepare_norm_i8(h, dev(ns), dev(ms), dev(sh), q, s, width=width, out_stride=stride, eps=eps)
    sync()
    return host(q), host(s)


def run_gated(a_bits, g_bits, tokens, width, stride, gate_stride):
    a = dev(a_bits.reshape(tokens, width), torch.float16)
    g = dev(g_bits.reshape(tokens, gate_stride), torch.float16)
    q = torch.full((tokens, stride), PAD, dtype=torch.int8, device="cuda")
    s = torch.zeros(tokens, dtype=torch.float32, device="cuda")
    k2.prepare_gated_i8(a, g, q, s, width=width, out_stride=stride, gate_stride=gate_stride)
    sync()
    return host(q), host(s)


def assert_same(q, s, q_ref, s_ref, width):
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q[:, :width], q_ref[:, :width])
    assert np.all(q[:, width:] == PAD)


@pytest.mark.parametrize("width", [2048, 6144, 16384])
def test_plain_prepare_is_bit_exact_on_the_reference_known_answers(width):
    g = np.load(os.path.join(GOLDEN, f"plain_kat_{width}.npz"))
    stride = int(g["stride"])
    q, s = run_plain(g["h"], 3, width, stride)
    assert np.array_equal(s.view(np.uint32), g["scales"].view(np.uint32))
    assert np.array_equal(q[:, :width], g["codes"])
    assert np.all(q[:, width:] == PAD)


@pytest.mark.parametrize("kind", ["norm", "gated", "plain"])
def test_prepares_match_the_kronecker_test_and_the_oracle(kind):
    g = np.load(os.path.join(GOLDEN, f"kronecker_{kind}.npz"))
    tokens, width, stride = int(g["tokens"]), int(g["width"]), int(g["stride"])
    if kind == "norm":
        q, s = run_norm(g["norm_input"], g["norm"], g["modulation"], g["shift"], tokens, width,
                        stride, 1e-5)
        q_ref, s_ref = oracle.prepare_norm(g["norm_input"], g["norm"], g["modulation"], g["shift"],
                                           width, stride, 1e-5)
    elif kind == "gated":
        gs = int(g["gate_stride"])
        q, s = run_gated(g["half_input"], g["gate"], tokens, width, stride, gs)
        q_ref, s_ref = oracle.prepare_gated(g["half_input"], g["gate"], width, stride, gs)
    else:
        q, s = run_plain(g["half_input"], tokens, width, stride)
        q_ref, s_ref = oracle.prepare_plain(g["half_input"], width, stride)
    assert_same(q, s, q_ref, s_ref, width)
    # and the reference's own tolerance against the f64 Kronecker rotation
    rotated, scale = g["rotated"], g["scale"]
    assert np.all(np.abs(s - scale) <= scale * 0.002 + 1e-30)
    want = np.clip(np.rint(rotated / scale[:, None]), -127, 127)
    assert np.all(np.abs(q[:, :width] - want) <= 1)


WIDTHS = [256, 2048, 2560, 3072, 9728, 12288, 16384, 32768]


@pytest.mark.parametrize("width", WIDTHS)
def test_plain_prepare_is_bit_exact_with_the_oracle(width):
    rng = np.random.default_rng(100 + width)
    tokens, stride = 7, width + 64
    x = activations(rng, tokens, width)
    x[1] = 0.0                      # zero row: scale 1e-30/127, codes 0
    x[2] *= np.float32(1e-6)        # subnormal f16 inputs
    x[3] = np.clip(x[3] * 3000, -65504, 65504)  # near the f16 range
    h = f16_bits(x)
    q, s = run_plain(h, tokens, width, stride)
    q_ref, s_ref = oracle.prepare_plain(h, width, stride)
    assert_same(q, s, q_ref, s_ref, width)


@pytest.mark.parametrize("width", WIDTHS)
def test_norm_prepare_is_bit_exact_with_the_oracle(width):
    rng = np.random.default_rng(200 + width)
    tokens, stride = 7, width + 64
    x = activations(rng, tokens, width)
    x[1] = 0.0
    x[2] *= np.float32(1e-20)
    h = bf16_bits(x)
    ns = (rng.uniform(0.5, 1.5, width) - 1.0).astype(np.float32)
    ms = (rng.standard_normal(width) * 0.1).astype(np.float32)
    sh = (rng.standard_normal(width) * 0.1).astype(np.float32)
    q, s = run_norm(h, ns, ms, sh, tokens, width, stride, 1e-6)
    q_ref, s_ref = oracle.prepare_norm(h, ns, ms, sh, width, stride, 1e-6)
    assert_same(q, s, q_ref, s_ref, width)


@pytest.mark.parametrize("case", ["zero", "signed_zero", "one_scale", "one_shift"])
def test_norm_prepare_with_and_without_modulation(case):
    # With every modulation scale and shift zero (+0 or -0) the kernel skips the two
    # identity steps; one nonzero element anywhere must bring them back. Both against
    # the oracle, which always runs the whole formula.
    rng = np.random.default_rng(250)
    tokens, width = 301, 3072
    h = bf16_bits(activations(rng, tokens, width))
    h[5] = 0x8000  # a row of -0.0
    ns = (rng.uniform(0.5, 1.5, width) - 1.0).astype(np.float32)
    ms = np.zeros(width, np.float32)
    sh = np.zeros(width, np.float32)
    if case == "signed_zero":
        ms[::3] = -0.0
        sh[1::3] = -0.0
    elif case == "one_scale":
        ms[width - 1] = 0.25
    elif case == "one_shift":
        sh[17] = -0.5
    q, s = run_norm(h, ns, ms, sh, tokens, width, width, 1e-6)
    q_ref, s_ref = oracle.prepare_norm(h, ns, ms, sh, width, width, 1e-6)
    assert_same(q, s, q_ref, s_ref, width)


@pytest.mark.parametrize("width", WIDTHS)
def test_gated_prepare_is_bit_exact_with_the_oracle(width):
    rng = np.random.default_rng(300 + width)
    tokens, stride, gate_stride = 7, width + 64, width + 264
    a = f16_bits(activations(rng, tokens, width))
    g = np.zeros((tokens, gate_stride), np.float32)
    g[:, :width] = activations(rng, tokens, width, scale=4.0)
    g[1, :width] = np.linspace(-120, 120, width)  # exp overflow / underflow ranges
    gb = f16_bits(g)
    q, s = run_gated(a, gb, tokens, width, stride, gate_stride)
    q_ref, s_ref = oracle.prepare_gated(a, gb, width, stride, gate_stride)
    assert_same(q, s, q_ref, s_ref, width)


def test_gated_prepare_over_every_gate_value():
    # The gate factor bf16(sigmoid(g)) comes from a table indexed by the gate's 16 bits:
    # rows holding every f16 pattern (NaNs replaced by 0), shuffled, with attn values
    # near 1 so that each product keeps the factor's magnitude.
    rng = np.random.default_rng(77)
    tokens, width = 16, 4096
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    nan = np.isnan(bits.view(np.float16))
    bits[nan] = 0
    gb = rng.permutation(bits).reshape(tokens, width)
    a = f16_bits(rng.uniform(0.5, 1.5, (tokens, width)).astype(np.float32))
    q, s = run_gated(a, gb, tokens, width, width, width)
    q_ref, s_ref = oracle.prepare_gated(a, gb, width, width, width)
    assert_same(q, s, q_ref, s_ref, width)


@pytest.mark.parametrize("kind", ["norm", "plain", "gated"])
def test_prepares_are_bit_exact_at_the_baseline_shape(kind):
    # M=4096 (and 4544) tokens of width 3072.
    rng = np.random.default_rng(400)
    for tokens, width in ((4096, 3072), (4544, 3072)):
        x = activations(rng, tokens, width)
        if kind == "plain":
            h = f16_bits(x)
            q, s = run_plain(h, tokens, width, width)
            q_ref, s_ref = oracle.prepare_plain(h, width, width)
        elif kind == "norm":
            h = bf16_bits(x)
            ns = (rng.uniform(0.5, 1.5, width) - 1.0).astype(np.float32)
            z = np.zeros(width, np.float32)
            q, s = run_norm(h, ns, z, z, tokens, width, width, 1e-6)
            q_ref, s_ref = oracle.prepare_norm(h, ns, z, z, width, width, 1e-6)
        else:
            a = f16_bits(x)
            g = f16_bits(activations(rng, tokens, width))
            q, s = run_gated(a, g, tokens, width, width, width)
            q_ref, s_ref = oracle.prepare_gated(a, g, width, width, width)
        assert_same(q, s, q_ref, s_ref, width)


def test_a_single_token_and_the_largest_pitch():
    rng = np.random.default_rng(500)
    width, stride = 32768, 65536
    h = f16_bits(activations(rng, 1, width))
    q, s = run_plain(h, 1, width, stride)
    q_ref, s_ref = oracle.prepare_plain(h, width, stride)
    assert_same(q, s, q_ref, s_ref, width)
