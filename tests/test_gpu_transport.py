"""GPU parity of the bf16 <-> f16 transport (kernels/native/lora_transport.loom) and of
the projection caller built on it, Quantized::forward (src/training/quantized.rs:51-112).

The transport is checked against numpy's IEEE f32 -> f16 conversion and the bf16
rounding of src/numerics.rs:18-26 (both round to nearest even), on every special class
(zeros, subnormals, the f16 overflow boundary, infinities) and on counts that leave a
tail past the 8-element vectors. The forward pass is checked against the reference's own
exact known answer (src/training/quantized.rs:187-224)."""

import os

import numpy as np
import pytest
import torch

from gpu_common import bf16_bits, bf16_value, dev, host, k2, sync

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def special_values():
    return np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6, 6.0e-8,
                     5.9e-8, 2.9e-8, 3.0e-8, 1e-10, 6.1e-5, np.inf, -np.inf, 0.33333334,
                     1.0009765625, 1.00048828125, 2047.5, 4097.0], np.float32)


@pytest.mark.parametrize("count", [1, 7, 8, 9, 4099, 1 << 20])
def test_bf16_to_f16_is_the_ieee_conversion(count):
    rng = np.random.default_rng(count)
    x32 = (rng.standard_normal(count) * np.exp(rng.uniform(-20, 14, count))).astype(np.float32)
    sv = special_values()
    x32[: min(count, sv.size)] = sv[: min(count, sv.size)]
    x = bf16_bits(x32)
    out = torch.empty(count, dtype=torch.float16, device="cuda")
    k2.lora_transport(dev(x, torch.bfloat16), out, reverse=1)
    sync()
    with np.errstate(over="ignore"):  # values past 65504 become infinities, as intended
        want = bf16_value(x).astype(np.float16).view(np.uint16)
    assert np.array_equal(host(out), want)


@pytest.mark.parametrize("count", [1, 15, 4099, 1 << 20])
def test_f16_to_bf16_rounds_to_nearest_even(count):
    rng = np.random.default_rng(count + 1)
    h = rng.integers(0, 0x7C00, count, dtype=np.uint16)  # every finite magnitude
    h |= (rng.integers(0, 2, count, dtype=np.uint16) << 15)  # both signs
    special = np.array([0x7C00, 0xFC00, 0x0001, 0x8001], np.uint16)  # infinities, subnormals
    h[: min(count, 4)] = special[: min(count, 4)]
    out = torch.empty(count, dtype=torch.bfloat16, device="cuda")
    k2.lora_transport(dev(h, torch.float16), out, reverse=2)
    sync()
    want = bf16_bits(h.view(np.float16).astype(np.float32))
    assert np.array_equal(host(out), want)


def test_transport_leaves_memory_past_count_untouched():
    x = dev(bf16_bits(np.ones(64, np.float32)), torch.bfloat16)
    out = torch.full((64,), 7, dtype=torch.int16, device="cuda")
    k2.lora_transport(x, out.view(torch.float16), reverse=1, count=13)
    sync()
    got = host(out)
    assert np.all(got[:13].view(np.uint16) == 0x3C00) and np.all(got[13:] == 7)


@pytest.mark.parametrize("inputs", [6144, 16384])
def test_quantized_forward_is_the_reference_known_answer(inputs):
    g = np.load(os.path.join(GOLDEN, f"convrot_kat_{inputs}.npz"))
    tokens, outputs = int(g["tokens"]), int(g["outputs"])
    proj = k2.Quantized.load(dev(g["weights"].reshape(outputs, inputs)), dev(g["scales"]))
    assert proj.pitch == k2.shape.gemm_pitch(inputs)
    out = proj.forward(dev(g["x_bf16"].reshape(tokens, inputs), torch.bfloat16))
    sync()
    assert np.array_equal(host(out), g["base_bf16"])
