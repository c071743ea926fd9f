"""The device sigmoid of the gated prepare (kernels/prepare_gated_i8.loom:97-101) and the
SwiGLU epilogue (kernels/gemm_i8_swiglu_256.loom:649-652) against its CPU definition,
1 / (1 + exp(-g)) with the oracle's exp and an IEEE f32 division, bit for bit.

The device evaluates the same function by other steps: the exponential's special cases
are selected instead of branched around, and the division is the hardware reciprocal
plus one fma correction (the IEEE division only where 1 + exp(-g) >= 2^126, whose
quotients are subnormal). The inputs cover the whole f32 range at a fine stride, every
value in the bands where those steps change (the cutoffs of the exponential, the
switch to the division, subnormal quotients, overflow to infinity) and the specials.
"""

import numpy as np
import pytest
import torch

import oracle
from gpu_common import k2, sync

pytestmark = pytest.mark.gpu


def cpu_sigmoid(g: np.ndarray) -> np.ndarray:
    g = np.asarray(g, np.float32)
    with np.errstate(over="ignore", divide="ignore", invalid="ignore"):
        e = oracle.expf(np.float32(0.0) - g)
        return np.float32(1.0) / (np.float32(1.0) + e)


def band(lo: float, hi: float) -> np.ndarray:
    """Every f32 from lo to hi (same sign, |lo| <= |hi|)."""
    a = np.array([lo, hi], np.float32).view(np.uint32)
    return np.arange(min(a), max(a) + 1, dtype=np.uint32).view(np.float32)


def inputs() -> np.ndarray:
    stride = np.arange(0, 1 << 32, 251, dtype=np.uint64).astype(np.uint32).view(np.float32)
    parts = [
        stride,
        band(-87.0, -88.0),     # 1 + exp(-g) crosses 2^126: reciprocal -> division
        band(-103.5, -104.5),   # exp(-g) overflows to infinity
        band(88.5, 89.0),       # exp(-g) underflows to zero (cutoff -103.97 of -g)
        band(-0.01, -0.02), band(0.01, 0.02),
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.4028235e38,
                  -3.4028235e38], np.float32),
        # every f16 value: the gated prepare looks bf16(sigmoid(g)) up in a table built
        # from this function for each of them
        np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32),
    ]
    return np.concatenate(parts)


def test_device_sigmoid_is_bit_identical_to_the_cpu_definition():
    x = inputs()
    want = cpu_sigmoid(x)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty_like(xd)
    k2.sigmoid_f32(xd, out)
    sync()
    got = out.cpu().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    diff = got.view(np.uint32)[~nan] != want.view(np.uint32)[~nan]
    assert not diff.any(), (int(diff.sum()), x[~nan][diff][:8], got[~nan][diff][:8],
                            want[~nan][diff][:8])
    # the bands above do reach the division path and subnormal quotients
    assert (want[~nan] < np.float32(2.0 ** -126)).any() and (want == 0).any()


def test_device_sigmoid_over_every_f32_input():
    # All 2^32 bit patterns, in chunks of 2^28: the device function against the oracle's
    # definition (ora_sigmoid_bits_n), bit for bit; NaN inputs give NaN on both.
    chunk = 1 << 28
    out = torch.empty(chunk, dtype=torch.float32, device="cuda")
    for c in range((1 << 32) // chunk):
        first = c * chunk
        start = first if first < (1 << 31) else first - (1 << 32)
        x = torch.arange(start, start + chunk, dtype=torch.int32, device="cuda").view(torch.float32)
        k2.sigmoid_f32(x, out)
        got = out.cpu().numpy()
        want = oracle.sigmoid_of_bits(first, chunk)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan), c
        diff = got.view(np.uint32)[~nan] != want.view(np.uint32)[~nan]
        assert not diff.any(), (c, int(diff.sum()))


def test_mfma_probe_counts_every_mfma():
    # With bytes of 1 every v_mfma_i32_32x32x32_i8 adds 32 to each accumulator: a lane's
    # eight chains of 16 accumulators sum to 4096 per step. Pseudo-random operands give
    # the same sums on every run.
    import krea2_w8a8 as k2
    out = torch.zeros(3 * 256, dtype=torch.int32, device="cuda")
    k2.probe_mfma_i8(out, blocks=3, iters=7, random=False)
    torch.cuda.synchronize()
    assert torch.all(out == 4096 * 7)
    a = torch.zeros_like(out)
    b = torch.zeros_like(out)
    k2.probe_mfma_i8(a, blocks=3, iters=5, random=True, seed=9)
    k2.probe_mfma_i8(b, blocks=3, iters=5, random=True, seed=9)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and int(a.abs().sum()) > 0
