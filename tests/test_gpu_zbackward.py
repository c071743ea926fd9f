"""The wide-tile GEMMs with odd rounds stepping through K backwards
(K2W8_GEMM_BACKWARD=1, gemm_kernel_backward): the same bits as the default order, since
the int32 sums do not depend on the order of the K steps; compared at the shapes whose
launches run several rounds of 256x192 and 256x256 tiles, for every epilogue that has
the backward form."""

import numpy as np
import pytest
import torch

from gpu_common import activations, bf16_bits, channel_scales, dev, int8_weights, k2

pytestmark = pytest.mark.gpu

SHAPES = [
    # (epilogue, m, k, n): configs[1] QKV (768 tiles of 256x192, 3 rounds), the north
    # star (768 tiles of 256x256), the block's wo with its residual (256x256 rounds
    # plus 128x128 tail columns), a SwiGLU-up and a bias GEMM
    ("plain", 4096, 3072, 9216),
    ("plain", 4096, 3072, 12288),
    ("resid", 4544, 3072, 3072),
    ("swiglu", 4608, 3072, 24576),
    ("bias", 4096, 3072, 3072),
]


@pytest.mark.parametrize("epi,m,k,n", SHAPES)
def test_backward_rounds_give_the_same_bits(epi, m, k, n, monkeypatch):
    rng = np.random.default_rng(m + n)
    a = dev(rng.integers(-127, 128, (m, k), dtype=np.int8))
    w = dev(int8_weights(rng, n, k))
    ws = dev(channel_scales(rng, n))
    s = dev(rng.uniform(1e-3, 3e-2, m).astype(np.float32))
    cfg = k2.GemmConfig(k_size=k, n_size=n, k_stride=k)
    bias = dev((rng.standard_normal(n) * 0.02).astype(np.float16))
    gate = dev(rng.uniform(0.5, 1.5, n).astype(np.float32))
    x0 = bf16_bits(activations(rng, m, n).reshape(-1)) if epi == "resid" else None
    outs = []
    for order in ("0", "1"):
        monkeypatch.setenv("K2W8_GEMM_BACKWARD", order)
        if epi == "plain":
            c = torch.zeros((m, n), dtype=torch.float16, device="cuda")
            k2.gemm_i8(a, w, ws, s, c, cfg=cfg)
        elif epi == "bias":
            c = torch.zeros((m, n), dtype=torch.float16, device="cuda")
            k2.gemm_i8_bias(a, w, ws, s, bias, c, cfg=cfg)
        elif epi == "swiglu":
            c = torch.zeros((m, n // 2), dtype=torch.float16, device="cuda")
            k2.gemm_i8_swiglu(a, w, ws, s, c, cfg=cfg)
        else:
            c = dev(x0, torch.bfloat16).view(m, n)
            k2.gemm_i8_resid(a, w, ws, s, c, gate, cfg=cfg)
        torch.cuda.synchronize()
        outs.append(c.view(torch.int16).clone())
    assert torch.equal(outs[0], outs[1])
