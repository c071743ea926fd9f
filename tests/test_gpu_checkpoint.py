"""GPU side of the checkpoint upload (src/session/weights.rs:48-100): every span's device
bytes equal the layout built independently in tests/ckpt_fixture.py (rows at the GEMM
pitch with zero padding, concatenated and 16-row interleaved operands, scales following
their rows, bf16 norm vectors upcast), and the uploaded gate|up operand drives the SwiGLU
GEMM to the oracle's result for the checkpoint's separate gate and up tensors."""

import numpy as np
import pytest
import torch

import oracle
from ckpt_fixture import block_tensors, expected_layout, write_safetensors
from gpu_common import dev, host, k2, sync
from krea2_w8a8.checkpoint import Checkpoint, Plan

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bf16_norms", [False, True])
def test_upload_places_every_span(tmp_path, bf16_norms):
    rng = np.random.default_rng(7 + bf16_norms)
    t = block_tensors(rng, layers=2, bf16_norms=bf16_norms)
    path = tmp_path / "ckpt.safetensors"
    write_safetensors(path, t)
    with Checkpoint(path) as f:
        plan = Plan(f)
        weights = plan.upload()
        sync()
        storage = host(weights.storage)
        expected = expected_layout(t, 2)
        covered = np.zeros(storage.size, bool)
        for name in plan.names():
            span = plan.span(name)
            want = np.ascontiguousarray(expected[name]).view(np.uint8).reshape(-1)
            got = storage[span.device_offset:span.device_offset + span.device_bytes]
            assert got.size == want.size, name
            assert np.array_equal(got, want), name
            covered[span.device_offset:span.device_offset + span.device_bytes] = True
        assert np.all(storage[~covered] == 0)  # alignment gaps stay zero


def test_the_uploaded_gate_up_operand_feeds_the_swiglu_gemm(tmp_path):
    rng = np.random.default_rng(9)
    t = block_tensors(rng, layers=1, inter=512)
    path = tmp_path / "ckpt.safetensors"
    write_safetensors(path, t)
    with Checkpoint(path) as f:
        weights = Plan(f).upload()
        w, ws = weights.operand("blocks.0.gu"), weights.scales("blocks.0.gu")
        m, k, n = 96, 256, 1024
        a = rng.integers(-127, 128, (m, k), dtype=np.int8)
        a_scale = rng.uniform(1e-3, 3e-2, m).astype(np.float32)
        out = torch.empty((m, n // 2), dtype=torch.float16, device="cuda")
        cfg = k2.GemmConfig(k_size=k, n_size=n, k_stride=w.shape[1])
        k2.gemm_i8_swiglu(dev(a), w, ws, dev(a_scale), out, cfg=cfg)
        sync()
        layout = expected_layout(t, 1)
        w_ref, ws_ref = layout["blocks.0.gu.q"], layout["blocks.0.gu.s"]
        acc = oracle.gemm_i32(a, w_ref, m, n, k, w_ref.shape[1])
        assert np.array_equal(host(out), oracle.epilogue_swiglu(acc, ws_ref, a_scale))
        # the same product from the separate tensors: output o pairs gate row o with up row o
        g, u = t["blocks.0.mlp.gate.weight"], t["blocks.0.mlp.up.weight"]
        dots_g = a.astype(np.int64) @ g.astype(np.int64).T
        assert np.array_equal(acc[:, 0:16], dots_g[:, 0:16])
        assert np.array_equal(acc[:, 16:32], (a.astype(np.int64) @ u.astype(np.int64).T)[:, 0:16])
