"""GPU parity of the block sequence (src/session/mod.rs:671-840, W8A8 stages): two
blocks of a synthetic checkpoint, uploaded through the plan, against the CPU oracle
chained stage by stage; the recorded graph's replays against eager runs."""

import numpy as np
import pytest
import torch

import oracle
from ckpt_fixture import block_tensors, expected_layout, write_safetensors
from gpu_common import bf16_bits, dev, f16_bits, host, k2, sync
from krea2_w8a8.block import BlockSession
from krea2_w8a8.checkpoint import Checkpoint, Plan

pytestmark = pytest.mark.gpu

HIDDEN, KV, INTER, TOKENS, LAYERS = 256, 64, 512, 40, 2
QKVG = HIDDEN + 2 * KV + HIDDEN
GATE_OFFSET = HIDDEN + 2 * KV
EPS = 1e-5


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    rng = np.random.default_rng(21)
    t = block_tensors(rng, layers=LAYERS, hidden=HIDDEN, kv=KV, inter=INTER)
    path = tmp_path_factory.mktemp("block") / "model.safetensors"
    write_safetensors(path, t)
    ckpt = Checkpoint(path)
    uploaded = Plan(ckpt).upload()
    x0 = bf16_bits(rng.standard_normal((TOKENS, HIDDEN)))
    mods = np.zeros((LAYERS, 6, HIDDEN), np.float32)
    mods[:, (0, 3)] = rng.uniform(-0.2, 0.2, (LAYERS, 2, HIDDEN))
    mods[:, (1, 4)] = rng.uniform(-0.1, 0.1, (LAYERS, 2, HIDDEN))
    mods[:, (2, 5)] = rng.uniform(0.5, 1.5, (LAYERS, 2, HIDDEN))
    attn0 = f16_bits(rng.standard_normal(TOKENS * INTER) * 0.5)
    return ckpt, uploaded, expected_layout(t, LAYERS), x0, mods, attn0


def session(uploaded, x0, mods, attn0):
    s = BlockSession.from_checkpoint(uploaded, tokens=TOKENS, hidden=HIDDEN, inter=INTER,
                                     qkvg=QKVG, gate_offset=GATE_OFFSET, eps=EPS)
    reset(s, x0, mods, attn0)
    return s


def reset(s, x0, mods, attn0):
    with torch.cuda.stream(s.stream):
        s.x.copy_(dev(x0, torch.bfloat16))
        s.mods.copy_(dev(mods))
        s.attn_gu.copy_(dev(attn0, torch.float16))


def oracle_blocks(layout, x, mods, attn):
    ph, pi = k2.shape.gemm_pitch(HIDDEN), k2.shape.gemm_pitch(INTER)
    x = x.copy()
    attn = attn.copy()
    for i in range(LAYERS):
        w = {k[len(f"blocks.{i}."):]: v for k, v in layout.items() if k.startswith(f"blocks.{i}.")}
        q, s = oracle.prepare_norm(x, w["prenorm"], mods[i, 0], mods[i, 1], HIDDEN, ph, EPS)
        fused = oracle.epilogue_plain(oracle.gemm_i32(q, w["qkvg.q"], TOKENS, QKVG, HIDDEN, ph),
                                      w["qkvg.s"], s)
        gate = np.concatenate([fused.reshape(-1)[GATE_OFFSET:], np.zeros(GATE_OFFSET, np.uint16)])
        q, s = oracle.prepare_gated(attn[: TOKENS * HIDDEN], gate, HIDDEN, ph, QKVG)
        acc = oracle.gemm_i32(q, w["wo.q"], TOKENS, HIDDEN, HIDDEN, ph)
        x = oracle.epilogue_resid(acc, w["wo.s"], s, mods[i, 2], x.reshape(-1)).reshape(TOKENS, HIDDEN)
        q, s = oracle.prepare_norm(x, w["postnorm"], mods[i, 3], mods[i, 4], HIDDEN, ph, EPS)
        acc = oracle.gemm_i32(q, w["gu.q"], TOKENS, 2 * INTER, HIDDEN, ph)
        attn[: TOKENS * INTER] = oracle.epilogue_swiglu(acc, w["gu.s"], s).reshape(-1)
        q, s = oracle.prepare_plain(attn[: TOKENS * INTER], INTER, pi)
        acc = oracle.gemm_i32(q, w["down.q"], TOKENS, HIDDEN, INTER, pi)
        x = oracle.epilogue_resid(acc, w["down.s"], s, mods[i, 5], x.reshape(-1)).reshape(TOKENS, HIDDEN)
    return x, fused, attn


def test_two_blocks_match_the_oracle_stage_chain(model):
    _, uploaded, layout, x0, mods, attn0 = model
    s = session(uploaded, x0, mods, attn0)
    s.run()
    s.stream.synchronize()
    x, fused, attn = oracle_blocks(layout, x0, mods, attn0)
    assert np.array_equal(host(s.fused), fused)
    assert np.array_equal(host(s.attn_gu)[: TOKENS * INTER], attn[: TOKENS * INTER])
    assert np.array_equal(host(s.x), x)


def test_graph_replays_match_eager_runs(model):
    _, uploaded, _, x0, mods, attn0 = model
    eager = session(uploaded, x0, mods, attn0)
    eager.run()
    eager.stream.synchronize()
    want = host(eager.x)
    s = session(uploaded, x0, mods, attn0)
    s.record()
    for replay in range(3):
        reset(s, x0, mods, attn0)  # eager work between replays
        s.replay()
        s.stream.synchronize()
        assert np.array_equal(host(s.x), want), replay
        assert np.array_equal(host(s.fused), host(eager.fused)), replay


def test_stage_profile_names_every_stage(model):
    _, uploaded, _, x0, mods, attn0 = model
    s = session(uploaded, x0, mods, attn0)
    stages = s.profile()
    assert set(stages) == {"prepare", "gemm qkvg", "prepare gated", "gemm wo + residual",
                           "gemm gate|up + swiglu", "prepare swiglu", "gemm down + residual"}
    assert all(v > 0 for v in stages.values())
