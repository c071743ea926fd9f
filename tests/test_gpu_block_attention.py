"""GPU parity of the whole block sequence with its attention step (src/session/mod.rs:
671-840): prepare, gemm qkvg, q/k norm + rope, V transpose, f16 attention, then the
post-attention W8A8 stages, for head ratios 4 (the reference's layout) and 2.

  wiring     the session's recorded/eager block equals the same kernels called one by
             one through their own entry points (bit for bit: the kernels are
             deterministic), so buffers, strides and head counts are the intended ones
  rope       bit-exact against the oracle from the GPU's fused qkvg output
  attention  against the oracle from the GPU's q, k, V^T (2e-3 abs + 4e-3 rel, as in the
             kernel test) and against an f64 softmax at the reference's 2e-2
  graph      replays equal eager runs
"""

import numpy as np
import pytest
import torch

import oracle
from ckpt_fixture import block_tensors, write_safetensors
from gpu_common import bf16_bits, dev, host, k2
from krea2_w8a8.block import BlockSession
from krea2_w8a8.checkpoint import Checkpoint, Plan
from test_oracle_attention import attention_f64, close

pytestmark = pytest.mark.gpu

TOKENS, INTER, LAYERS, EPS = 40, 512, 2, 1e-5
LAYOUTS = {4: (512, 128), 2: (256, 128)}  # group -> (hidden, kv width)


@pytest.fixture(scope="module", params=[4, 2])
def model(request, tmp_path_factory):
    group = request.param
    hidden, kv = LAYOUTS[group]
    rng = np.random.default_rng(30 + group)
    t = block_tensors(rng, layers=LAYERS, hidden=hidden, kv=kv, inter=INTER)
    path = tmp_path_factory.mktemp(f"blockattn{group}") / "model.safetensors"
    write_safetensors(path, t)
    uploaded = Plan(Checkpoint(path)).upload()
    x0 = bf16_bits(rng.standard_normal((TOKENS, hidden)))
    mods = np.zeros((LAYERS, 6, hidden), np.float32)
    mods[:, (0, 3)] = rng.uniform(-0.2, 0.2, (LAYERS, 2, hidden))
    mods[:, (1, 4)] = rng.uniform(-0.1, 0.1, (LAYERS, 2, hidden))
    mods[:, (2, 5)] = rng.uniform(0.5, 1.5, (LAYERS, 2, hidden))
    ang = rng.uniform(0, 6.3, (TOKENS, 64)).astype(np.float32)
    cos = np.repeat(np.cos(ang), 2, axis=1).astype(np.float32)
    sin = np.repeat(np.sin(ang), 2, axis=1).astype(np.float32)
    return dict(group=group, hidden=hidden, kv=kv, uploaded=uploaded, x0=x0, mods=mods,
                cos=cos, sin=sin)


def session(m):
    h = m["hidden"]
    s = BlockSession.from_checkpoint(m["uploaded"], tokens=TOKENS, hidden=h, inter=INTER,
                                     qkvg=2 * h + 2 * m["kv"], gate_offset=h + 2 * m["kv"],
                                     eps=EPS, attention=True)
    reset(s, m)
    return s


def reset(s, m):
    with torch.cuda.stream(s.stream):
        s.x.copy_(dev(m["x0"], torch.bfloat16))
        s.mods.copy_(dev(m["mods"]))
        s.cos.copy_(dev(m["cos"]))
        s.sin.copy_(dev(m["sin"]))


def by_hand(s, m, index):
    """Block `index` with the attention step launched through the single-kernel calls."""
    h, kv = m["hidden"], m["kv"]
    cap = k2.shape.capacity(TOKENS)
    w = s._weights[index]
    with torch.cuda.stream(s.stream):
        s.pre_attention(index)
        k2.rope_qknorm_f16(s.fused, w["qnorm"], w["knorm"], s.cos, s.sin, s.q, s.k, s.v,
                           row_stride=2 * h + 2 * kv, q_heads=h // 128, kv_heads=kv // 128,
                           k_offset=h, eps=EPS, tokens=TOKENS)
        k2.v_transpose(s.v, s.vt, width=kv, row_capacity=cap, rows=TOKENS)
        k2.attention_f16(s.q, s.k, s.vt, s.attn_gu, q_stride=h, kv_stride=kv, out_stride=h,
                         tokens=TOKENS, token_capacity=cap, scale=0.08838834764831845,
                         kv_heads=kv // 128, group=m["group"])
        s.post_attention(index)


def test_block_with_attention_is_its_kernels_in_order_and_matches_the_oracle(model):
    m = model
    h, kv, group = m["hidden"], m["kv"], m["group"]
    eager = session(m)
    eager.run()
    eager.stream.synchronize()

    manual = session(m)
    for i in range(LAYERS):
        by_hand(manual, m, i)
        manual.stream.synchronize()
        # the attention step of block i, from the GPU's own inputs, against the oracle
        fused = host(manual.fused)
        w = manual._weights[i]
        q, k, v = oracle.rope_qknorm(fused, host(w["qnorm"]), host(w["knorm"]), m["cos"], m["sin"],
                                     row_stride=2 * h + 2 * kv, q_heads=h // 128,
                                     kv_heads=kv // 128, k_offset=h, eps=EPS)
        assert np.array_equal(host(manual.q)[:TOKENS], q)
        assert np.array_equal(host(manual.k)[:TOKENS], k)
        assert np.array_equal(host(manual.v)[:TOKENS], v)
        cap = k2.shape.capacity(TOKENS)
        vt = host(manual.vt)
        assert np.array_equal(vt[:, :TOKENS], v.T) and not vt[:, TOKENS:].any()
        qd, kd = host(manual.q), host(manual.k)
        ora = oracle.attention(qd, kd, vt, tokens=TOKENS, capacity=cap, q_stride=h,
                               kv_stride=kv, out_stride=h, kv_heads=kv // 128,
                               scale=0.08838834764831845, group=group, key_tile=64)
        # attn_gu now holds the SwiGLU output; recompute the attention output alone
        out = torch.empty((TOKENS, h), dtype=torch.float16, device="cuda")
        k2.attention_f16(manual.q, manual.k, manual.vt, out, q_stride=h, kv_stride=kv,
                         out_stride=h, tokens=TOKENS, token_capacity=cap,
                         scale=0.08838834764831845, kv_heads=kv // 128, group=group)
        torch.cuda.synchronize()
        got = host(out).view(np.float16)
        close(got, ora.view(np.float16), 2e-3, 4e-3)
        want = attention_f64(qd.view(np.float16).ravel(), kd.view(np.float16).ravel(),
                             vt.T.copy().view(np.float16).ravel(), TOKENS, h // 128, kv // 128)
        close(got, want, 2e-2, 2e-2)
    assert np.array_equal(host(eager.x), host(manual.x))
    assert np.array_equal(host(eager.q), host(manual.q))


def test_graph_replays_of_the_whole_block_match_eager_runs(model):
    m = model
    eager = session(m)
    eager.run()
    eager.stream.synchronize()
    want = host(eager.x)
    s = session(m)
    s.record()
    for replay in range(3):
        reset(s, m)  # eager work between replays
        s.replay()
        s.stream.synchronize()
        assert np.array_equal(host(s.x), want), replay
        assert np.array_equal(host(s.attn_gu), host(eager.attn_gu)), replay


def test_stage_profile_includes_the_attention_step(model):
    s = session(model)
    stages = s.profile()
    assert {"qk norm + rope", "V transpose", "f16 attention"} <= set(stages)
    assert len(stages) == 10 and all(v > 0 for v in stages.values())
