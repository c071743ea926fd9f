"""The split-K workspace contract: a caller-owned workspace per stream (used also under
stream capture, with no priming call), and a recorded block graph that owns its
workspace, so replaying it on any stream never shares partial sums with eager calls on
the recording stream (the reference's session owns every workspace,
src/session/mod.rs:321-340)."""

import ctypes

import numpy as np
import pytest
import torch

import oracle
from gpu_common import channel_scales, dev, host, int8_weights, k2, sync
from krea2_w8a8._lib import lib
from krea2_w8a8.block import BlockSession

pytestmark = pytest.mark.gpu

SENTINEL = 0x5A5A5A5A


def cfg(k, n, stride):
    return k2.GemmConfig(k_size=k, n_size=n, k_stride=stride)


def split_case(rng, m=256, k=9728, n=2560):
    # 128x128 tiles of (256, 2560) cover 40 CUs: K splits (the config-4 down projection)
    a = int8_weights(rng, m, k)
    w = int8_weights(rng, n, k)
    ws = channel_scales(rng, n)
    s = rng.uniform(1e-3, 3e-2, m).astype(np.float32)
    want = oracle.epilogue_plain(oracle.gemm_i32(a, w, m, n, k, k), ws, s)
    return dict(a=dev(a), w=dev(w), ws=dev(ws), s=dev(s), m=m, k=k, n=n, want=want)


def test_a_registered_workspace_lets_a_captured_gemm_split_without_priming():
    rng = np.random.default_rng(31)
    c = split_case(rng)
    # one-time device set-up (kernel attributes) happens on a first call, outside capture
    warm = torch.zeros((c["m"], c["n"]), dtype=torch.float16, device="cuda")
    k2.gemm_i8(c["a"], c["w"], c["ws"], c["s"], warm, cfg=cfg(c["k"], c["n"], c["k"]))
    stream = torch.cuda.Stream()  # a fresh stream: the library has no workspace for it
    ws = torch.full((k2.gemm_workspace_bytes() // 4,), SENTINEL, dtype=torch.int32, device="cuda")
    out = torch.zeros((c["m"], c["n"]), dtype=torch.float16, device="cuda")
    k2.gemm_set_workspace(ws, stream=stream)
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            k2.gemm_i8(c["a"], c["w"], c["ws"], c["s"], out, cfg=cfg(c["k"], c["n"], c["k"]))
        sync()
        assert torch.all(ws == SENTINEL)  # capture recorded, ran nothing
        for replay in range(3):
            out.zero_()  # eager work between the replays
            graph.replay()
            sync()
            assert np.array_equal(host(out), c["want"]), replay
        # the replays split K: their int32 partial sums overwrote the sentinel
        assert int((ws != SENTINEL).sum()) >= 2 * c["m"] * c["n"] * 9 // 10
    finally:
        k2.gemm_set_workspace(None, stream=stream)
    sync()
    # registration removed: an eager call on the stream still gets the right answer
    out2 = torch.zeros_like(out)
    with torch.cuda.stream(stream):
        k2.gemm_i8(c["a"], c["w"], c["ws"], c["s"], out2, cfg=cfg(c["k"], c["n"], c["k"]))
    sync()
    assert np.array_equal(host(out2), c["want"])


def test_a_small_registered_workspace_splits_less_and_stays_exact():
    rng = np.random.default_rng(32)
    c = split_case(rng, m=77)
    stream = torch.cuda.Stream()
    ws = torch.empty(2 * c["m"] * c["n"], dtype=torch.int32, device="cuda")  # two slices
    out = torch.zeros((c["m"], c["n"]), dtype=torch.float16, device="cuda")
    k2.gemm_set_workspace(ws, stream=stream)
    try:
        with torch.cuda.stream(stream):
            k2.gemm_i8(c["a"], c["w"], c["ws"], c["s"], out, cfg=cfg(c["k"], c["n"], c["k"]))
        sync()
    finally:
        k2.gemm_set_workspace(None, stream=stream)
    assert np.array_equal(host(out), c["want"])


def test_set_workspace_rejects_a_misaligned_or_tiny_buffer():
    buf = torch.empty(4096, dtype=torch.uint8, device="cuda")
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib().k2w8_gemm_set_workspace(s, ctypes.c_void_p(buf.data_ptr() + 16), 1024) == -1
    assert lib().k2w8_gemm_set_workspace(s, ctypes.c_void_p(buf.data_ptr()), 128) == -1


def test_a_graph_replayed_on_another_stream_keeps_its_own_workspace():
    # A block whose down projection splits K (tokens 64, K = inter = 2048, N = 256).
    rng = np.random.default_rng(33)
    tokens, hidden, inter, kv = 64, 256, 2048, 64
    qkvg, gate_off = hidden + 2 * kv + hidden, hidden + 2 * kv
    ph, pi = int(k2.shape.gemm_pitch(hidden)), int(k2.shape.gemm_pitch(inter))
    w = {"qkvg_q": dev(int8_weights(rng, qkvg, hidden, ph)), "qkvg_s": dev(channel_scales(rng, qkvg)),
         "wo_q": dev(int8_weights(rng, hidden, hidden, ph)), "wo_s": dev(channel_scales(rng, hidden)),
         "gu_q": dev(int8_weights(rng, 2 * inter, hidden, ph)),
         "gu_s": dev(channel_scales(rng, 2 * inter)),
         "down_q": dev(int8_weights(rng, hidden, inter, pi)), "down_s": dev(channel_scales(rng, hidden)),
         "prenorm": dev(np.zeros(hidden, np.float32)), "postnorm": dev(np.zeros(hidden, np.float32))}
    x0 = torch.from_numpy(rng.standard_normal((tokens, hidden)).astype(np.float32)).to(torch.bfloat16)
    attn0 = torch.from_numpy(rng.standard_normal(tokens * inter).astype(np.float32) * 0.5).half()

    def reset(s):
        with torch.cuda.stream(s.stream):
            s.x.copy_(x0.cuda())
            s.mods.zero_()
            s.mods[:, (2, 5)] = 1.0
            s.attn_gu.copy_(attn0.cuda())
        s.stream.synchronize()

    eager = BlockSession([w, w], tokens=tokens, hidden=hidden, inter=inter, qkvg=qkvg,
                         gate_offset=gate_off, eps=1e-6)
    reset(eager)
    eager.run()
    eager.stream.synchronize()
    want = host(eager.x)

    s = BlockSession([w, w], tokens=tokens, hidden=hidden, inter=inter, qkvg=qkvg,
                     gate_offset=gate_off, eps=1e-6)
    s.record()
    c = split_case(rng)
    outs = [torch.zeros((c["m"], c["n"]), dtype=torch.float16, device="cuda") for _ in range(4)]
    other = torch.cuda.Stream()
    for rep in range(3):
        reset(s)
        for o in outs:
            o.zero_()
        sync()
        # the replay on `other` overlaps eager split-K GEMMs on the recording stream
        assert lib().k2w8_graph_launch(ctypes.c_void_p(other.cuda_stream), s._graph) == 0
        with torch.cuda.stream(s.stream):
            for o in outs:
                k2.gemm_i8(c["a"], c["w"], c["ws"], c["s"], o, cfg=cfg(c["k"], c["n"], c["k"]))
        sync()
        assert np.array_equal(host(s.x), want), rep
        for o in outs:
            assert np.array_equal(host(o), c["want"]), rep
