"""The fused prepare -> GEMM entry points (k2w8_linear_norm_i8, k2w8_linear_plain_i8):
bit-identical to the two entry points called in turn (q, q_scale and the output), in
the one-launch form (K2W8_LINEAR_ONE_LAUNCH=1: whole rounds of 256x192 tiles in one
persistent kernel) and in the default two-launch form. The one-launch kernel's grid
barrier count is the launch's own (cleared before each launch, kept in the stream's
workspace), so back-to-back calls, graph replays and calls on two streams at once give
the same results; and a barrier that gives up (forced from the host by a poll bound of
0) still gives exact output, every kernel exiting normally."""

import os

import numpy as np
import pytest
import torch

import oracle
from gpu_common import activations, bf16_bits, channel_scales, dev, f16_bits, host, int8_weights, k2

pytestmark = pytest.mark.gpu


@pytest.fixture(params=["one_launch", "two_launches"])
def mode(request, monkeypatch):
    monkeypatch.setenv("K2W8_LINEAR_ONE_LAUNCH", "1" if request.param == "one_launch" else "0")
    assert os.environ["K2W8_LINEAR_ONE_LAUNCH"] in ("0", "1")
    return request.param


def case(kind, m, k, n, seed):
    rng = np.random.default_rng(seed)
    x = activations(rng, m, k)
    h = bf16_bits(x) if kind == "norm" else f16_bits(x)
    w = int8_weights(rng, n, k)
    ws = channel_scales(rng, n)
    ns = (rng.uniform(0.5, 1.5, k) - 1.0).astype(np.float32)
    zero = np.zeros(k, np.float32)
    dtype = torch.bfloat16 if kind == "norm" else torch.float16
    return dict(kind=kind, m=m, k=k, n=n, h=dev(h, dtype), h_bits=h, w=dev(w), ws=dev(ws),
                ns=dev(ns), zero=dev(zero), ns_np=ns, zero_np=zero)


def run(c, fused, out=None, q=None, s=None):
    m, k, n = c["m"], c["k"], c["n"]
    q = torch.full((m, k), 91, dtype=torch.int8, device="cuda") if q is None else q
    s = torch.zeros(m, dtype=torch.float32, device="cuda") if s is None else s
    out = torch.zeros((m, n), dtype=torch.float16, device="cuda") if out is None else out
    cfg = k2.GemmConfig(k_size=k, n_size=n, k_stride=k)
    if fused and c["kind"] == "norm":
        k2.linear_norm_i8(c["h"], c["ns"], c["zero"], c["zero"], q, s, c["w"], c["ws"], out, cfg=cfg,
                          eps=1e-6)
    elif fused:
        k2.linear_plain_i8(c["h"], q, s, c["w"], c["ws"], out, cfg=cfg)
    elif c["kind"] == "norm":
        k2.prepare_norm_i8(c["h"], c["ns"], c["zero"], c["zero"], q, s, width=k, out_stride=k, eps=1e-6)
        k2.gemm_i8(q, c["w"], c["ws"], s, out, cfg=cfg)
    else:
        k2.prepare_plain_i8(c["h"], q, s, width=k, out_stride=k)
        k2.gemm_i8(q, c["w"], c["ws"], s, out, cfg=cfg)
    return q, s, out


SHAPES = [
    ("plain", 4096, 3072, 12288),  # north star: 1024 tiles of 256x192, one launch
    ("norm", 4096, 3072, 9216),    # configs[1]: 768 tiles of 256x192, one launch
    ("norm", 2048, 2048, 12288),   # 512 tiles of 256x192, width 2048 (two runs per lane)
    ("norm", 2048, 2048, 8192),    # not whole 256x192 columns: the two-launch fallback
    ("norm", 4544, 3072, 9216),    # ragged rounds: the two-launch fallback
    ("plain", 300, 1024, 1024),    # mid-M: the two-launch fallback
]


@pytest.mark.parametrize("kind,m,k,n", SHAPES)
def test_fused_equals_the_two_entry_points(kind, m, k, n, mode):
    c = case(kind, m, k, n, seed=m + k + n)
    q1, s1, o1 = run(c, fused=True)
    q2, s2, o2 = run(c, fused=False)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(s1, s2)
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    # and the prepared rows against the oracle (the GEMM halves are pinned elsewhere)
    rows = np.arange(0, m, max(1, m // 16))
    if kind == "norm":
        q_ref, s_ref = oracle.prepare_norm(c["h_bits"][rows], c["ns_np"], c["zero_np"], c["zero_np"],
                                           k, k, 1e-6)
    else:
        q_ref, s_ref = oracle.prepare_plain(c["h_bits"][rows], k, k)
    assert np.array_equal(host(q1)[rows], q_ref) and np.array_equal(host(s1)[rows], s_ref)


def test_back_to_back_calls_and_graph_replays(mode):
    c = case("norm", 4096, 3072, 9216, seed=5)
    q, s, want = run(c, fused=False)
    torch.cuda.synchronize()
    out = torch.zeros_like(want)
    for _ in range(3):  # eager, back to back: the barrier's counters return to zero
        run(c, fused=True, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    qg = torch.zeros_like(q)
    sg = torch.zeros_like(s)
    og = torch.zeros_like(want)
    run(c, fused=True, out=og, q=qg, s=sg)  # one-time set-up outside the capture
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        run(c, fused=True, out=og, q=qg, s=sg)
    for replay in range(3):
        og.zero_()
        qg.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(og.view(torch.int16), want.view(torch.int16)), replay
        assert torch.equal(qg, q), replay


PAIRS = [
    # (pair, tokens, width, n): the block's projections at a small and a ragged size
    ("gated_resid", 300, 1024, 1024),
    ("gated_resid", 77, 3072, 3072),
    ("norm_swiglu", 300, 1024, 4096),
    ("norm_swiglu", 513, 2048, 8192),
    ("plain_resid", 300, 4096, 1024),
    ("plain_resid", 256, 9728, 2560),  # the down projection that splits K
]


@pytest.mark.parametrize("pair,m,k,n", PAIRS)
def test_block_pairs_equal_their_two_entry_points(pair, m, k, n):
    rng = np.random.default_rng(m * 3 + k + n)
    x = activations(rng, m, k)
    w = dev(int8_weights(rng, n, k))
    ws = dev(channel_scales(rng, n))
    cfg = k2.GemmConfig(k_size=k, n_size=n, k_stride=k)
    if pair == "gated_resid":
        attn = dev(f16_bits(x), torch.float16)
        g_in = dev(f16_bits(rng.standard_normal((m, k)).astype(np.float32)), torch.float16)
        gate = dev(rng.uniform(0.5, 1.5, n).astype(np.float32))
        x0 = dev(bf16_bits(rng.standard_normal(m * n).astype(np.float32)), torch.bfloat16)
        res = []
        for fused in (True, False):
            q = torch.full((m, k), 91, dtype=torch.int8, device="cuda")
            s = torch.zeros(m, dtype=torch.float32, device="cuda")
            xx = x0.clone()
            if fused:
                k2.linear_gated_resid_i8(attn, g_in, q, s, w, ws, xx, gate, cfg=cfg, gate_stride=k)
            else:
                k2.prepare_gated_i8(attn, g_in, q, s, width=k, out_stride=k, gate_stride=k)
                k2.gemm_i8_resid(q, w, ws, s, xx, gate, cfg=cfg)
            res.append((q, s, xx))
    elif pair == "norm_swiglu":
        h = dev(bf16_bits(x), torch.bfloat16)
        ns = dev((rng.uniform(0.5, 1.5, k) - 1.0).astype(np.float32))
        ms = dev((rng.uniform(-0.2, 0.2, k)).astype(np.float32))
        sh = dev((rng.uniform(-0.1, 0.1, k)).astype(np.float32))
        res = []
        for fused in (True, False):
            q = torch.full((m, k), 91, dtype=torch.int8, device="cuda")
            s = torch.zeros(m, dtype=torch.float32, device="cuda")
            c = torch.zeros((m, n // 2), dtype=torch.float16, device="cuda")
            if fused:
                k2.linear_norm_swiglu_i8(h, ns, ms, sh, q, s, w, ws, c, cfg=cfg, eps=1e-6)
            else:
                k2.prepare_norm_i8(h, ns, ms, sh, q, s, width=k, out_stride=k, eps=1e-6)
                k2.gemm_i8_swiglu(q, w, ws, s, c, cfg=cfg)
            res.append((q, s, c))
    else:
        h = dev(f16_bits(x), torch.float16)
        gate = dev(rng.uniform(0.5, 1.5, n).astype(np.float32))
        x0 = dev(bf16_bits(rng.standard_normal(m * n).astype(np.float32)), torch.bfloat16)
        res = []
        for fused in (True, False):
            q = torch.full((m, k), 91, dtype=torch.int8, device="cuda")
            s = torch.zeros(m, dtype=torch.float32, device="cuda")
            xx = x0.clone()
            if fused:
                k2.linear_plain_resid_i8(h, q, s, w, ws, xx, gate, cfg=cfg)
            else:
                k2.prepare_plain_i8(h, q, s, width=k, out_stride=k)
                k2.gemm_i8_resid(q, w, ws, s, xx, gate, cfg=cfg)
            res.append((q, s, xx))
    torch.cuda.synchronize()
    (q1, s1, o1), (q2, s2, o2) = res
    assert torch.equal(q1, q2) and torch.equal(s1, s2)
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))


@pytest.mark.parametrize("kind,m,k,n", [("norm", 4096, 3072, 9216), ("plain", 2048, 2048, 12288)])
def test_a_barrier_that_gives_up_still_gives_exact_output(kind, m, k, n, monkeypatch):
    # A poll bound of 0: every workgroup gives up at the barrier at once and prepares
    # the rows of each of its tiles itself. The output must equal the two launches',
    # and a following call with the default bound must too (its count starts at 0).
    c = case(kind, m, k, n, seed=11 + m)
    q2, s2, o2 = run(c, fused=False)
    monkeypatch.setenv("K2W8_LINEAR_ONE_LAUNCH", "1")
    monkeypatch.setenv("K2W8_FUSED_BARRIER_POLLS", "0")
    q1, s1, o1 = run(c, fused=True)
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(s1, s2)
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    monkeypatch.delenv("K2W8_FUSED_BARRIER_POLLS")
    q3, s3, o3 = run(c, fused=True)
    torch.cuda.synchronize()
    assert torch.equal(q3, q2) and torch.equal(o3.view(torch.int16), o2.view(torch.int16))


def test_one_launch_calls_on_two_streams_at_once(monkeypatch):
    # Two host threads, each calling the one-launch form on its own stream several
    # times: the launches overlap on the device, each counts its own arrivals, and
    # every output equals the two launches' (ctypes releases the GIL during a call).
    import threading

    monkeypatch.setenv("K2W8_LINEAR_ONE_LAUNCH", "1")
    cases = [case("norm", 4096, 3072, 9216, seed=21), case("plain", 4096, 3072, 12288, seed=22)]
    wants = []
    for c in cases:
        _, _, o = run(c, fused=False)
        wants.append(o)
    torch.cuda.synchronize()
    outs = [[torch.zeros_like(w) for _ in range(4)] for w in wants]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()  # the outputs' fills (default stream) before the workers' streams
    errors = []

    def worker(i):
        try:
            with torch.cuda.stream(streams[i]):
                for o in outs[i]:
                    run(cases[i], fused=True, out=o)
        except Exception as e:  # noqa: BLE001 - reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i, w in enumerate(wants):
        for j, o in enumerate(outs[i]):
            assert torch.equal(o.view(torch.int16), w.view(torch.int16)), (i, j)
