"""GPU parity at the reference's production specialisation (src/kernels/blocks.rs:38-107):
hidden 6144 (eps 1e-5), intermediate 16384 at pitch 16448 (src/kernels/shape.rs:105-107),
and the fused QKVG output of 15360 columns whose gate half starts at column 9216
(src/session/mod.rs:35-45, 140-144) and feeds the gated prepare with gate_stride 15360.

300 tokens: the last 256-row tile has ghost rows, and the count is not a multiple of 64.
Prepares are bit-exact on every row; GEMM accumulators are checked on every row through
row and column checksums (integer identities) and exactly on sampled rows, whose
epilogues are compared bit for bit with the oracle."""

import numpy as np
import pytest
import torch

import oracle
from gpu_common import (PAD, activations, bf16_bits, channel_scales, dev, f16_bits, host,
                        int8_weights, k2, sync)

pytestmark = pytest.mark.gpu

TOKENS = 300
HIDDEN, INTER, QKVG, GATE_OFFSET = 6144, 16384, 15360, 9216


def test_production_widths_and_pitches():
    assert k2.shape.gemm_pitch(HIDDEN) == HIDDEN
    assert k2.shape.gemm_pitch(INTER) == 16448


def test_norm_prepare_at_hidden_6144():
    rng = np.random.default_rng(61)
    h = bf16_bits(activations(rng, TOKENS, HIDDEN))
    ns = rng.uniform(-0.5, 0.5, HIDDEN).astype(np.float32)
    ms = rng.uniform(-0.2, 0.2, HIDDEN).astype(np.float32)
    sh = rng.uniform(-0.1, 0.1, HIDDEN).astype(np.float32)
    stride = k2.shape.gemm_pitch(HIDDEN)
    q = torch.full((TOKENS, stride), PAD, dtype=torch.int8, device="cuda")
    s = torch.zeros(TOKENS, dtype=torch.float32, device="cuda")
    k2.prepare_norm_i8(dev(h.reshape(TOKENS, HIDDEN), torch.bfloat16), dev(ns), dev(ms), dev(sh),
                       q, s, width=HIDDEN, out_stride=stride, eps=1e-5)
    sync()
    q_ref, s_ref = oracle.prepare_norm(h, ns, ms, sh, HIDDEN, stride, 1e-5)
    assert np.array_equal(host(s).view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(host(q)[:, :HIDDEN], q_ref[:, :HIDDEN])


def test_gated_prepare_reads_the_gate_half_of_the_fused_qkvg_buffer():
    rng = np.random.default_rng(62)
    attn = f16_bits(activations(rng, TOKENS, HIDDEN))
    fused = f16_bits(activations(rng, TOKENS, QKVG, outliers=0, scale=2.0))
    stride = k2.shape.gemm_pitch(HIDDEN)
    fused_dev = dev(fused.reshape(TOKENS, QKVG), torch.float16)
    gate_half = fused_dev.view(-1)[GATE_OFFSET:]  # from the gate offset to the end
    q = torch.full((TOKENS, stride), PAD, dtype=torch.int8, device="cuda")
    s = torch.zeros(TOKENS, dtype=torch.float32, device="cuda")
    k2.prepare_gated_i8(dev(attn.reshape(TOKENS, HIDDEN), torch.float16), gate_half, q, s,
                        width=HIDDEN, out_stride=stride, gate_stride=QKVG)
    sync()
    gate_rows = fused.reshape(TOKENS, QKVG).reshape(-1)[GATE_OFFSET:]
    gate_rows = np.concatenate([gate_rows, np.zeros(GATE_OFFSET, np.uint16)])
    q_ref, s_ref = oracle.prepare_gated(attn, gate_rows, HIDDEN, stride, QKVG)
    assert np.array_equal(host(s).view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(host(q)[:, :HIDDEN], q_ref[:, :HIDDEN])


def test_plain_prepare_at_intermediate_16384_leaves_the_pitch_padding():
    rng = np.random.default_rng(63)
    h = f16_bits(activations(rng, TOKENS, INTER))
    stride = k2.shape.gemm_pitch(INTER)
    q = torch.full((TOKENS, stride), PAD, dtype=torch.int8, device="cuda")
    s = torch.zeros(TOKENS, dtype=torch.float32, device="cuda")
    k2.prepare_plain_i8(dev(h.reshape(TOKENS, INTER), torch.float16), q, s, width=INTER,
                        out_stride=stride)
    sync()
    q_ref, s_ref = oracle.prepare_plain(h, INTER, stride)
    got = host(q)
    assert np.array_equal(host(s).view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(got[:, :INTER], q_ref[:, :INTER])
    assert np.all(got[:, INTER:] == PAD)


def checked_accumulators(a, w, m, n, k, stride, rows):
    """Accumulators of every row through checksums; the sampled rows exactly."""
    A, W = dev(a), dev(w)
    acc = torch.empty((m, n), dtype=torch.int32, device="cuda")
    cfg = k2.GemmConfig(k_size=k, n_size=n, k_stride=stride)
    k2.gemm_i8_acc(A, W, acc, cfg=cfg, m=m)
    A64, W64 = A[:, :k].to(torch.int64), W[:, :k].to(torch.int64)
    assert torch.equal(acc.to(torch.int64).sum(1), (A64 * W64.sum(0)).sum(1))
    assert torch.equal(acc.to(torch.int64).sum(0), (W64 * A64.sum(0)).sum(1))
    ref = oracle.gemm_i32(a[rows], w, len(rows), n, k, stride)
    assert np.array_equal(host(acc)[rows], ref)
    return ref, cfg


# (name, epilogue, K, N) of the four production GEMMs.
GEMMS = [
    ("gemm_qkvg", "plain", HIDDEN, QKVG),
    ("gemm_gu", "swiglu", HIDDEN, 2 * INTER),
    ("gemm_wo", "resid", HIDDEN, HIDDEN),
    ("gemm_down", "resid_wide", INTER, HIDDEN),
]


@pytest.mark.parametrize("name,epilogue,k,n", GEMMS)
def test_production_gemm(name, epilogue, k, n):
    rng = np.random.default_rng(sum(name.encode()))
    stride = k2.shape.gemm_pitch(k)
    a = int8_weights(rng, TOKENS, k, stride)
    w = int8_weights(rng, n, k, stride)
    ws = channel_scales(rng, n)
    a_scale = rng.uniform(1e-3, 3e-2, TOKENS).astype(np.float32)
    rows = np.array([0, 1, 77, 255, 256, 299])
    ref_acc, cfg = checked_accumulators(a, w, TOKENS, n, k, stride, rows)
    A, W, WS, AS = dev(a), dev(w), dev(ws), dev(a_scale)
    if epilogue == "plain":
        out = torch.empty((TOKENS, n), dtype=torch.float16, device="cuda")
        k2.gemm_i8(A, W, WS, AS, out, cfg=cfg)
        want = oracle.epilogue_plain(ref_acc, ws, a_scale[rows])
    elif epilogue == "swiglu":
        out = torch.empty((TOKENS, n // 2), dtype=torch.float16, device="cuda")
        k2.gemm_i8_swiglu(A, W, WS, AS, out, cfg=cfg)
        want = oracle.epilogue_swiglu(ref_acc, ws, a_scale[rows])
    else:
        gate = rng.uniform(0.5, 1.5, n).astype(np.float32)
        prior = bf16_bits(rng.standard_normal((TOKENS, n)))
        out = dev(prior, torch.bfloat16)
        schedule = k2.GemmConfig(k_size=k, n_size=n, k_stride=stride,
                                 schedule_rows=int(k2.shape.gemm_schedule_rows(TOKENS)))
        fn = k2.gemm_i8_resid_256x256 if epilogue == "resid_wide" else k2.gemm_i8_resid
        fn(A, W, WS, AS, out, dev(gate), cfg=schedule)
        want = oracle.epilogue_resid(ref_acc, ws, a_scale[rows], gate, prior[rows])
    sync()
    assert np.array_equal(host(out)[rows], want)
