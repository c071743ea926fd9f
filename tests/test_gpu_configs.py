"""GPU parity at the exact shapes of every benchmark configuration (BASELINE configs 0-4
and the north-star GEMM), each against the CPU oracle on every output element.

The inputs follow the configurations' distributions: f16/bf16 hidden states N(0,1) with
eight seeded outlier channels x20, int8 weights uniform in [-127, 127], per-channel
scales U(1e-3, 1e-2), an f16 bias N(0, 0.02). Each chain runs stage by stage on the GPU
(the same entry points the benchmark times) and in the oracle, and every intermediate
(int8 codes, token scales, f16 / bf16 outputs) is compared bit for bit. The oracle's
integer GEMM is multithreaded C, so full-size checks take seconds.
"""

import numpy as np
import pytest
import torch

import oracle
from gpu_common import (activations, bf16_bits, channel_scales, dev, f16_bits, host, int8_weights,
                        k2, sync)
from krea2_w8a8.block import BlockSession

pytestmark = pytest.mark.gpu


def cfg(k, n, stride, schedule_rows=0):
    return k2.GemmConfig(k_size=k, n_size=n, k_stride=stride, schedule_rows=schedule_rows)


def prepare_plain_gpu(h_bits, width, pitch):
    tokens = h_bits.shape[0]
    q = torch.empty((tokens, pitch), dtype=torch.int8, device="cuda")
    s = torch.empty(tokens, dtype=torch.float32, device="cuda")
    k2.prepare_plain_i8(dev(h_bits, torch.float16), q, s, width=width, out_stride=pitch)
    return q, s


def test_config0_prepare_plain_then_bias_gemm_4096x3072x3072():
    # f16 A [4096, 3072] -> prepare_plain_i8 -> gemm_i8_bias (W [3072, 3072]).
    rng = np.random.default_rng(1000)
    m, k, n = 4096, 3072, 3072
    h = f16_bits(activations(rng, m, k))
    w = int8_weights(rng, n, k)
    ws = channel_scales(rng, n)
    bias = f16_bits(rng.standard_normal(n) * 0.02)
    q, s = prepare_plain_gpu(h, k, k)
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    k2.gemm_i8_bias(q, dev(w), dev(ws), s, dev(bias, torch.float16), out, cfg=cfg(k, n, k))
    sync()
    q_ref, s_ref = oracle.prepare_plain(h, k, k)
    assert np.array_equal(host(q), q_ref)
    assert np.array_equal(host(s), s_ref)
    acc = oracle.gemm_i32(q_ref, w, m, n, k, k)
    assert np.array_equal(host(out), oracle.epilogue_bias(acc, ws, s_ref, bias))


def test_config1_prepare_norm_then_qkv_gemm_4096x3072x9216():
    # configs[1] (the headline step): bf16 h [4096, 3072] -> RMSNorm (w ~ U(0.5, 1.5),
    # eps 1e-6) + rotation + quantisation -> QKV gemm_i8 (W [9216, 3072]).
    rng = np.random.default_rng(2000)
    m, k, n = 4096, 3072, 9216
    h = bf16_bits(activations(rng, m, k).astype(np.float16).astype(np.float32))
    ns = (rng.uniform(0.5, 1.5, k) - 1.0).astype(np.float32)
    zero = np.zeros(k, np.float32)
    w = int8_weights(rng, n, k)
    ws = channel_scales(rng, n)
    q = torch.empty((m, k), dtype=torch.int8, device="cuda")
    s = torch.empty(m, dtype=torch.float32, device="cuda")
    k2.prepare_norm_i8(dev(h, torch.bfloat16), dev(ns), dev(zero), dev(zero), q, s, width=k,
                       out_stride=k, eps=1e-6)
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    k2.gemm_i8(q, dev(w), dev(ws), s, out, cfg=cfg(k, n, k))
    sync()
    q_ref, s_ref = oracle.prepare_norm(h, ns, zero, zero, k, k, 1e-6)
    assert np.array_equal(host(q), q_ref)
    assert np.array_equal(host(s), s_ref)
    acc = oracle.gemm_i32(q_ref, w, m, n, k, k)
    assert np.array_equal(host(out), oracle.epilogue_plain(acc, ws, s_ref))


def test_north_star_gemm_4096x3072x12288_every_element():
    # The target shape through prepared activations: prepare_plain_i8 -> gemm_i8 (256x256
    # tiles, three whole rounds), every int32 accumulator and every f16 output.
    rng = np.random.default_rng(3000)
    m, k, n = 4096, 3072, 12288
    h = f16_bits(activations(rng, m, k))
    w = int8_weights(rng, n, k)
    ws = channel_scales(rng, n)
    q, s = prepare_plain_gpu(h, k, k)
    W = dev(w)
    out = torch.empty((m, n), dtype=torch.float16, device="cuda")
    k2.gemm_i8(q, W, dev(ws), s, out, cfg=cfg(k, n, k))
    acc = torch.empty((m, n), dtype=torch.int32, device="cuda")
    k2.gemm_i8_acc(q, W, acc, cfg=cfg(k, n, k))
    sync()
    q_ref, s_ref = oracle.prepare_plain(h, k, k)
    assert np.array_equal(host(q), q_ref)
    ref_acc = oracle.gemm_i32(q_ref, w, m, n, k, k)
    assert np.array_equal(host(acc), ref_acc)
    assert np.array_equal(host(out), oracle.epilogue_plain(ref_acc, ws, s_ref))


def test_config2_mlp_pair_at_4608_tokens():
    # prepared activations [4608, 3072] -> gemm_i8_swiglu (W [2 x 12288, 3072],
    # 16-row gate|up interleave) -> f16 [4608, 12288] -> prepare_plain_i8 (width 12288)
    # -> gemm_i8_resid_256x256 (W [3072, 12288]) in place on a bf16 N(0,1) residual, gate 1.
    rng = np.random.default_rng(4000)
    m, hdim, inter = 4608, 3072, 12288
    pitch_i = int(k2.shape.gemm_pitch(inter))
    h = f16_bits(activations(rng, m, hdim))
    wgu = int8_weights(rng, 2 * inter, hdim)
    sgu = channel_scales(rng, 2 * inter)
    wd = int8_weights(rng, hdim, inter, pitch_i)
    sd = channel_scales(rng, hdim)
    x0 = bf16_bits(rng.standard_normal((m, hdim)))
    gate = np.ones(hdim, np.float32)
    qa, sa = prepare_plain_gpu(h, hdim, hdim)
    up = torch.empty((m, inter), dtype=torch.float16, device="cuda")
    k2.gemm_i8_swiglu(qa, dev(wgu), dev(sgu), sa, up, cfg=cfg(hdim, 2 * inter, hdim))
    qd = torch.empty((m, pitch_i), dtype=torch.int8, device="cuda")
    sdn = torch.empty(m, dtype=torch.float32, device="cuda")
    k2.prepare_plain_i8(up, qd, sdn, width=inter, out_stride=pitch_i)
    x = dev(x0, torch.bfloat16)
    k2.gemm_i8_resid_256x256(qd, dev(wd), dev(sd), sdn, x, dev(gate),
                             cfg=cfg(inter, hdim, pitch_i, int(k2.shape.gemm_schedule_rows(m))))
    sync()
    qa_ref, sa_ref = oracle.prepare_plain(h, hdim, hdim)
    assert np.array_equal(host(qa), qa_ref)
    up_ref = oracle.epilogue_swiglu(oracle.gemm_i32(qa_ref, wgu, m, 2 * inter, hdim, hdim), sgu,
                                    sa_ref)
    assert np.array_equal(host(up), up_ref)
    qd_ref, sd_ref = oracle.prepare_plain(up_ref, inter, pitch_i)
    assert np.array_equal(host(qd), qd_ref)
    assert np.array_equal(host(sdn), sd_ref)
    acc = oracle.gemm_i32(qd_ref, wd, m, hdim, inter, pitch_i)
    assert np.array_equal(host(x), oracle.epilogue_resid(acc, sd, sd_ref, gate, x0))


def test_config3_block_linears_at_4544_tokens():
    # one block of the 3072-hidden DiT at M=4544 through the block session
    # (the benchmark's launcher): prepare_norm -> QKV [9216 x 3072]; prepare_gated(attn,
    # gate = QKV columns 6144..9215) -> out-proj + residual [3072 x 3072];
    # prepare_norm -> SwiGLU up [2 x 12288 x 3072]; prepare_plain -> down + residual
    # [3072 x 12288]. Every intermediate buffer against the oracle chain.
    rng = np.random.default_rng(5000)
    m, hdim, inter, qkv, gate_off, eps = 4544, 3072, 12288, 9216, 6144, 1e-6
    ph, pi = int(k2.shape.gemm_pitch(hdim)), int(k2.shape.gemm_pitch(inter))
    wq, sq = int8_weights(rng, qkv, hdim, ph), channel_scales(rng, qkv)
    wo, so = int8_weights(rng, hdim, hdim, ph), channel_scales(rng, hdim)
    wgu, sgu = int8_weights(rng, 2 * inter, hdim, ph), channel_scales(rng, 2 * inter)
    wd, sd = int8_weights(rng, hdim, inter, pi), channel_scales(rng, hdim)
    prenorm = (rng.uniform(0.5, 1.5, hdim) - 1.0).astype(np.float32)
    postnorm = (rng.uniform(0.5, 1.5, hdim) - 1.0).astype(np.float32)
    mods = np.zeros((1, 6, hdim), np.float32)
    mods[0, (0, 3)] = rng.uniform(-0.2, 0.2, (2, hdim))
    mods[0, (1, 4)] = rng.uniform(-0.1, 0.1, (2, hdim))
    mods[0, (2, 5)] = rng.uniform(0.5, 1.5, (2, hdim))
    x0 = bf16_bits(activations(rng, m, hdim))
    attn0 = f16_bits(activations(rng, m, hdim, outliers=0))
    block = {"qkvg_q": dev(wq), "qkvg_s": dev(sq), "wo_q": dev(wo), "wo_s": dev(so),
             "gu_q": dev(wgu), "gu_s": dev(sgu), "down_q": dev(wd), "down_s": dev(sd),
             "prenorm": dev(prenorm), "postnorm": dev(postnorm)}
    s = BlockSession([block], tokens=m, hidden=hdim, inter=inter, qkvg=qkv,
                     gate_offset=gate_off, eps=eps)
    with torch.cuda.stream(s.stream):
        s.x.copy_(dev(x0, torch.bfloat16))
        s.mods.copy_(dev(mods))
        s.attn_gu[: m * hdim].copy_(dev(attn0.reshape(-1), torch.float16))
    s.pre_attention(0)
    s.stream.synchronize()
    fused = host(s.fused)
    s.post_attention(0)
    s.stream.synchronize()

    q, sc = oracle.prepare_norm(x0, prenorm, mods[0, 0], mods[0, 1], hdim, ph, eps)
    fused_ref = oracle.epilogue_plain(oracle.gemm_i32(q, wq, m, qkv, hdim, ph), sq, sc)
    assert np.array_equal(fused, fused_ref)
    gate = np.concatenate([fused_ref.reshape(-1)[gate_off:], np.zeros(gate_off, np.uint16)])
    q, sc = oracle.prepare_gated(attn0.reshape(-1), gate, hdim, ph, qkv)
    x = oracle.epilogue_resid(oracle.gemm_i32(q, wo, m, hdim, hdim, ph), so, sc, mods[0, 2],
                              x0.reshape(-1)).reshape(m, hdim)
    q, sc = oracle.prepare_norm(x, postnorm, mods[0, 3], mods[0, 4], hdim, ph, eps)
    up = oracle.epilogue_swiglu(oracle.gemm_i32(q, wgu, m, 2 * inter, hdim, ph), sgu, sc)
    assert np.array_equal(host(s.attn_gu)[: m * inter].reshape(m, inter), up)
    q, sc = oracle.prepare_plain(up, inter, pi)
    x = oracle.epilogue_resid(oracle.gemm_i32(q, wd, m, hdim, inter, pi), sd, sc, mods[0, 5],
                              x.reshape(-1)).reshape(m, hdim)
    assert np.array_equal(host(s.x), x)


SKINNY = [(m, g) for m in (1, 16, 77, 256, 512) for g in ("qkv", "up_swiglu", "down_resid")]


@pytest.mark.parametrize("m,gemm", SKINNY)
def test_config4_skinny_sweep(m, gemm):
    # hidden 2560, intermediate 9728; QKV [4096 x 2560], SwiGLU up
    # [2 x 9728 x 2560], down [2560 x 9728] with a bf16 residual; activations prepared
    # from N(0,1) rows with outliers.
    rng = np.random.default_rng(6000 + m)
    hdim, inter = 2560, 9728
    k, n = {"qkv": (hdim, 4096), "up_swiglu": (hdim, 2 * inter), "down_resid": (inter, hdim)}[gemm]
    pitch = int(k2.shape.gemm_pitch(k))
    h = f16_bits(activations(rng, m, k))
    w = int8_weights(rng, n, k, pitch)
    ws = channel_scales(rng, n)
    q, s = prepare_plain_gpu(h, k, pitch)
    q_ref, s_ref = oracle.prepare_plain(h, k, pitch)
    acc = oracle.gemm_i32(q_ref, w, m, n, k, pitch)
    c = cfg(k, n, pitch)
    if gemm == "qkv":
        out = torch.empty((m, n), dtype=torch.float16, device="cuda")
        k2.gemm_i8(q, dev(w), dev(ws), s, out, cfg=c)
        want = oracle.epilogue_plain(acc, ws, s_ref)
    elif gemm == "up_swiglu":
        out = torch.empty((m, n // 2), dtype=torch.float16, device="cuda")
        k2.gemm_i8_swiglu(q, dev(w), dev(ws), s, out, cfg=c)
        want = oracle.epilogue_swiglu(acc, ws, s_ref)
    else:
        x0 = bf16_bits(rng.standard_normal((m, n)))
        gate = np.ones(n, np.float32)
        out = dev(x0, torch.bfloat16)
        k2.gemm_i8_resid(q, dev(w), dev(ws), s, out, dev(gate), cfg=c)
        want = oracle.epilogue_resid(acc, ws, s_ref, gate, x0)
    sync()
    assert np.array_equal(host(q), q_ref)
    assert np.array_equal(host(out).reshape(want.shape), want)


PRODUCTION = [(name, m) for name in ("gemm_qkvg", "gemm_gu", "gemm_wo", "gemm_down")
              for m in (12301, 16397)]


@pytest.mark.parametrize("name,m", PRODUCTION)
def test_production_gemm_at_the_largest_token_counts(name, m):
    # The reference's bench matrix (benches/kernels.rs:58-64) at M=12301 and 16397 (ragged
    # 256-row tiles; the most tile rounds). Full-size int64 row and column checksums of
    # the int32 accumulators (size-independent identities), then 40 rows (two per 1024,
    # the first and the last) exact through the production epilogue against the oracle.
    k, n, kind = {"gemm_qkvg": (6144, 15360, "plain"), "gemm_gu": (6144, 32768, "swiglu"),
                  "gemm_wo": (6144, 6144, "resid"), "gemm_down": (16384, 6144, "resid_wide")}[name]
    rng = np.random.default_rng(7000 + m + k + n)
    pitch = int(k2.shape.gemm_pitch(k))
    a = int8_weights(rng, m, k, pitch)
    w = int8_weights(rng, n, k, pitch)
    ws = channel_scales(rng, n)
    sc = rng.uniform(1e-3, 3e-2, m).astype(np.float32)
    A, W = dev(a), dev(w)
    c = cfg(k, n, pitch, int(k2.shape.gemm_schedule_rows(m)))
    acc = torch.empty((m, n), dtype=torch.int32, device="cuda")
    k2.gemm_i8_acc(A, W, acc, cfg=c)
    Ak, Wk = A[:, :k].to(torch.int64), W[:, :k].to(torch.int64)
    assert torch.equal(acc.to(torch.int64).sum(1), (Ak * Wk.sum(0)).sum(1))
    assert torch.equal(acc.to(torch.int64).sum(0), (Wk * Ak.sum(0)).sum(1))
    del Ak, Wk
    rows = np.unique(np.concatenate([rng.choice(m, 38, replace=False), [0, m - 1]]))
    ref = oracle.gemm_i32(a[rows], w, len(rows), n, k, pitch)
    pick = torch.from_numpy(rows).cuda()
    assert np.array_equal(host(acc[pick]), ref)
    del acc
    if kind == "plain":
        out = torch.empty((m, n), dtype=torch.float16, device="cuda")
        k2.gemm_i8(A, W, dev(ws), dev(sc), out, cfg=c)
        want = oracle.epilogue_plain(ref, ws, sc[rows])
    elif kind == "swiglu":
        out = torch.empty((m, n // 2), dtype=torch.float16, device="cuda")
        k2.gemm_i8_swiglu(A, W, dev(ws), dev(sc), out, cfg=c)
        want = oracle.epilogue_swiglu(ref, ws, sc[rows])
    else:
        x0 = bf16_bits(rng.standard_normal((m, n)).astype(np.float32))
        gate = rng.uniform(0.5, 1.5, n).astype(np.float32)
        out = dev(x0, torch.bfloat16)
        op = k2.gemm_i8_resid if kind == "resid" else k2.gemm_i8_resid_256x256
        op(A, W, dev(ws), dev(sc), out, dev(gate), cfg=c)
        want = oracle.epilogue_resid(ref, ws, sc[rows], gate, x0[rows])
    sync()
    assert np.array_equal(host(out[pick]), want)
