#!/usr/bin/env python3
"""Benchmark of the MI355X W8A8 transformer-product path (one GPU).

Headline (BASELINE.json `metric`): W8A8 GEMM TOPS and % of dense INT8 MFMA peak at
M=4096, K=3072; DiT block linear ms.

A step is BASELINE configs[1], the fused attention-input projection: an f16-valued
hidden state [4096, 3072] (bf16 on the wire, as the reference's prepare_norm takes)
-> prepare_norm_i8 (RMSNorm, group-256 Hadamard, per-token int8) -> gemm_i8 QKV with
int8 W [9216, 3072] and per-channel scales -> f16 [4096, 9216]. `value` is that step's
whole-job throughput in TOPS (2*M*N*K per step), inputs resident in HBM. Operand sets
rotate through several copies so the 256 MB MALL cannot hold them between steps.

Also reported: the north-star GEMM alone (M=4096, K=3072, N=12288), the per-block
linear sequence of configs[3] (M=4544, 8 blocks) in ms per block, the dominant
kernel's roofline (HIP events on the launch stream), and the CPU oracle timed on a
bounded sample on this host (cpu_baseline).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "krea2-hrx_amd"))

PEAK_INT8_TOPS = 5000.0  # MI355X dense INT8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0
PEAK_F16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
COPY_PROBE_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_i8_qkv_4096x3072x9216_traffic.json")
METRIC = "W8A8 GEMM TOPS and % of INT8 MFMA peak at M=4096,K=3072; DiT block linear ms"


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-extra", action="store_true", help="headline step only")
    p.add_argument("--backward-k", action="store_true",
                   help="also time the north star with odd rounds stepping through K backwards "
                        "(K2W8_GEMM_BACKWARD=1, an opt-in variant)")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--probe", choices=["north_star", "skinny", "attention", "mfma_peak"],
                   help="run one workload a few times and exit (a short program for "
                        "rocprofv3 --pmc counter passes)")
    p.add_argument("--traffic-probe", action="store_true",
                   help="run a 256 MiB device copy and 5 QKV steps only (for rocprofv3 --pmc "
                        "FETCH_SIZE / WRITE_SIZE passes)")
    return p.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import krea2_w8a8 as k2

    torch.cuda.set_device(0)
    dev = "cuda"
    gen = torch.Generator(device=dev)
    gen.manual_seed(2000)

    M, K, N = 4096, 3072, 9216
    pitch = k2.shape.gemm_pitch(K)

    def hidden(rows, cols, seed):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        x = torch.randn((rows, cols), generator=g, device=dev, dtype=torch.float32)
        ch = torch.randperm(cols, generator=g, device=dev)[:8]
        x[:, ch] *= 20.0
        return x

    def weights(rows, cols, seed):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        w = torch.randint(-127, 128, (rows, cols), generator=g, device=dev, dtype=torch.int8)
        s = torch.rand(rows, generator=g, device=dev) * 9e-3 + 1e-3
        return w, s

    if args.probe:
        args.steps, args.warmup = 3, 1
        if args.probe == "north_star":
            print(json.dumps(north_star(k2, torch, weights, hidden, args)), flush=True)
        elif args.probe == "mfma_peak":
            print(json.dumps(mfma_peak(k2, torch)), flush=True)
        elif args.probe == "skinny":
            skinny_sweep(k2, torch, weights, hidden, args, warm=False)
        else:
            attention_production(k2, torch, args)
        torch.cuda.synchronize()
        print(f"probe {args.probe} done", flush=True)
        return

    # --- headline step: configs[1] -------------------------------------------------
    copies = 4  # 4 x ~140 MB of operands > 256 MB MALL
    sets = []
    for c in range(copies):
        h = hidden(M, K, 2100 + c).to(torch.float16).to(torch.bfloat16)  # f16 values, bf16 wire
        w, ws = weights(N, pitch, 2200 + c)
        sets.append(dict(
            h=h,
            ns=(torch.rand(K, generator=gen, device=dev) - 0.5),  # w - 1, w ~ U(0.5, 1.5)
            zero=torch.zeros(K, device=dev),
            q=torch.empty((M, pitch), dtype=torch.int8, device=dev),
            s=torch.empty(M, dtype=torch.float32, device=dev),
            w=w, ws=ws,
            out=torch.empty((M, N), dtype=torch.float16, device=dev),
        ))
    cfg = k2.GemmConfig(k_size=K, n_size=N, k_stride=pitch, m_group=k2.shape.gemm_m_group())
    stream = torch.cuda.current_stream()

    def step(i, ev=None):
        d = sets[i % copies]
        if ev is not None:
            ev[0].record(stream)
        k2.prepare_norm_i8(d["h"], d["ns"], d["zero"], d["zero"], d["q"], d["s"], width=K,
                           out_stride=pitch, eps=1e-6)
        if ev is not None:
            ev[1].record(stream)
        k2.gemm_i8(d["q"], d["w"], d["ws"], d["s"], d["out"], cfg=cfg)
        if ev is not None:
            ev[2].record(stream)

    if args.traffic_probe:
        # The copy kernel of known size that calibrates the byte counters.
        src = torch.empty(COPY_PROBE_BYTES, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        dst.copy_(src)
        for i in range(5):
            step(i)
        torch.cuda.synchronize()
        print("traffic probe done", flush=True)
        return

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # Eager: one host call per kernel.
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step_eager = (t1 - t0) * 1e3 / args.steps
    # The timed run: the K steps recorded once into a HIP graph and replayed, as the
    # reference's session records its launch sequence (src/session/mod.rs:596-616).
    # Same kernels, same operands, same order; only the host launches are batched.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(args.steps):
            step(i)
    graph.replay()  # warm replay
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    graph.replay()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    del graph
    ops_step = 2.0 * M * N * K
    value = ops_step / (ms_per_step * 1e-3) / 1e12

    # Per-kernel durations: HIP events on the launch stream over a second timed pass.
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for i in range(args.steps):
        step(i, evs[i])
    torch.cuda.synchronize()
    prep_us = sum(e[0].elapsed_time(e[1]) for e in evs) * 1e3 / args.steps
    gemm_us = sum(e[1].elapsed_time(e[2]) for e in evs) * 1e3 / args.steps
    gemm_tops = ops_step / (gemm_us * 1e-6) / 1e12
    prep_bytes = 2 * M * K + M * K + 4 * M + 4 * K
    gemm_bytes = M * K + N * K + 4 * N + 4 * M + 2 * M * N

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "ms_per_step_eager": round(ms_per_step_eager, 4),
        "timing": "K steps recorded into one HIP graph, replayed once between device syncs",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,1) activations with 8 outlier channels x20, int8 U[-127,127] weights)",
        "config": {
            "workload": "configs[1] fused attention-input projection: prepare_norm_i8 -> gemm_i8 (QKV)",
            "M": M, "K": K, "N": N, "k_stride": pitch, "eps": 1e-6,
            "ops_per_step": ops_step,
            "pct_of_int8_peak": round(100.0 * value / PEAK_INT8_TOPS, 2),
        },
        "kernels": {
            "prepare_norm_i8_us": round(prep_us, 2),
            "prepare_norm_i8_GBps": round(prep_bytes / (prep_us * 1e-6) / 1e9, 1),
            "gemm_i8_us": round(gemm_us, 2),
            "gemm_i8_TOPS": round(gemm_tops, 1),
        },
        "roofline": {
            "kernel": "gemm_i8 (QKV, M=4096 K=3072 N=9216): one launch of 256x192 tiles",
            "bound": "mfma",
            "achieved": round(gemm_tops, 1),
            "peak": PEAK_INT8_TOPS,
            "unit": "TOPS",
            "frac": round(gemm_tops / PEAK_INT8_TOPS, 4),
            "traffic": measured_traffic(),
            "traffic_source": traffic_source(),
            "algorithmic_bytes": gemm_bytes,
        },
    }
    del sets
    torch.cuda.empty_cache()

    if not args.no_extra:
        result["north_star"] = north_star(k2, torch, weights, hidden, args)
        torch.cuda.empty_cache()
        result["config1_single_gemm"] = single_gemm(k2, torch, weights, hidden, args)
        torch.cuda.empty_cache()
        result["config3_mlp_pair"] = mlp_pair(k2, torch, weights, hidden, args)
        torch.cuda.empty_cache()
        result["block_linears"] = block_linears(k2, torch, weights, hidden, args)
        torch.cuda.empty_cache()
        result["block_with_attention"] = block_linears(k2, torch, weights, hidden, args,
                                                       attention=True)
        torch.cuda.empty_cache()
        result["attention_production"] = attention_production(k2, torch, args)
        torch.cuda.empty_cache()
        result["config5_skinny"] = skinny_sweep(k2, torch, weights, hidden, args)
        torch.cuda.empty_cache()
        result["production_gemms"] = production_gemms(k2, torch, args)
        torch.cuda.empty_cache()

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(M, K, N, pitch, args.cpu_seconds)
    result["gemm_kernel_choice"] = kernel_choices(k2, torch.cuda.get_device_properties(0).multi_processor_count)

    print(json.dumps(result), flush=True)


def kernel_choices(k2, cus):
    """The kernel and tile each benchmarked GEMM shape runs on this device
    (k2w8_gemm_choose: the rule the GEMM entry points apply; no launch)."""
    shapes = [("configs[1] QKV", 4096, 3072, 9216, "plain"), ("north star", 4096, 3072, 12288, "plain"),
              ("configs[0]", 4096, 3072, 3072, "bias"), ("configs[2] up", 4608, 3072, 24576, "swiglu"),
              ("configs[2] down", 4608, 12288, 3072, "resid"), ("configs[3] qkv", 4544, 3072, 9216, "plain"),
              ("configs[3] wo", 4544, 3072, 3072, "resid"), ("configs[3] up", 4544, 3072, 24576, "swiglu"),
              ("configs[3] down", 4544, 12288, 3072, "resid")]
    for m in (1, 16, 77, 256, 512):
        shapes += [(f"configs[4] qkv M={m}", m, 2560, 4096, "plain"), (f"configs[4] up M={m}", m, 2560, 19456, "swiglu"),
                   (f"configs[4] down M={m}", m, 9728, 2560, "resid")]
    out = {"cus": cus}
    for name, m, k, n, epi in shapes:
        c = k2.gemm_choose(m, cfg=k2.GemmConfig(k_size=k, n_size=n, k_stride=k2.shape.gemm_pitch(k)),
                           epilogue=epi, cus=cus)
        out[name] = c["kernel"] + (f" {c['tile'][0]}x{c['tile'][1]}" if "tile" in c else "") + (
            f" x{c['splits']} slices" if "splits" in c else "")
    return out


def measured_traffic():
    """HBM bytes per gemm_i8 launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes (calibrated against a copy kernel), or None if they are absent. The counters
    cannot be read inside this run (they need rocprofv3 --pmc passes of their own), so
    the value is the committed profile's, and traffic_source() names it."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["gemm_i8"]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def traffic_source():
    """Where roofline.traffic comes from: the profile file, the launch and the build it
    measured, and that this run did not measure it."""
    src = {"file": os.path.relpath(TRAFFIC_FILE, ROOT), "measured_in_this_run": False}
    try:
        with open(TRAFFIC_FILE) as f:
            d = json.load(f)
        src.update(launch=d["gemm_i8"]["launch"], build=d.get("measured_build"), commands=d["commands"])
    except (OSError, KeyError, ValueError):
        src["missing"] = True
    return src


def event_timed(torch, fn, steps, warmup):
    """Mean GPU time of fn's launches: HIP events recorded on the launch stream around each
    call, so host-side launch overhead between calls is excluded."""
    for i in range(warmup):
        fn(i)
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    # Keep the GPU busy while the host enqueues, so that each event pair brackets only
    # its kernels and not the host's launch latency (~40 us of spin per step queued).
    torch.cuda.synchronize()
    torch.cuda._sleep(int(steps * 40e-6 * 2.4e9))
    for i, (e0, e1) in enumerate(evs):
        e0.record(stream)
        fn(i)
        e1.record(stream)
    torch.cuda.synchronize()
    return sum(e0.elapsed_time(e1) for e0, e1 in evs) * 1e-3 / steps


def batch_timed(torch, fn, steps, warmup):
    """Mean GPU time per call of `steps` calls launched back to back: one HIP event pair
    on the launch stream around the whole batch. The GPU is kept busy while the host
    enqueues, so the batch runs as the device executes it (each launch's dispatch
    overlapping the previous kernel), without the host's per-call overhead."""
    for i in range(warmup):
        fn(i)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    torch.cuda._sleep(int(steps * 40e-6 * 2.4e9))
    e0.record(stream)
    for i in range(steps):
        fn(i)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e-3 / steps


def mfma_peak(k2, torch):
    """The INT8 MFMA rate with nothing but MFMAs running (k2w8_probe_mfma_i8): two waves
    per SIMD on every CU, register operands of pseudo-random bytes and of bytes of 1.
    The chip's power limit sets the clock it holds, and the MFMA's power depends on its
    operand bits: this is the ceiling the tile GEMM is measured against."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks, iters = 2 * cus, 20000
    out = torch.empty(blocks * 256, dtype=torch.int32, device="cuda")
    res = {"blocks": blocks, "iters": iters}
    for name, random in (("random", True), ("ones", False)):
        def fn(_):
            k2.probe_mfma_i8(out, blocks=blocks, iters=iters, random=random)
        sec = event_timed(torch, fn, 5, 2)
        tops = blocks * iters * float(1 << 21) / sec / 1e12  # 4 waves x 8 MFMAs x 2^16 ops
        res[name] = {"us": round(sec * 1e6, 1), "TOPS": round(tops, 1),
                     "pct_of_int8_peak": round(100 * tops / PEAK_INT8_TOPS, 1)}
    return res


def north_star(k2, torch, weights, hidden, args):
    """The target GEMM: M=4096, K=3072, N=12288, plain epilogue, timed by HIP events on the
    launch stream. Its A operand is what the path feeds it: f16 N(0,1) rows with 8
    outlier channels x20 through prepare_plain_i8 (the north star's prepare -> GEMM).
    The MFMAs' power, and so the clock the chip holds, depends on the operand bytes, so
    the same GEMM on uniform random int8 A (every bit toggling) is reported beside it."""
    M, K, N = 4096, 3072, 12288
    copies = 3
    hs = [hidden(M, K, 3100 + c).to(torch.float16) for c in range(copies)]
    a = [torch.empty((M, K), device="cuda", dtype=torch.int8) for _ in range(copies)]
    s = [torch.empty(M, device="cuda") for _ in range(copies)]
    for c in range(copies):
        k2.prepare_plain_i8(hs[c], a[c], s[c], width=K, out_stride=K)
    au = [torch.randint(-127, 128, (M, K), device="cuda", dtype=torch.int8) for _ in range(copies)]
    ws = [weights(N, K, 3000 + c) for c in range(copies)]
    out = [torch.empty((M, N), dtype=torch.float16, device="cuda") for _ in range(copies)]
    cfg = k2.GemmConfig(k_size=K, n_size=N, k_stride=K)

    def gemm(i, ops=a):
        c = i % copies
        k2.gemm_i8(ops[c], ws[c][0], ws[c][1], s[c], out[c], cfg=cfg)

    def chain(i):
        c = i % copies
        k2.prepare_plain_i8(hs[c], a[c], s[c], width=K, out_stride=K)
        gemm(i)

    def one_launch(i):
        c = i % copies
        k2.linear_plain_i8(hs[c], a[c], s[c], ws[c][0], ws[c][1], out[c], cfg=cfg)

    # Weights as a W8A8 checkpoint holds them: N(0,1) rows quantised per channel by
    # absmax to [-127, 127] (most codes small), against the uniform random bytes above.
    def gauss_weights(c):
        g = torch.Generator(device="cuda")
        g.manual_seed(3300 + c)
        x = torch.randn((N, K), generator=g, device="cuda")
        return torch.round(x * (127.0 / x.abs().amax(dim=1, keepdim=True))).to(torch.int8)
    wg = [gauss_weights(c) for c in range(copies)]

    def gemm_gauss_w(i):
        c = i % copies
        k2.gemm_i8(a[c], wg[c], ws[c][1], s[c], out[c], cfg=cfg)

    sec = event_timed(torch, gemm, args.steps, args.warmup)
    sec_u = event_timed(torch, lambda i: gemm(i, au), args.steps, args.warmup)
    sec_g = event_timed(torch, gemm_gauss_w, args.steps, args.warmup)
    sec_c = event_timed(torch, chain, args.steps, args.warmup)
    # The fused prepare -> GEMM as one persistent launch (same bits; not the default).
    os.environ["K2W8_LINEAR_ONE_LAUNCH"] = "1"
    sec_f = event_timed(torch, one_launch, args.steps, args.warmup)
    os.environ["K2W8_LINEAR_ONE_LAUNCH"] = "0"
    # Odd rounds stepping through K backwards (same bits; fewer L2 misses by the model),
    # on request only: an opt-in variant.
    sec_b = None
    if args.backward_k:
        os.environ["K2W8_GEMM_BACKWARD"] = "1"
        sec_b = event_timed(torch, gemm, args.steps, args.warmup)
        os.environ["K2W8_GEMM_BACKWARD"] = "0"
    ops = 2.0 * M * N * K
    tops = ops / sec / 1e12
    return {"M": M, "K": K, "N": N, "us": round(sec * 1e6, 2), "TOPS": round(tops, 1),
            "pct_of_int8_peak": round(100 * tops / PEAK_INT8_TOPS, 2), "target_pct": 60.0,
            "a_operand": "prepare_plain_i8 of f16 N(0,1) rows with 8 outlier channels x20",
            "us_uniform_a": round(sec_u * 1e6, 2),
            "pct_of_int8_peak_uniform_a": round(100 * ops / sec_u / 1e12 / PEAK_INT8_TOPS, 2),
            "us_checkpoint_like_w": round(sec_g * 1e6, 2),
            "pct_of_int8_peak_checkpoint_like_w": round(100 * ops / sec_g / 1e12 / PEAK_INT8_TOPS, 2),
            "us_prepare_plus_gemm": round(sec_c * 1e6, 2),
            "pct_of_int8_peak_prepare_plus_gemm": round(100 * ops / sec_c / 1e12 / PEAK_INT8_TOPS, 2),
            "us_prepare_gemm_one_launch": round(sec_f * 1e6, 2),
            "us_backward_k_odd_rounds": round(sec_b * 1e6, 2) if sec_b is not None else None,
            "timing": "HIP events on the launch stream around each call, mean"}


def single_gemm(k2, torch, weights, hidden, args):
    """f16 A [4096, 3072] quantised per token (prepare_plain_i8) -> gemm_i8 with
    int8 W [3072, 3072], per-channel scales and an f16 bias (gemm_i8_bias) -> f16 out."""
    M, K, N = 4096, 3072, 3072
    h = hidden(M, K, 1000).to(torch.float16)
    q = torch.empty((M, K), dtype=torch.int8, device="cuda")
    qs = torch.empty(M, dtype=torch.float32, device="cuda")
    w, ws = weights(N, K, 1001)
    g = torch.Generator(device="cuda")
    g.manual_seed(1002)
    bias = (torch.randn(N, generator=g, device="cuda") * 0.02).to(torch.float16)
    out = torch.empty((M, N), dtype=torch.float16, device="cuda")
    cfg = k2.GemmConfig(K, N, K)

    def fn(_):
        k2.prepare_plain_i8(h, q, qs, width=K, out_stride=K)
        k2.gemm_i8_bias(q, w, ws, qs, bias, out, cfg=cfg)

    sec = event_timed(torch, fn, args.steps, args.warmup)
    gsec = event_timed(torch, lambda _: k2.gemm_i8_bias(q, w, ws, qs, bias, out, cfg=cfg),
                       args.steps, args.warmup)
    ops = 2.0 * M * N * K
    return {"M": M, "K": K, "N": N, "us_prepare_plus_gemm": round(sec * 1e6, 2),
            "us_gemm": round(gsec * 1e6, 2), "TOPS_gemm": round(ops / gsec / 1e12, 1),
            "TOPS_with_prepare": round(ops / sec / 1e12, 1)}


def mlp_pair(k2, torch, weights, hidden, args):
    """M=4608 -> gemm_i8_swiglu (W [2x12288, 3072], interleaved) -> f16 [4608, 12288]
    -> prepare_plain_i8 -> gemm_i8_resid_256x256 (W [3072, 12288]) on a bf16 residual."""
    M, H, I = 4608, 3072, 12288
    pitch_i = k2.shape.gemm_pitch(I)
    qa = torch.randint(-127, 128, (M, H), device="cuda", dtype=torch.int8)
    qas = torch.rand(M, device="cuda") * 1e-2 + 1e-3
    wgu, sgu = weights(2 * I, H, 3100)
    wd, sd = weights(H, pitch_i, 3101)
    up = torch.empty((M, I), dtype=torch.float16, device="cuda")
    q = torch.empty((M, pitch_i), dtype=torch.int8, device="cuda")
    qs = torch.empty(M, dtype=torch.float32, device="cuda")
    x = hidden(M, H, 3102).to(torch.bfloat16)
    one = torch.ones(H, device="cuda")
    c_gu = k2.GemmConfig(H, 2 * I, H)
    c_d = k2.GemmConfig(I, H, pitch_i, schedule_rows=int(k2.shape.gemm_schedule_rows(M)))

    def fn(_):
        k2.gemm_i8_swiglu(qa, wgu, sgu, qas, up, cfg=c_gu)
        k2.prepare_plain_i8(up, q, qs, width=I, out_stride=pitch_i)
        k2.gemm_i8_resid_256x256(q, wd, sd, qs, x, one, cfg=c_d)

    sec = event_timed(torch, fn, max(2, args.steps // 2), max(1, args.warmup // 2))
    ops = 2.0 * M * H * 2 * I + 2.0 * M * I * H
    return {"M": M, "ms": round(sec * 1e3, 4), "TOPS": round(ops / sec / 1e12, 1),
            "pct_of_int8_peak": round(100 * ops / sec / 1e12 / PEAK_INT8_TOPS, 2)}


def production_gemms(k2, torch, args):
    """The reference's own GEMM benchmark matrix (benches/kernels.rs:58-64): the four
    production projections at hidden 6144 -- qkvg (K=6144, N=15360), gate|up + SwiGLU
    (N=32768), wo + residual (6144x6144) and down + residual (K=16384, pitch 16448, its
    256x256 kernel) -- at M in {1043, 4095, 4096, 4109, 12301, 16397}, with that bench's
    operands (bytes (73 i + salt) mod 255 within K, zero padding; scales 1e-3 / 1e-2,
    residual gate 0.25). Times are HIP events on the launch stream, mean per call."""
    rows = []
    for name, k, n, kind in [("gemm_qkvg", 6144, 15360, "plain"), ("gemm_gu", 6144, 32768, "swiglu"),
                             ("gemm_wo", 6144, 6144, "resid"), ("gemm_down", 16384, 6144, "resid_wide")]:
        pitch = int(k2.shape.gemm_pitch(k))

        def operand(r, salt):
            i = torch.arange(r * pitch, device="cuda", dtype=torch.int64)
            v = ((i * 73 + salt) % 255).to(torch.uint8).view(torch.int8).reshape(r, pitch)
            v[:, k:] = 0
            return v

        w = operand(n, 31)
        ws = torch.full((n,), 1e-3, device="cuda")
        gate = torch.full((n,), 0.25, device="cuda")
        for m in (1043, 4095, 4096, 4109, 12301, 16397):
            a = operand(m, 17)
            sc = torch.full((m,), 1e-2, device="cuda")
            cfg = k2.GemmConfig(k_size=k, n_size=n, k_stride=pitch,
                                schedule_rows=int(k2.shape.gemm_schedule_rows(m)))
            if kind == "swiglu":
                out = torch.empty((m, n // 2), dtype=torch.float16, device="cuda")
                fn = lambda _: k2.gemm_i8_swiglu(a, w, ws, sc, out, cfg=cfg)  # noqa: E731
            elif kind == "plain":
                out = torch.empty((m, n), dtype=torch.float16, device="cuda")
                fn = lambda _: k2.gemm_i8(a, w, ws, sc, out, cfg=cfg)  # noqa: E731
            else:
                out = torch.zeros((m, n), dtype=torch.bfloat16, device="cuda")
                op = k2.gemm_i8_resid if kind == "resid" else k2.gemm_i8_resid_256x256
                fn = lambda _: op(a, w, ws, sc, out, gate, cfg=cfg)  # noqa: E731
            steps = max(3, min(args.steps, 20))
            sec = event_timed(torch, fn, steps, 2)
            tops = 2.0 * m * n * k / sec / 1e12
            rows.append({"gemm": name, "M": m, "K": k, "N": n, "us": round(sec * 1e6, 2),
                         "TOPS": round(tops, 1),
                         "pct_of_int8_peak": round(100 * tops / PEAK_INT8_TOPS, 2)})
            del a, out
        del w
        torch.cuda.empty_cache()
    return rows


COLD_BYTES = 320 << 20  # weight copies rotated per call: more than the 256 MB MALL


def skinny_sweep(k2, torch, weights, hidden, args, sizes=(1, 16, 77, 256, 512), warm=True):
    """text-encoder-shaped few-token regime, hidden 2560, intermediate 9728:
    QKV [4096 x 2560], SwiGLU up [2 x 9728 x 2560], down [2560 x 9728] (with residual) for
    M in {1, 16, 77, 256, 512}. HBM-bound on the weights at small M: reported as GB/s of
    algorithmic bytes against the 8 TB/s peak.

    ``GBps`` is MALL-cold: each call reads a different copy of the weights, enough copies
    (more than 256 MB) that none is still in the MALL when it comes round again.
    ``GBps_warm`` repeats one copy (weights served from the MALL). Calls run back to back
    (one event pair around the batch), as a text encoder's launches do."""
    H, I = 2560, 9728
    pitch_i = k2.shape.gemm_pitch(I)

    def copies(rows, cols, seed):
        n = max(2, -(-COLD_BYTES // (rows * cols)))
        return [weights(rows, cols, seed + 100 * c) for c in range(n)]

    wq, wgu, wd = copies(4096, H, 5100), copies(2 * I, H, 5101), copies(H, pitch_i, 5102)
    one = torch.ones(H, device="cuda")
    rows = []
    for M in sizes:
        a_h = torch.randint(-127, 128, (M, H), device="cuda", dtype=torch.int8)
        a_i = torch.randint(-127, 128, (M, pitch_i), device="cuda", dtype=torch.int8)
        sc = torch.rand(M, device="cuda") * 1e-2 + 1e-3
        o_q = torch.empty((M, 4096), dtype=torch.float16, device="cuda")
        o_u = torch.empty((M, I), dtype=torch.float16, device="cuda")
        x = torch.zeros((M, H), dtype=torch.bfloat16, device="cuda")
        cfg_q, cfg_u, cfg_d = k2.GemmConfig(H, 4096, H), k2.GemmConfig(H, 2 * I, H), \
            k2.GemmConfig(I, H, pitch_i)
        cases = [
            ("qkv", lambda i, w: k2.gemm_i8(a_h, w[i % len(w)][0], w[i % len(w)][1], sc, o_q,
                                            cfg=cfg_q), wq, 4096, H, 2 * M * 4096),
            ("up_swiglu", lambda i, w: k2.gemm_i8_swiglu(a_h, w[i % len(w)][0], w[i % len(w)][1],
                                                         sc, o_u, cfg=cfg_u),
             wgu, 2 * I, H, 2 * M * I),
            ("down_resid", lambda i, w: k2.gemm_i8_resid(a_i, w[i % len(w)][0], w[i % len(w)][1],
                                                         sc, x, one, cfg=cfg_d),
             wd, H, I, 4 * M * H),
        ]
        for name, fn, w, n, k, out_bytes in cases:
            byts = n * k + M * k + 4 * n + 4 * M + out_bytes
            steps = max(2 * len(w), args.steps)
            sec = batch_timed(torch, lambda i: fn(i, w), steps, len(w))
            row = {"M": M, "gemm": name, "N": n, "K": k, "us": round(sec * 1e6, 2),
                   "GBps": round(byts / sec / 1e9, 1),
                   "pct_of_hbm_peak": round(100 * byts / sec / 1e9 / PEAK_HBM_GBS, 1),
                   "TOPS": round(2.0 * M * n * k / sec / 1e12, 1)}
            if warm:
                sec_w = batch_timed(torch, lambda i: fn(0, w), max(20, args.steps), 5)
                row["us_warm"] = round(sec_w * 1e6, 2)
                row["GBps_warm"] = round(byts / sec_w / 1e9, 1)
            rows.append(row)
    return rows


def block_linears(k2, torch, weights, hidden, args, attention=False):
    """the per-block linear sequence of a 3072-hidden DiT, M=4544, 8 blocks
    with the same weights, recorded once into a hipGraph and replayed.

    With ``attention`` each block also runs the attention step between the QKV GEMM and
    the gated prepare (q/k norm + rope, V transpose, f16 attention over 24 query and 12
    key-value heads of 128, as the 9216-wide QKV output splits): the whole block.

    Per block, the reference's W8A8 stages in order (src/session/mod.rs:671-840, attention
    excluded): prepare_norm -> QKV [9216x3072]; prepare_gated(attn, gate) -> out-proj
    with residual [3072x3072]; prepare_norm -> SwiGLU up [2x12288x3072]; prepare_plain
    -> down with residual [3072x12288]. The "attention output" is whatever the session's
    attention buffer holds and the gate half is the QKV output's last 3072 columns.
    """
    from krea2_w8a8.block import BlockSession

    M, H, I = 4544, 3072, 12288
    blocks = 8
    pitch_h, pitch_i = k2.shape.gemm_pitch(H), k2.shape.gemm_pitch(I)
    wq, sq = weights(9216, pitch_h, 4100)
    wo, so = weights(H, pitch_h, 4101)
    wgu, sgu = weights(2 * I, pitch_h, 4102)
    wd, sd = weights(H, pitch_i, 4103)
    norm = torch.rand(H, device="cuda") - 0.5
    block = {"qkvg_q": wq, "qkvg_s": sq, "wo_q": wo, "wo_s": so, "gu_q": wgu, "gu_s": sgu,
             "down_q": wd, "down_s": sd, "prenorm": norm, "postnorm": norm,
             "qnorm": norm[:128].contiguous(), "knorm": norm[128:256].contiguous()}
    session = BlockSession([block] * blocks, tokens=M, hidden=H, inter=I, qkvg=9216,
                           gate_offset=6144, eps=1e-6, attention=attention)
    with torch.cuda.stream(session.stream):
        session.x.copy_(hidden(M, H, 4000).to(torch.bfloat16))
        session.attn_gu[: M * H].copy_(hidden(M, H, 4001).to(torch.float16).reshape(-1))
        session.mods[:, (2, 5)] = 1.0  # residual gates; scales and shifts zero
        if attention:
            ang = torch.rand((M, 64), device="cuda") * 6.3
            session.cos.copy_(torch.cos(ang).repeat_interleave(2, dim=1))
            session.sin.copy_(torch.sin(ang).repeat_interleave(2, dim=1))
    session.record()
    steps = max(2, args.steps // 8)
    for _ in range(max(1, args.warmup // 4)):
        session.replay()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(session.stream):
        e0.record()
        for _ in range(steps):
            session.replay()
        e1.record()
    session.stream.synchronize()
    ms_block = e0.elapsed_time(e1) / (steps * blocks)
    stages = {k: round(v / blocks, 1) for k, v in session.profile().items()}
    ops_block = 2.0 * M * H * (9216 + H + 2 * I) + 2.0 * M * I * H
    out = {"M": M, "hidden": H, "intermediate": I, "blocks": blocks, "replay": "hipGraph",
           "ms_per_block": round(ms_block, 4),
           "TOPS": round(ops_block / (ms_block * 1e-3) / 1e12, 1),
           "ideal_ms_per_block_at_peak": round(ops_block / (PEAK_INT8_TOPS * 1e12) * 1e3, 4),
           "stage_us_per_block_eager": stages}
    if attention:
        flops_attn = 4.0 * M * M * 128 * (H // 128)
        ideal = ops_block / (PEAK_INT8_TOPS * 1e12) + flops_attn / (PEAK_F16_TFLOPS * 1e12)
        out.update({"attention": "24 query / 12 key-value heads of 128, non-causal, f16",
                    "attention_flops_per_block": flops_attn,
                    "attention_TFLOPs": round(flops_attn / (stages["f16 attention"] * 1e-6) / 1e12, 1),
                    "ideal_ms_per_block_at_peak": round(ideal * 1e3, 4)})
        del out["TOPS"]
    return out


def attention_production(k2, torch, args):
    """The attention step at the reference's production heads (48 query, 12 key-value
    heads of 128; src/session/mod.rs:37-45) for M=4544 tokens: rope_qknorm, V transpose
    and the f16 attention kernel, each timed with HIP events (inputs resident)."""
    M, QH, KVH = 4544, 48, 12
    cap = k2.shape.capacity(M)
    qkvg = (QH + 2 * KVH) * 128 + QH * 128
    g = torch.Generator(device="cuda").manual_seed(4200)
    fused = torch.randn((M, qkvg), device="cuda", generator=g).half()
    qs = torch.rand(128, device="cuda", generator=g) - 0.5
    ang = torch.rand((M, 64), device="cuda", generator=g) * 6.3
    cos = torch.cos(ang).repeat_interleave(2, dim=1).contiguous()
    sin = torch.sin(ang).repeat_interleave(2, dim=1).contiguous()
    q = torch.zeros((cap, QH * 128), device="cuda", dtype=torch.float16)
    k = torch.zeros((cap, KVH * 128), device="cuda", dtype=torch.float16)
    v = torch.zeros_like(k)
    vt = torch.zeros((KVH * 128, cap), device="cuda", dtype=torch.float16)
    out = torch.empty((M, QH * 128), device="cuda", dtype=torch.float16)
    rope = lambda _: k2.rope_qknorm_f16(fused, qs, qs, cos, sin, q, k, v, row_stride=qkvg,
                                        q_heads=QH, kv_heads=KVH, k_offset=QH * 128, eps=1e-5)
    trans = lambda _: k2.v_transpose(v, vt, width=KVH * 128, row_capacity=cap, rows=M)
    attn = lambda _: k2.attention_f16(q, k, vt, out, q_stride=QH * 128, kv_stride=KVH * 128,
                                      out_stride=QH * 128, tokens=M, token_capacity=cap,
                                      scale=0.08838834764831845, kv_heads=KVH)
    steps = max(3, args.steps // 5)
    t_rope = event_timed(torch, rope, steps, 2)
    t_trans = event_timed(torch, trans, steps, 2)
    t_attn = event_timed(torch, attn, steps, 2)
    flops = 4.0 * M * M * 128 * QH
    rope_bytes = M * (QH + 2 * KVH) * 128 * 2 * 2 + 2 * M * 128 * 4
    return {"M": M, "q_heads": QH, "kv_heads": KVH,
            "rope_qknorm_us": round(t_rope * 1e6, 2),
            "rope_qknorm_GBps": round(rope_bytes / t_rope / 1e9, 1),
            "v_transpose_us": round(t_trans * 1e6, 2),
            "attention_us": round(t_attn * 1e6, 2),
            "attention_TFLOPs": round(flops / t_attn / 1e12, 1),
            "attention_pct_of_f16_peak": round(100.0 * flops / t_attn / 1e12 / PEAK_F16_TFLOPS, 2)}


def cpu_baseline(M, K, N, pitch, budget_s):
    """The CPU oracle (same arithmetic, OpenMP over tokens and N blocks) on a bounded
    sample of the step: the first S tokens through prepare_norm + GEMM + epilogue."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle

    threads = oracle.max_threads()
    rng = np.random.default_rng(2100)
    w = rng.integers(-127, 128, (N, pitch), dtype=np.int8)
    ws = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
    ns = (rng.uniform(0.5, 1.5, K) - 1.0).astype(np.float32)
    z = np.zeros(K, np.float32)

    def run(rows, nt=threads):
        x = rng.standard_normal((rows, K)).astype(np.float32)
        u = x.astype(np.float16).astype(np.float32).view(np.uint32).astype(np.uint64)
        h = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        t0 = time.perf_counter()
        q, s = oracle.prepare_norm(h, ns, z, z, K, pitch, 1e-6, threads=nt)
        oracle.gemm_i8(q, w, rows, N, K, pitch, ws, s, threads=nt)
        return time.perf_counter() - t0

    rows = 64
    t = run(rows)
    # Repeat the whole step until about budget_s of CPU work has been timed (at most
    # the full 4096 tokens per repetition), and report the median repetition.
    rows = int(max(64, min(M, rows * budget_s / 5 / max(t, 1e-3))))
    reps = max(3, min(9, int(budget_s / max(run(rows), 1e-3))))
    times = sorted(run(rows) for _ in range(reps))
    t = times[len(times) // 2]
    tops = 2.0 * rows * N * K / t / 1e12
    # One thread: the same step on a sample of about a quarter of the budget.
    rows1 = 16
    t1 = run(rows1, 1)
    rows1 = int(max(16, min(M, rows1 * budget_s / 4 / max(t1, 1e-3))))
    t1 = run(rows1, 1)
    return {"value": round(tops, 5), "unit": "TOPS", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{rows} of {M} tokens through prepare_norm_i8 + gemm_i8 (K={K}, N={N}), "
                      f"median of {reps} repetitions of {t:.2f} s",
            "single_thread": {"value": round(2.0 * rows1 * N * K / t1 / 1e12, 6), "unit": "TOPS",
                              "cores": 1,
                              "sample": f"{rows1} of {M} tokens, one run of {t1:.2f} s"}}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


if __name__ == "__main__":
    main()
