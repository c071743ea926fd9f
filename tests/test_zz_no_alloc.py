"""The allocation-free GEMM entry point (k2w8_gemm_i8_noalloc), called through the C ABI:
bit-identical to k2w8_gemm_i8 on two calls in a row (the second smaller, both splitting
K into the static scratch) and on a shape that does not split; and no device memory
allocated by a call on a stream the library has never seen (where k2w8_gemm_i8 would
allocate its 64 MiB per-stream workspace); and eager calls on two streams at once,
which share the scratch, stay exact (the library orders them on the device)."""

import ctypes

import numpy as np
import pytest
import torch

from gpu_common import channel_scales, dev, host, int8_weights, k2
from krea2_w8a8._lib import GemmCfg, lib

pytestmark = pytest.mark.gpu


def operands(rng, m, k, n):
    return (dev(int8_weights(rng, m, k)), dev(int8_weights(rng, n, k)), dev(channel_scales(rng, n)),
            dev(rng.uniform(1e-3, 3e-2, m).astype(np.float32)))


def call(name, stream, m, k, n, ops, out):
    a, w, ws, s = ops
    cfg = GemmCfg(k, n, k, 4, 0)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    rc = getattr(lib(), name)(ctypes.c_void_p(stream.cuda_stream), ctypes.byref(cfg), m, P(a), P(w),
                              P(ws), P(s), P(out))
    assert rc == 0, lib().k2w8_last_error()


@pytest.mark.parametrize("shapes", [
    # (m, k, n): split K (config-4 down projection at 256 then 77 tokens), then a shape
    # whose tiles fill the chip (no scratch)
    [(256, 9728, 2560), (77, 9728, 2560), (1024, 3072, 4096)],
])
def test_no_alloc_gemm_equals_the_allocating_entry_point(shapes):
    rng = np.random.default_rng(71)
    stream = torch.cuda.current_stream()
    for m, k, n in shapes:
        ops = operands(rng, m, k, n)
        want = torch.zeros((m, n), dtype=torch.float16, device="cuda")
        got = torch.full((m, n), 7.0, dtype=torch.float16, device="cuda")
        call("k2w8_gemm_i8", stream, m, k, n, ops, want)
        call("k2w8_gemm_i8_noalloc", stream, m, k, n, ops, got)
        torch.cuda.synchronize()
        assert np.array_equal(host(got), host(want)), (m, k, n)


def test_no_alloc_gemm_allocates_nothing_on_a_new_stream():
    rng = np.random.default_rng(72)
    m, k, n = 256, 9728, 2560
    ops = operands(rng, m, k, n)
    want = torch.zeros((m, n), dtype=torch.float16, device="cuda")
    got = torch.zeros((m, n), dtype=torch.float16, device="cuda")
    warm = torch.cuda.current_stream()
    call("k2w8_gemm_i8_noalloc", warm, m, k, n, ops, got)  # loads the code object
    call("k2w8_gemm_i8", warm, m, k, n, ops, want)
    torch.cuda.synchronize()
    fresh = torch.cuda.Stream()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(3):
        call("k2w8_gemm_i8_noalloc", fresh, m, k, n, ops, got)
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free0 - free1 < (8 << 20), (free0, free1)  # a per-stream workspace is 64 MiB
    assert np.array_equal(host(got), host(want))


def test_no_alloc_calls_on_two_streams_at_once():
    # Two host threads enqueue split-K calls on their own streams with no ordering of
    # their own: the library makes each wait for the previous user of the scratch.
    import threading

    rng = np.random.default_rng(73)
    shapes = [(256, 9728, 2560), (200, 9728, 2560)]
    ops = [operands(rng, m, k, n) for m, k, n in shapes]
    wants = []
    for (m, k, n), o in zip(shapes, ops):
        want = torch.zeros((m, n), dtype=torch.float16, device="cuda")
        call("k2w8_gemm_i8", torch.cuda.current_stream(), m, k, n, o, want)
        wants.append(want)
    torch.cuda.synchronize()
    outs = [[torch.zeros_like(w) for _ in range(6)] for w in wants]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()  # the outputs' fills (default stream) before the workers' streams
    errors = []

    def worker(i):
        try:
            m, k, n = shapes[i]
            for o in outs[i]:
                call("k2w8_gemm_i8_noalloc", streams[i], m, k, n, ops[i], o)
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
            assert np.array_equal(host(o), host(w)), (i, j)
