"""Pins the CPU oracle of the attention step (rope_qknorm, V transpose, attention)
against the reference's own tests of these kernels, restated in f64 numpy:

  rope_qknorm  tests/quantized.rs:85-166 (check_rotary): f64 RMS norm, bf16 rounding of
               the normalised values, the rotary sum in f32, tolerance 1e-3 abs + 4e-3 rel,
               outputs bf16-representable, v copied exactly
  attention    tests/quantized.rs:313-380: f64 softmax attention over the reference's
               generators, tolerance 2e-2 abs + 2e-2 rel, at the ragged token counts the
               reference tests
  v_transpose  a permutation: numpy's transpose, columns past `rows` untouched
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle


def values(n: int, scale: float) -> np.ndarray:
    """tests/quantized.rs:80-82: ((i*37 % 101) - 50) * scale / 50 in f32."""
    i = np.arange(n, dtype=np.int64)
    return (((i * 37 % 101) - 50).astype(np.float32) * np.float32(scale)) / np.float32(50)


def f16_of(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16)


def bf16_round_f64(x: np.ndarray) -> np.ndarray:
    """Round f64 values to bf16 (nearest even) via f32: at the tolerance below a tie
    that the double rounding moves by one bf16 unit still passes."""
    b = oracle.bf16_bits(np.asarray(x, np.float64).astype(np.float32))
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def close(actual, expected, atol, rtol):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert np.all(np.isfinite(actual))
    bad = np.abs(actual - expected) > atol + rtol * np.abs(expected)
    assert not bad.any(), f"{bad.sum()} elements off, first at {np.argwhere(bad)[0]}"


def rope_case(tokens, q_heads, kv_heads, stride):
    """The inputs of tests/quantized.rs:93-105."""
    dim = 128
    inp = values(tokens * stride, 0.7)
    inp = oracle.bf16_bits(inp)  # through bf16, then to f16 as the reference does
    inp = (inp.astype(np.uint32) << 16).view(np.float32).astype(np.float16)
    qs = values(dim, 0.3)
    ks = values(dim, -0.2)
    i = np.arange(tokens * dim)
    cos = np.cos((i // 2).astype(np.float32) * np.float32(0.03)).astype(np.float32)
    sin = np.sin((i // 2).astype(np.float32) * np.float32(0.03)).astype(np.float32)
    return inp, qs, ks, cos, sin


def rope_expected(inp, scale, cos, sin, tokens, heads, offset, stride):
    """tests/quantized.rs:124-155 in numpy."""
    dim = 128
    out = []
    x = inp.astype(np.float64).reshape(tokens, stride)
    c32 = cos.reshape(tokens, dim)
    s32 = sin.reshape(tokens, dim)
    for t in range(tokens):
        for h in range(heads):
            row = x[t, offset + h * dim: offset + (h + 1) * dim]
            rms = np.sqrt((row ** 2).sum() / dim + 1e-5)
            norm = bf16_round_f64(row / rms * (1.0 + scale.astype(np.float64)))
            partner = np.empty(dim)
            partner[0::2] = -norm[1::2]
            partner[1::2] = norm[0::2]
            rot = norm.astype(np.float32) * c32[t] + partner.astype(np.float32) * s32[t]
            out.append(bf16_round_f64(rot))
    return np.concatenate(out)


@pytest.mark.parametrize("tokens,q_heads,kv_heads,stride", [(3, 9, 2, 1664), (3, 48, 12, 15360)])
def test_rope_qknorm_matches_the_reference_rotary_test(tokens, q_heads, kv_heads, stride):
    inp, qs, ks, cos, sin = rope_case(tokens, q_heads, kv_heads, stride)
    q, k, v = oracle.rope_qknorm(inp.view(np.uint16), qs, ks, cos, sin, row_stride=stride,
                                 q_heads=q_heads, kv_heads=kv_heads, k_offset=q_heads * 128,
                                 eps=1e-5)
    for got, heads, offset, scale in [(q, q_heads, 0, qs), (k, kv_heads, q_heads * 128, ks)]:
        actual = got.view(np.float16).astype(np.float64).ravel()
        assert np.array_equal(bf16_round_f64(actual), actual)  # bf16-representable
        close(actual, rope_expected(inp, scale, cos, sin, tokens, heads, offset, stride), 1e-3,
              4e-3)
    x = inp.view(np.uint16).reshape(tokens, stride)
    assert np.array_equal(v, x[:, (q_heads + kv_heads) * 128:(q_heads + 2 * kv_heads) * 128])


def test_head_sum_of_squares_is_the_head_energy():
    rng = np.random.default_rng(3)
    for scale in (1e-3, 1.0, 30.0):
        h = f16_of(rng.standard_normal(128) * scale)
        want = (h.astype(np.float64) ** 2).sum()
        assert abs(oracle.head_sum_squares(h.view(np.uint16)) - want) <= 1e-6 * want


def test_rope_rotation_is_a_rotation_of_each_pair():
    """cos = 1, sin = 0 leaves the normalised values; cos = 0, sin = 1 maps each pair
    (a, b) to (-b, a): a swapped or sign-flipped partner fails one of the two."""
    tokens, qh, kvh, stride = 2, 4, 1, 768
    rng = np.random.default_rng(5)
    inp = f16_of(rng.standard_normal(tokens * stride))
    qs = rng.uniform(-0.5, 0.5, 128).astype(np.float32)
    ks = rng.uniform(-0.5, 0.5, 128).astype(np.float32)
    one, zero = np.ones(tokens * 128, np.float32), np.zeros(tokens * 128, np.float32)
    args = dict(row_stride=stride, q_heads=qh, kv_heads=kvh, k_offset=qh * 128, eps=1e-5)
    q_id, _, _ = oracle.rope_qknorm(inp.view(np.uint16), qs, ks, one, zero, **args)
    q_rot, _, _ = oracle.rope_qknorm(inp.view(np.uint16), qs, ks, zero, one, **args)
    a = q_id.view(np.float16).reshape(tokens, qh, 64, 2)
    b = q_rot.view(np.float16).reshape(tokens, qh, 64, 2)
    assert np.array_equal(b[..., 0], -a[..., 1])
    assert np.array_equal(b[..., 1], a[..., 0])


@pytest.mark.parametrize("rows,width,capacity", [(1, 32, 32), (77, 96, 96), (130, 256, 160)])
def test_v_transpose_is_the_transpose_and_leaves_headroom(rows, width, capacity):
    rng = np.random.default_rng(rows)
    x = rng.integers(0, 65535, (rows, width), dtype=np.uint16)
    out = np.full((width, capacity), 0x1234, np.uint16)
    oracle.v_transpose(x, rows, width, capacity, out)
    assert np.array_equal(out[:, :rows], x.T)
    assert np.all(out[:, rows:] == 0x1234)


def attention_case(tokens, heads, kv, d=128):
    """tests/quantized.rs:316-324: capacity (tokens + 79) rounded up to 64; q, k, v from
    the reference's generator, zero past `tokens`."""
    capacity = (tokens + 79 + 63) // 64 * 64
    q = f16_of(values(capacity * heads * d, 0.5))
    k = f16_of(values(capacity * kv * d, 0.3))
    v = f16_of(values(capacity * kv * d, 0.7))
    q[tokens * heads * d:] = 0
    k[tokens * kv * d:] = 0
    v[tokens * kv * d:] = 0
    return capacity, q, k, v


def attention_f64(q, k, v, tokens, heads, kv, d=128, rows=None):
    """tests/quantized.rs:325-348 (query head h reads kv head h * kv / heads)."""
    rows = tokens if rows is None else rows
    qf = q.astype(np.float64)[: rows * heads * d].reshape(rows, heads, d)
    kf = k.astype(np.float64)[: tokens * kv * d].reshape(tokens, kv, d)
    vf = v.astype(np.float64)[: tokens * kv * d].reshape(tokens, kv, d)
    group = heads // kv
    out = np.empty((rows, heads, d))
    for h in range(heads):
        s = qf[:, h, :] @ kf[:, h // group, :].T / np.sqrt(d)
        s -= s.max(axis=1, keepdims=True)
        w = np.exp(s)
        out[:, h, :] = (w / w.sum(axis=1, keepdims=True)) @ vf[:, h // group, :]
    return out.reshape(rows, heads * d)


@pytest.mark.parametrize("tokens", [16, 17, 31, 32, 33, 63, 64, 65, 97])
def test_attention_matches_the_reference_softmax_test(tokens):
    heads, kv, d = 4, 1, 128
    capacity, q, k, v = attention_case(tokens, heads, kv, d)
    vt = v.reshape(capacity, kv * d).T.copy()
    want = attention_f64(q, k, v, tokens, heads, kv, d)
    for key_tile in (16, 64):
        out = oracle.attention(q.view(np.uint16), k.view(np.uint16), vt.view(np.uint16),
                               tokens=tokens, capacity=capacity, q_stride=heads * d,
                               kv_stride=kv * d, out_stride=heads * d, kv_heads=kv,
                               scale=1 / np.sqrt(d), key_tile=key_tile)
        close(out.view(np.float16), want, 2e-2, 2e-2)


@pytest.mark.parametrize("group", [1, 2, 4])
def test_attention_groups_map_query_heads_to_their_kv_head(group):
    """Random data with distinct kv heads: a wrong head mapping, a missing scale or a
    transposed V fails the f64 comparison (a tighter tolerance than the reference's
    generators allow, since these values are not near-degenerate)."""
    tokens, kv, d = 70, 2, 128
    heads = group * kv
    capacity = 160
    rng = np.random.default_rng(group)
    q = np.zeros((capacity, heads * d), np.float16)
    k = np.zeros((capacity, kv * d), np.float16)
    v = np.zeros((capacity, kv * d), np.float16)
    q[:tokens] = f16_of(rng.standard_normal((tokens, heads * d)))
    k[:tokens] = f16_of(rng.standard_normal((tokens, kv * d)))
    v[:tokens] = f16_of(rng.standard_normal((tokens, kv * d)))
    want = attention_f64(q.ravel(), k.ravel(), v.ravel(), tokens, heads, kv, d)
    out = oracle.attention(q.view(np.uint16), k.view(np.uint16), v.T.copy().view(np.uint16),
                           tokens=tokens, capacity=capacity, q_stride=heads * d,
                           kv_stride=kv * d, out_stride=heads * d, kv_heads=kv,
                           scale=1 / np.sqrt(d), group=group, key_tile=64)
    close(out.view(np.float16), want, 3e-3, 1e-2)
