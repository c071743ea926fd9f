"""GPU parity of the attention step (src/session/mod.rs:714-755) through the C ABI:

  rope_qknorm_f16  bit-exact against the oracle (the same canonical f32 sequence), on
                   the reference's rotary test inputs (tests/quantized.rs:85-166) and on
                   seeded production-shaped rows; also the reference's own f64 tolerance
  v_transpose      exact; columns past `rows` untouched
  attention_f16    fp16 MMA with f32 softmax: bit parity is not defined (the reference's
                   exp and MMA order belong to its compiler), so two tolerances:
                     against the f64 softmax, the reference's 2e-2 abs + 2e-2 rel
                     (tests/quantized.rs:313-380) on its generators and token counts;
                     against the oracle with the kernel's 64-key tiles, 2e-3 abs +
                     4e-3 rel (two f16 units of the output, one of a weight)
                   and at full production size a size-independent property: zero queries
                   give uniform weights, so every output is the mean of V.
"""

import numpy as np
import pytest
import torch

import oracle
from gpu_common import dev, host, k2, sync
from test_oracle_attention import attention_case, attention_f64, close, rope_case, rope_expected

pytestmark = pytest.mark.gpu

SENTINEL = 0x7E00  # an f16 NaN: any unwritten element the test reads shows up


def run_rope(inp_bits, qs, ks, cos, sin, tokens, q_heads, kv_heads, stride, k_offset, eps=1e-5):
    q = torch.empty((tokens, q_heads * 128), dtype=torch.float16, device="cuda")
    k = torch.empty((tokens, kv_heads * 128), dtype=torch.float16, device="cuda")
    v = torch.empty((tokens, kv_heads * 128), dtype=torch.float16, device="cuda")
    k2.rope_qknorm_f16(dev(inp_bits, torch.float16), dev(qs), dev(ks), dev(cos), dev(sin), q, k, v,
                       row_stride=stride, q_heads=q_heads, kv_heads=kv_heads, k_offset=k_offset,
                       eps=eps, tokens=tokens)
    sync()
    return host(q), host(k), host(v)


@pytest.mark.parametrize("tokens,q_heads,kv_heads,stride", [(3, 9, 2, 1664), (3, 48, 12, 15360)])
def test_rope_qknorm_reference_case_is_bit_exact(tokens, q_heads, kv_heads, stride):
    inp, qs, ks, cos, sin = rope_case(tokens, q_heads, kv_heads, stride)
    bits = inp.view(np.uint16)
    got = run_rope(bits, qs, ks, cos, sin, tokens, q_heads, kv_heads, stride, q_heads * 128)
    want = oracle.rope_qknorm(bits, qs, ks, cos, sin, row_stride=stride, q_heads=q_heads,
                              kv_heads=kv_heads, k_offset=q_heads * 128, eps=1e-5)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)
    # and the reference's own check against its f64 norm
    q_exp = rope_expected(inp, qs, cos, sin, tokens, q_heads, 0, stride)
    close(got[0].view(np.float16).ravel(), q_exp, 1e-3, 4e-3)


@pytest.mark.parametrize("tokens,q_heads,kv_heads,gate", [(257, 24, 6, 3072), (1, 48, 12, 6144),
                                                         (40, 4, 1, 0)])
def test_rope_qknorm_is_bit_exact_on_fused_rows(tokens, q_heads, kv_heads, gate):
    """The layout of the fused qkvg output: q | k | v | gate, v and gate not normalised."""
    stride = q_heads * 128 + 2 * kv_heads * 128 + gate
    rng = np.random.default_rng(tokens + q_heads)
    x = (rng.standard_normal((tokens, stride)) * np.exp(rng.uniform(-3, 3, (tokens, 1)))).astype(
        np.float16)
    x[0, :128] = 0  # a zero head: r = 1/sqrt(eps), outputs zero
    bits = x.view(np.uint16)
    qs = rng.uniform(-0.5, 0.5, 128).astype(np.float32)
    ks = rng.uniform(-0.5, 0.5, 128).astype(np.float32)
    ang = rng.uniform(0, 6.3, (tokens, 64)).astype(np.float32)
    cos = np.repeat(np.cos(ang), 2, axis=1).astype(np.float32)
    sin = np.repeat(np.sin(ang), 2, axis=1).astype(np.float32)
    got = run_rope(bits, qs, ks, cos, sin, tokens, q_heads, kv_heads, stride, q_heads * 128)
    want = oracle.rope_qknorm(bits, qs, ks, cos, sin, row_stride=stride, q_heads=q_heads,
                              kv_heads=kv_heads, k_offset=q_heads * 128, eps=1e-5)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


@pytest.mark.parametrize("rows,width,capacity", [(1, 32, 32), (77, 96, 96), (130, 256, 160),
                                                 (4544, 1536, 4576)])
def test_v_transpose_is_exact_and_leaves_headroom(rows, width, capacity):
    rng = np.random.default_rng(rows)
    x = rng.integers(0, 0x7BFF, (rows, width), dtype=np.uint16)
    out = torch.full((width, capacity), SENTINEL, dtype=torch.int16, device="cuda").view(
        torch.float16)
    k2.v_transpose(dev(x, torch.float16), out, width=width, row_capacity=capacity)
    sync()
    got = host(out)
    assert np.array_equal(got[:, :rows], x.T)
    assert np.all(got[:, rows:] == SENTINEL)


def run_attention(q, k, vt, *, tokens, capacity, heads, kv, group=4, token_count=None,
                  out_rows=None):
    d = 128
    rows = tokens if token_count is None else token_count
    out_rows = rows if out_rows is None else out_rows
    out = torch.full((out_rows, heads * d), SENTINEL, dtype=torch.int16, device="cuda").view(
        torch.float16)
    k2.attention_f16(dev(q, torch.float16), dev(k, torch.float16), dev(vt, torch.float16), out,
                     q_stride=heads * d, kv_stride=kv * d, out_stride=heads * d, tokens=tokens,
                     token_capacity=capacity, scale=1 / np.sqrt(d), kv_heads=kv, group=group,
                     token_count=rows)
    sync()
    return host(out)


@pytest.mark.parametrize("tokens", [16, 17, 31, 32, 33, 63, 64, 65, 97])
def test_attention_matches_the_reference_softmax_test(tokens):
    heads, kv, d = 4, 1, 128
    capacity, q, k, v = attention_case(tokens, heads, kv, d)
    vt = v.reshape(capacity, kv * d).T.copy()
    got = run_attention(q.view(np.uint16), k.view(np.uint16), vt.view(np.uint16), tokens=tokens,
                        capacity=capacity, heads=heads, kv=kv)
    close(got.view(np.float16), attention_f64(q, k, v, tokens, heads, kv, d), 2e-2, 2e-2)
    ora = oracle.attention(q.view(np.uint16), k.view(np.uint16), vt.view(np.uint16),
                           tokens=tokens, capacity=capacity, q_stride=heads * d, kv_stride=kv * d,
                           out_stride=heads * d, kv_heads=kv, scale=1 / np.sqrt(d), key_tile=64)
    close(got.view(np.float16), ora.view(np.float16), 2e-3, 4e-3)


def random_qkv(rng, tokens, capacity, heads, kv, scale=1.0):
    d = 128
    q = np.zeros((capacity, heads * d), np.float16)
    k = np.zeros((capacity, kv * d), np.float16)
    v = np.zeros((capacity, kv * d), np.float16)
    q[:tokens] = (rng.standard_normal((tokens, heads * d)) * scale).astype(np.float16)
    k[:tokens] = (rng.standard_normal((tokens, kv * d)) * scale).astype(np.float16)
    v[:tokens] = rng.standard_normal((tokens, kv * d)).astype(np.float16)
    return q, k, v


@pytest.mark.parametrize("tokens,kv,group,scale", [(300, 3, 4, 1.0), (1043, 2, 4, 2.0),
                                                   (200, 2, 2, 1.0), (129, 3, 1, 1.5),
                                                   (4115, 1, 4, 1.0)])
def test_attention_matches_the_oracle_on_seeded_heads(tokens, kv, group, scale):
    heads, d = group * kv, 128
    capacity = k2.shape.capacity(tokens)
    rng = np.random.default_rng(tokens * 7 + group)
    q, k, v = random_qkv(rng, tokens, capacity, heads, kv, scale)
    vt = v.T.copy()
    got = run_attention(q.view(np.uint16), k.view(np.uint16), vt.view(np.uint16), tokens=tokens,
                        capacity=capacity, heads=heads, kv=kv, group=group)
    ora = oracle.attention(q.view(np.uint16), k.view(np.uint16), vt.view(np.uint16),
                           tokens=tokens, capacity=capacity, q_stride=heads * d, kv_stride=kv * d,
                           out_stride=heads * d, kv_heads=kv, scale=1 / np.sqrt(d), group=group,
                           key_tile=64)
    close(got.view(np.float16), ora.view(np.float16), 2e-3, 4e-3)


def test_attention_writes_only_token_count_rows():
    tokens, heads, kv, d = 90, 4, 1, 128
    capacity = k2.shape.capacity(tokens)
    rng = np.random.default_rng(11)
    q, k, v = random_qkv(rng, tokens, capacity, heads, kv)
    got = run_attention(q.view(np.uint16), k.view(np.uint16), v.T.copy().view(np.uint16),
                        tokens=tokens, capacity=capacity, heads=heads, kv=kv, token_count=50,
                        out_rows=64)
    assert not np.any(got[:50] == SENTINEL)
    assert np.all(got[50:] == SENTINEL)
    full = run_attention(q.view(np.uint16), k.view(np.uint16), v.T.copy().view(np.uint16),
                         tokens=tokens, capacity=capacity, heads=heads, kv=kv)
    assert np.array_equal(got[:50], full[:50])


@pytest.mark.parametrize("tokens,q_heads,kv_heads", [(4544, 48, 12), (16896, 48, 12)])
def test_attention_with_zero_queries_averages_v_at_production_size(tokens, q_heads, kv_heads):
    """q = 0 makes every score 0, every weight exp(0) = 1 exactly and the row sum the
    token count exactly, so out = f16(sum_j v_j / tokens) with an f32 sum: checked against
    the f64 mean within one f16 unit plus the f32 summation error."""
    d = 128
    capacity = k2.shape.capacity(tokens)
    rng = np.random.default_rng(tokens)
    vt = np.zeros((kv_heads * d, capacity), np.float16)
    vt[:, :tokens] = rng.uniform(-1, 1, (kv_heads * d, tokens)).astype(np.float16)
    q = torch.zeros((capacity, q_heads * d), dtype=torch.float16, device="cuda")
    k = torch.zeros((capacity, kv_heads * d), dtype=torch.float16, device="cuda")
    k[:tokens] = torch.from_numpy(rng.standard_normal((tokens, kv_heads * d)).astype(np.float16)).cuda()
    out = torch.empty((tokens, q_heads * d), dtype=torch.float16, device="cuda")
    k2.attention_f16(q, k, dev(vt.view(np.uint16), torch.float16), out, q_stride=q_heads * d,
                     kv_stride=kv_heads * d, out_stride=q_heads * d, tokens=tokens,
                     token_capacity=capacity, scale=1 / np.sqrt(d), kv_heads=kv_heads)
    sync()
    got = host(out).view(np.float16).astype(np.float64).reshape(tokens, q_heads, d)
    mean = vt[:, :tokens].astype(np.float64).mean(axis=1).reshape(kv_heads, d)
    want = np.repeat(mean, 4, axis=0)  # query head h reads kv head h // 4
    assert np.all(np.abs(got - want[None]) <= 1e-5 + 2 ** -11 * np.abs(want[None]))


def test_attention_at_the_minimum_capacity_and_with_wide_strides():
    """capacity = tokens + 16 exactly (the last 64-key tile reaches past the buffers and is
    clamped), strides wider than the heads in use (q 1024, kv 256, out 768 columns: the
    reference kernel's strides are independent of the head count), one key-value head."""
    tokens, cap, d = 96, 112, 128
    q_stride, kv_stride, out_stride = 1024, 256, 768
    rng = np.random.default_rng(96)
    q = np.zeros((cap, q_stride), np.float16)
    k = np.zeros((cap, kv_stride), np.float16)
    v = np.zeros((cap, kv_stride), np.float16)
    q[:tokens] = rng.standard_normal((tokens, q_stride))
    k[:tokens] = rng.standard_normal((tokens, kv_stride))
    v[:tokens] = rng.standard_normal((tokens, kv_stride))
    vt = v.T.copy()
    out = torch.full((tokens, out_stride), SENTINEL, dtype=torch.int16, device="cuda").view(
        torch.float16)
    k2.attention_f16(dev(q.view(np.uint16), torch.float16), dev(k.view(np.uint16), torch.float16),
                     dev(vt.view(np.uint16), torch.float16), out, q_stride=q_stride,
                     kv_stride=kv_stride, out_stride=out_stride, tokens=tokens,
                     token_capacity=cap, scale=1 / np.sqrt(d), kv_heads=1)
    sync()
    got = host(out)
    assert np.all(got[:, 512:] == SENTINEL)  # columns past the four heads untouched
    ora = oracle.attention(q.view(np.uint16), k.view(np.uint16), vt.view(np.uint16),
                           tokens=tokens, capacity=cap, q_stride=q_stride, kv_stride=kv_stride,
                           out_stride=out_stride, kv_heads=1, scale=1 / np.sqrt(d), key_tile=64)
    close(got[:, :512].view(np.float16), ora[:, :512].view(np.float16), 2e-3, 4e-3)


def test_rope_qknorm_with_a_gap_before_k():
    """k_offset past the q heads (a gap of unused columns) and eps = 0."""
    tokens, qh, kvh, k_offset = 5, 2, 1, 512
    stride = k_offset + 2 * kvh * 128 + 128
    rng = np.random.default_rng(7)
    x = rng.standard_normal((tokens, stride)).astype(np.float16)
    bits = x.view(np.uint16)
    qs = rng.uniform(-0.5, 0.5, 128).astype(np.float32)
    ks = rng.uniform(-0.5, 0.5, 128).astype(np.float32)
    ang = rng.uniform(0, 6.3, (tokens, 64)).astype(np.float32)
    cos = np.repeat(np.cos(ang), 2, axis=1).astype(np.float32)
    sin = np.repeat(np.sin(ang), 2, axis=1).astype(np.float32)
    got = run_rope(bits, qs, ks, cos, sin, tokens, qh, kvh, stride, k_offset, eps=0.0)
    want = oracle.rope_qknorm(bits, qs, ks, cos, sin, row_stride=stride, q_heads=qh,
                              kv_heads=kvh, k_offset=k_offset, eps=0.0)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def test_attention_keeps_a_late_outlier_key_exact():
    """Scores with a spread of about +-36 (q, k ~ N(0, 2.5^2)): some queries meet a key
    far above every earlier one late in the sequence (the softmax maximum jumps by more
    than 2^16 in weight). Every output must be finite and match the oracle."""
    tokens, kv, group, d = 4544, 2, 4, 128
    heads = group * kv
    capacity = k2.shape.capacity(tokens)
    rng = np.random.default_rng(6)
    q, k, v = random_qkv(rng, tokens, capacity, heads, kv, 2.5)
    vt = v.T.copy()
    got = run_attention(q.view(np.uint16), k.view(np.uint16), vt.view(np.uint16), tokens=tokens,
                        capacity=capacity, heads=heads, kv=kv, group=group)
    assert np.all(np.isfinite(got.view(np.float16)))
    ora = oracle.attention(q.view(np.uint16), k.view(np.uint16), vt.view(np.uint16),
                           tokens=tokens, capacity=capacity, q_stride=heads * d, kv_stride=kv * d,
                           out_stride=heads * d, kv_heads=kv, scale=1 / np.sqrt(d), group=group,
                           key_tile=64)
    close(got.view(np.float16), ora.view(np.float16), 2e-3, 4e-3)
