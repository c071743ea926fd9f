"""The C ABI library on the CPU: it loads, exports what include/krea2_w8a8.h declares,
implements the reference's shape rules, and rejects bad arguments before any GPU work
(the reference's host-side rejections, tests/constructor.rs style)."""

import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "krea2_w8a8.h")
LIBDIR = os.path.join(ROOT, "krea2-hrx_amd")


@pytest.fixture(scope="module")
def k2():
    if not os.path.exists(os.path.join(LIBDIR, "libkrea2_w8a8.so")):
        subprocess.run(["make", "-s", "-C", LIBDIR], check=True)
    import krea2_w8a8

    return krea2_w8a8


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(k2w8_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_entry_point_is_exported_and_bound(k2):
    lib = k2.lib()
    names = declared_symbols()
    assert len(names) >= 17
    for name in names:
        assert hasattr(lib, name), name
        assert name in k2._lib.SIGNATURES, name
    assert lib.k2w8_abi_version() == 1


def test_shape_rules_are_the_reference_rules(k2):
    # src/kernels/shape.rs:114-149
    s = k2.shape
    assert [s.gemm_pitch(6144), s.gemm_pitch(16384)] == [6144, 16448]
    assert [s.gemm_pitch(3072), s.gemm_pitch(12288), s.gemm_pitch(8192)] == [3072, 12288, 8256]
    assert [s.capacity(4115), s.capacity(16), s.capacity(2048)] == [4160, 64, 2080]
    assert [s.gemm_grid_rows(4115), s.gemm_grid_rows(256), s.gemm_grid_rows(16)] == [17, 1, 1]
    assert [s.gemm_schedule_rows(t) for t in (16, 4095, 4096, 16896)] == [False, False, True, True]
    assert s.gemm_rows() == 256 and s.gemm_m_group() == 4
    r = s.tokens_range()
    assert (r.start, r.stop - 1) == (16, 16896)
    for tokens in (16, 4115, 9000, 16896):
        assert s.capacity(tokens) >= tokens + 16


FAKE = ctypes.c_void_p(0x10000)  # aligned, never dereferenced: every call below fails validation


def call_gemm(k2, **over):
    cfg = dict(k_size=3072, n_size=3072, k_stride=3072, m_group=4, schedule_rows=0)
    m = over.pop("m", 64)
    ptrs = over.pop("ptrs", [FAKE] * 5)
    cfg.update(over)
    c = k2._lib.GemmCfg(**cfg)
    return k2.lib().k2w8_gemm_i8(None, ctypes.byref(c), m, *ptrs)


@pytest.mark.parametrize("over,fragment", [
    (dict(k_size=3000), "k_size"),
    (dict(k_size=0), "k_size"),
    (dict(n_size=100), "n_size"),
    (dict(n_size=65536), "n_size"),
    (dict(k_stride=3000), "k_stride"),
    (dict(k_stride=2048), "k_stride"),
    (dict(m_group=0), "m_group"),
    (dict(m_group=5), "m_group"),
    (dict(m=0), "m must be"),
    (dict(ptrs=[FAKE, None, FAKE, FAKE, FAKE]), "null"),
    (dict(ptrs=[ctypes.c_void_p(0x10008), FAKE, FAKE, FAKE, FAKE]), "aligned"),
])
def test_gemm_rejects_what_the_reference_config_rejects(k2, over, fragment):
    rc = call_gemm(k2, **over)
    assert rc == k2._lib.K2W8_INVALID_ARGUMENT
    assert fragment in k2.lib().k2w8_last_error().decode()


def test_gemm_rejects_a_null_configuration(k2):
    rc = k2.lib().k2w8_gemm_i8(None, None, 1, FAKE, FAKE, FAKE, FAKE, FAKE)
    assert rc == k2._lib.K2W8_INVALID_ARGUMENT
    with pytest.raises(k2.InvalidArgument, match="null configuration"):
        k2._lib.check(rc)


def test_resid_and_bias_require_their_extra_operand(k2):
    c = k2._lib.GemmCfg(3072, 3072, 3072, 4, 0)
    rc = k2.lib().k2w8_gemm_i8_resid(None, ctypes.byref(c), 64, FAKE, FAKE, FAKE, FAKE, FAKE, None)
    assert rc == k2._lib.K2W8_INVALID_ARGUMENT and "gate" in k2.lib().k2w8_last_error().decode()
    rc = k2.lib().k2w8_gemm_i8_bias(None, ctypes.byref(c), 64, FAKE, FAKE, FAKE, FAKE, None, FAKE)
    assert rc == k2._lib.K2W8_INVALID_ARGUMENT and "bias" in k2.lib().k2w8_last_error().decode()


@pytest.mark.parametrize("width,out_stride,tokens,fragment", [
    (3000, 3072, 4, "width"),
    (128, 128, 4, "width"),
    (65536, 65536, 4, "width"),
    (3072, 3000, 4, "out_stride"),
    (3072, 2048, 4, "out_stride"),
    (3072, 3072, 0, "tokens"),
    (3072, 3072, (1 << 20) + 1, "tokens"),
])
def test_prepares_reject_what_the_reference_config_rejects(k2, width, out_stride, tokens, fragment):
    L = k2.lib()
    plain = k2._lib.PreparePlainCfg(width, out_stride)
    assert L.k2w8_prepare_plain_i8(None, ctypes.byref(plain), tokens, FAKE, FAKE, FAKE) == -1
    assert fragment in L.k2w8_last_error().decode()
    norm = k2._lib.PrepareNormCfg(width, out_stride, 1e-6)
    assert L.k2w8_prepare_norm_i8(None, ctypes.byref(norm), tokens, FAKE, FAKE, FAKE, FAKE, FAKE,
                                  FAKE) == -1
    gated = k2._lib.PrepareGatedCfg(width, out_stride, max(width, 256))
    assert L.k2w8_prepare_gated_i8(None, ctypes.byref(gated), tokens, FAKE, FAKE, FAKE, FAKE) == -1


def test_gated_prepare_rejects_a_short_gate_pitch(k2):
    L = k2.lib()
    gated = k2._lib.PrepareGatedCfg(3072, 3072, 2048)
    assert L.k2w8_prepare_gated_i8(None, ctypes.byref(gated), 4, FAKE, FAKE, FAKE, FAKE) == -1
    assert "gate_stride" in L.k2w8_last_error().decode()


def test_error_classes_keep_the_reference_split(k2):
    assert issubclass(k2.InvalidArgument, k2.Krea2Error)
    assert issubclass(k2.Runtime, k2.Krea2Error)
    assert not issubclass(k2.Internal, k2.InvalidArgument)


def test_transport_rejects_a_bad_direction_count_or_alignment(k2):
    lib = k2.lib()
    odd = ctypes.c_void_p(0x10008)
    cases = [(0, 16, FAKE, FAKE, "direction"), (3, 16, FAKE, FAKE, "direction"),
             (1, 0, FAKE, FAKE, "count"), (2, 1 << 30, FAKE, FAKE, "count"),
             (1, 16, odd, FAKE, "aligned"), (1, 16, FAKE, None, "null")]
    for direction, count, x, out, fragment in cases:
        rc = lib.k2w8_lora_transport(None, direction, count, x, out)
        assert rc == -1, (direction, count)
        assert fragment in lib.k2w8_last_error().decode()


def test_quantized_forward_validates_before_any_launch(k2):
    lib = k2.lib()
    cfg = k2._lib.QuantizedCfg(6144, 128, 6144)
    args = [FAKE] * 8
    assert lib.k2w8_quantized_forward(None, None, 3, *args) == -1
    assert lib.k2w8_quantized_forward(None, ctypes.byref(cfg), 0, *args) == -1
    bad = k2._lib.QuantizedCfg(6000, 128, 6144)  # inputs not a multiple of 256
    # the transport of x runs first on a stream; FAKE buffers would be dereferenced, so
    # this case only checks the shape rejection of a zero-row call and a null cfg above
    assert lib.k2w8_quantized_forward(None, ctypes.byref(bad), 1 << 30, *args) == -1
    assert "2^30" in lib.k2w8_last_error().decode()
