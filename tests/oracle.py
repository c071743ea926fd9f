"""ctypes view of the CPU oracle (oracle/liboracle_w8a8.so) over numpy arrays.

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it, and only as the checker or the timed CPU baseline.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_LIB = os.path.join(ORACLE_DIR, "liboracle_w8a8.so")

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_LIB):
            build()
        L = ctypes.CDLL(ORACLE_LIB)
        P, I, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
        sigs = {
            "ora_bf16_from_f32": (ctypes.c_uint16, [F]),
            "ora_f16_from_f32": (ctypes.c_uint16, [F]),
            "ora_expf": (F, [F]),
            "ora_expf_n": (None, [P, P, I]),
            "ora_sigmoid_bits_n": (None, [ctypes.c_uint32, P, I]),
            "ora_f16_from_f32_n": (None, [P, P, I]),
            "ora_bf16_from_f32_n": (None, [P, P, I]),
            "ora_prepare_plain_i8": (None, [I, I, I, P, P, P, ctypes.c_int]),
            "ora_prepare_norm_i8": (None, [I, I, I, F, P, P, P, P, P, P, ctypes.c_int]),
            "ora_prepare_gated_i8": (None, [I, I, I, I, P, P, P, P, ctypes.c_int]),
            "ora_norm_sum_squares": (F, [I, P]),
            "ora_gemm_i32": (None, [I, I, I, I, P, P, P, ctypes.c_int]),
            "ora_epilogue_plain": (None, [I, I, P, P, P, P]),
            "ora_epilogue_resid": (None, [I, I, P, P, P, P, P]),
            "ora_epilogue_swiglu": (None, [I, I, P, P, P, P]),
            "ora_epilogue_bias": (None, [I, I, P, P, P, P, P]),
            "ora_gemm_i8": (None, [I, I, I, I, P, P, P, P, P, ctypes.c_int]),
            "ora_max_threads": (ctypes.c_int, []),
            "ora_rope_qknorm_f16": (None, [I, I, I, I, I, F, P, P, P, P, P, P, P, P]),
            "ora_head_sum_squares": (F, [P]),
            "ora_v_transpose": (None, [I, I, I, P, P]),
            "ora_attention_f16": (None, [I, I, I, I, I, I, I, I, F, I, P, P, P, P, ctypes.c_int]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray) -> ctypes.c_void_p:
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().ora_expf_n(_p(x), _p(y), x.size)
    return y


def sigmoid_of_bits(first: int, count: int) -> np.ndarray:
    """sigmoid of the f32 values with bit patterns first, first + 1, ... (count of them)."""
    y = np.empty(count, np.float32)
    lib().ora_sigmoid_bits_n(first, _p(y), count)
    return y


def f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().ora_f16_from_f32_n(_p(x), _p(y), x.size)
    return y


def bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().ora_bf16_from_f32_n(_p(x), _p(y), x.size)
    return y


def prepare_plain(h_f16_bits: np.ndarray, width: int, out_stride: int, q=None, threads=0):
    tokens = h_f16_bits.size // width
    h = np.ascontiguousarray(h_f16_bits, dtype=np.uint16)
    if q is None:
        q = np.zeros((tokens, out_stride), np.int8)
    s = np.zeros(tokens, np.float32)
    lib().ora_prepare_plain_i8(tokens, width, out_stride, _p(h), _p(q), _p(s), threads)
    return q, s


def prepare_norm(h_bf16_bits, norm_scale, mod_scale, mod_shift, width, out_stride, eps, q=None,
                 threads=0):
    tokens = h_bf16_bits.size // width
    h = np.ascontiguousarray(h_bf16_bits, dtype=np.uint16)
    ns = np.ascontiguousarray(norm_scale, dtype=np.float32)
    ms = np.ascontiguousarray(mod_scale, dtype=np.float32)
    sh = np.ascontiguousarray(mod_shift, dtype=np.float32)
    if q is None:
        q = np.zeros((tokens, out_stride), np.int8)
    s = np.zeros(tokens, np.float32)
    lib().ora_prepare_norm_i8(tokens, width, out_stride, eps, _p(h), _p(ns), _p(ms), _p(sh), _p(q),
                              _p(s), threads)
    return q, s


def prepare_gated(attn_f16_bits, gate_f16_bits, width, out_stride, gate_stride, q=None, threads=0):
    tokens = attn_f16_bits.size // width
    a = np.ascontiguousarray(attn_f16_bits, dtype=np.uint16)
    g = np.ascontiguousarray(gate_f16_bits, dtype=np.uint16)
    if q is None:
        q = np.zeros((tokens, out_stride), np.int8)
    s = np.zeros(tokens, np.float32)
    lib().ora_prepare_gated_i8(tokens, width, out_stride, gate_stride, _p(a), _p(g), _p(q), _p(s),
                               threads)
    return q, s


def norm_sum_squares(h_row_bf16_bits: np.ndarray) -> float:
    h = np.ascontiguousarray(h_row_bf16_bits, dtype=np.uint16)
    return float(lib().ora_norm_sum_squares(h.size, _p(h)))


def gemm_i32(a: np.ndarray, w: np.ndarray, m: int, n: int, k_size: int, k_stride: int, threads=0):
    a = np.ascontiguousarray(a, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    acc = np.empty((m, n), np.int32)
    lib().ora_gemm_i32(m, n, k_size, k_stride, _p(a), _p(w), _p(acc), threads)
    return acc


def epilogue_plain(acc, w_scale, a_scale):
    m, n = acc.shape
    out = np.empty((m, n), np.uint16)
    lib().ora_epilogue_plain(m, n, _p(acc), _p(np.ascontiguousarray(w_scale, np.float32)),
                             _p(np.ascontiguousarray(a_scale, np.float32)), _p(out))
    return out


def epilogue_resid(acc, w_scale, a_scale, gate, x_bf16_bits):
    m, n = acc.shape
    x = np.array(x_bf16_bits, dtype=np.uint16, copy=True).reshape(m, n)
    lib().ora_epilogue_resid(m, n, _p(acc), _p(np.ascontiguousarray(w_scale, np.float32)),
                             _p(np.ascontiguousarray(a_scale, np.float32)),
                             _p(np.ascontiguousarray(gate, np.float32)), _p(x))
    return x


def epilogue_swiglu(acc, w_scale, a_scale):
    m, n = acc.shape
    out = np.empty((m, n // 2), np.uint16)
    lib().ora_epilogue_swiglu(m, n, _p(acc), _p(np.ascontiguousarray(w_scale, np.float32)),
                              _p(np.ascontiguousarray(a_scale, np.float32)), _p(out))
    return out


def epilogue_bias(acc, w_scale, a_scale, bias_f16_bits):
    m, n = acc.shape
    out = np.empty((m, n), np.uint16)
    lib().ora_epilogue_bias(m, n, _p(acc), _p(np.ascontiguousarray(w_scale, np.float32)),
                            _p(np.ascontiguousarray(a_scale, np.float32)),
                            _p(np.ascontiguousarray(bias_f16_bits, np.uint16)), _p(out))
    return out


def gemm_i8(a, w, m, n, k_size, k_stride, w_scale, a_scale, threads=0):
    out = np.empty((m, n), np.uint16)
    lib().ora_gemm_i8(m, n, k_size, k_stride, _p(np.ascontiguousarray(a, np.int8)),
                      _p(np.ascontiguousarray(w, np.int8)),
                      _p(np.ascontiguousarray(w_scale, np.float32)),
                      _p(np.ascontiguousarray(a_scale, np.float32)), _p(out), threads)
    return out


def max_threads() -> int:
    return int(lib().ora_max_threads())


def rope_qknorm(qkv_f16_bits, q_scale, k_scale, cos, sin, *, row_stride, q_heads, kv_heads,
                k_offset, eps):
    """(q_out, k_out, v_out) as f16 bit patterns, [tokens][heads*128]."""
    qkv = np.ascontiguousarray(qkv_f16_bits, np.uint16)
    tokens = qkv.size // row_stride
    q_out = np.empty((tokens, q_heads * 128), np.uint16)
    k_out = np.empty((tokens, kv_heads * 128), np.uint16)
    v_out = np.empty((tokens, kv_heads * 128), np.uint16)
    lib().ora_rope_qknorm_f16(tokens, row_stride, q_heads, kv_heads, k_offset, eps, _p(qkv),
                              _p(np.ascontiguousarray(q_scale, np.float32)),
                              _p(np.ascontiguousarray(k_scale, np.float32)),
                              _p(np.ascontiguousarray(cos, np.float32)),
                              _p(np.ascontiguousarray(sin, np.float32)), _p(q_out), _p(k_out),
                              _p(v_out))
    return q_out, k_out, v_out


def head_sum_squares(h_f16_bits) -> float:
    return float(lib().ora_head_sum_squares(_p(np.ascontiguousarray(h_f16_bits, np.uint16))))


def v_transpose(x_f16_bits, rows, width, capacity, out=None):
    x = np.ascontiguousarray(x_f16_bits, np.uint16)
    if out is None:
        out = np.zeros((width, capacity), np.uint16)
    lib().ora_v_transpose(rows, width, capacity, _p(x), _p(out))
    return out


def attention(q_bits, k_bits, vt_bits, *, tokens, capacity, q_stride, kv_stride, out_stride,
              kv_heads, scale, group=4, key_tile=16, rows_out=None, threads=0):
    """f16 bit patterns [rows_out][out_stride] (columns past 4*kv_heads*128 zero)."""
    rows = tokens if rows_out is None else rows_out
    out = np.zeros((rows, out_stride), np.uint16)
    lib().ora_attention_f16(tokens, rows, capacity, q_stride, kv_stride, out_stride, kv_heads,
                            group, scale, key_tile, _p(np.ascontiguousarray(q_bits, np.uint16)),
                            _p(np.ascontiguousarray(k_bits, np.uint16)),
                            _p(np.ascontiguousarray(vt_bits, np.uint16)), _p(out), threads)
    return out
