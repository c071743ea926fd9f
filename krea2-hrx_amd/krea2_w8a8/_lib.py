"""Loading ``libkrea2_w8a8.so`` and declaring its C ABI for ctypes.

The library lives next to this package (``krea2-hrx_amd/libkrea2_w8a8.so``) and is
built by ``krea2-hrx_amd/Makefile``. A missing library is an error: the W8A8 path
has no CPU or PyTorch fallback.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
library_path = os.path.join(os.path.dirname(_HERE), "libkrea2_w8a8.so")

K2W8_OK = 0
K2W8_INVALID_ARGUMENT = -1
K2W8_INTERNAL = -2
K2W8_RUNTIME = -3


class Krea2Error(RuntimeError):
    """A failed W8A8 call (the reference's ``krea2::Error``)."""


class InvalidArgument(Krea2Error, ValueError):
    """The request cannot be served as asked (``Error::InvalidArgument``)."""


class Internal(Krea2Error):
    """The host broke its own contract with a kernel (``Error::Internal``)."""


class Runtime(Krea2Error):
    """The GPU runtime failed or refused the work (``Error::Runtime``)."""


class PrepareNormCfg(ctypes.Structure):
    _fields_ = [("width", ctypes.c_int64), ("out_stride", ctypes.c_int64), ("eps", ctypes.c_float)]


class PreparePlainCfg(ctypes.Structure):
    _fields_ = [("width", ctypes.c_int64), ("out_stride", ctypes.c_int64)]


class PrepareGatedCfg(ctypes.Structure):
    _fields_ = [
        ("width", ctypes.c_int64),
        ("out_stride", ctypes.c_int64),
        ("gate_stride", ctypes.c_int64),
    ]


class QuantizedCfg(ctypes.Structure):
    _fields_ = [("inputs", ctypes.c_int64), ("outputs", ctypes.c_int64), ("pitch", ctypes.c_int64)]


class RopeQknormCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ("row_stride", "q_heads", "kv_heads", "k_offset")] + [
        ("eps", ctypes.c_float)
    ]


class VTransposeCfg(ctypes.Structure):
    _fields_ = [("width", ctypes.c_int64), ("row_capacity", ctypes.c_int64)]


class AttentionCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in (
        "q_stride", "kv_stride", "out_stride", "tokens", "token_capacity")] + [
        ("scale", ctypes.c_float)
    ]


class TensorInfo(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("ndim", ctypes.c_int32),
        ("shape", ctypes.c_int64 * 8),
        ("data", ctypes.c_void_p),
        ("nbytes", ctypes.c_int64),
    ]


class SpanInfo(ctypes.Structure):
    _fields_ = [
        ("device_offset", ctypes.c_int64),
        ("device_bytes", ctypes.c_int64),
        ("rows", ctypes.c_int64),
        ("row_bytes", ctypes.c_int64),
        ("device_row_bytes", ctypes.c_int64),
        ("file_bytes", ctypes.c_int64),
        ("segments", ctypes.c_int64),
    ]


class BlockCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ("tokens", "hidden", "inter", "qkvg", "gate_offset")] + [
        ("eps", ctypes.c_float)
    ]


class BlockWeights(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "qkvg_q", "qkvg_s", "wo_q", "wo_s", "gu_q", "gu_s", "down_q", "down_s", "prenorm",
        "postnorm", "qnorm", "knorm")]


class BlockBuffers(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "x", "a_q", "a_s", "fused", "attn_gu", "mods", "q", "k", "v", "vt", "cos", "sin")]


class GemmCfg(ctypes.Structure):
    _fields_ = [
        ("k_size", ctypes.c_int64),
        ("n_size", ctypes.c_int64),
        ("k_stride", ctypes.c_int64),
        ("m_group", ctypes.c_int64),
        ("schedule_rows", ctypes.c_int64),
    ]


class GemmChoice(ctypes.Structure):
    _fields_ = [
        ("kernel", ctypes.c_int32),
        ("tile_m", ctypes.c_int32),
        ("tile_n", ctypes.c_int32),
        ("stages", ctypes.c_int32),
        ("n_big", ctypes.c_int64),
        ("split_steps", ctypes.c_int32),
        ("splits", ctypes.c_int32),
    ]


_P = ctypes.c_void_p
_I64 = ctypes.c_int64

# name -> (restype, argtypes); the exported surface of include/krea2_w8a8.h
SIGNATURES = {
    "k2w8_abi_version": (ctypes.c_int, []),
    "k2w8_last_error": (ctypes.c_char_p, []),
    "k2w8_prepare_norm_i8": (
        ctypes.c_int,
        [_P, ctypes.POINTER(PrepareNormCfg), _I64, _P, _P, _P, _P, _P, _P],
    ),
    "k2w8_prepare_plain_i8": (ctypes.c_int, [_P, ctypes.POINTER(PreparePlainCfg), _I64, _P, _P, _P]),
    "k2w8_prepare_gated_i8": (
        ctypes.c_int,
        [_P, ctypes.POINTER(PrepareGatedCfg), _I64, _P, _P, _P, _P],
    ),
    "k2w8_gemm_i8": (ctypes.c_int, [_P, ctypes.POINTER(GemmCfg), _I64, _P, _P, _P, _P, _P]),
    "k2w8_gemm_i8_resid": (ctypes.c_int, [_P, ctypes.POINTER(GemmCfg), _I64, _P, _P, _P, _P, _P, _P]),
    "k2w8_gemm_i8_resid_256x256": (
        ctypes.c_int,
        [_P, ctypes.POINTER(GemmCfg), _I64, _P, _P, _P, _P, _P, _P],
    ),
    "k2w8_gemm_i8_swiglu": (ctypes.c_int, [_P, ctypes.POINTER(GemmCfg), _I64, _P, _P, _P, _P, _P]),
    "k2w8_gemm_i8_bias": (ctypes.c_int, [_P, ctypes.POINTER(GemmCfg), _I64, _P, _P, _P, _P, _P, _P]),
    "k2w8_gemm_i8_acc": (ctypes.c_int, [_P, ctypes.POINTER(GemmCfg), _I64, _P, _P, _P]),
    "k2w8_gemm_set_workspace": (ctypes.c_int, [_P, _P, _I64]),
    "k2w8_gemm_choose": (ctypes.c_int, [ctypes.c_int32, _I64, ctypes.POINTER(GemmCfg), _I64, _I64,
                                        ctypes.c_int32, ctypes.POINTER(GemmChoice)]),
    "k2w8_linear_norm_i8": (
        ctypes.c_int,
        [_P, ctypes.POINTER(PrepareNormCfg), ctypes.POINTER(GemmCfg), _I64, _P, _P, _P, _P, _P, _P,
         _P, _P, _P],
    ),
    "k2w8_linear_plain_i8": (
        ctypes.c_int,
        [_P, ctypes.POINTER(PreparePlainCfg), ctypes.POINTER(GemmCfg), _I64, _P, _P, _P, _P, _P, _P],
    ),
    "k2w8_linear_gated_resid_i8": (
        ctypes.c_int,
        [_P, ctypes.POINTER(PrepareGatedCfg), ctypes.POINTER(GemmCfg), _I64, _P, _P, _P, _P, _P, _P, _P,
         _P],
    ),
    "k2w8_linear_norm_swiglu_i8": (
        ctypes.c_int,
        [_P, ctypes.POINTER(PrepareNormCfg), ctypes.POINTER(GemmCfg), _I64, _P, _P, _P, _P, _P, _P,
         _P, _P, _P],
    ),
    "k2w8_linear_plain_resid_i8": (
        ctypes.c_int,
        [_P, ctypes.POINTER(PreparePlainCfg), ctypes.POINTER(GemmCfg), _I64, _P, _P, _P, _P, _P, _P,
         _P],
    ),
    "k2w8_gemm_i8_noalloc": (ctypes.c_int, [_P, ctypes.POINTER(GemmCfg), _I64, _P, _P, _P, _P, _P]),
    "k2w8_gemm_workspace_bytes": (_I64, []),
    "k2w8_lora_transport": (ctypes.c_int, [_P, ctypes.c_int, _I64, _P, _P]),
    "k2w8_sigmoid_f32": (ctypes.c_int, [_P, _I64, _P, _P]),
    "k2w8_quantized_forward": (
        ctypes.c_int,
        [_P, ctypes.POINTER(QuantizedCfg), _I64, _P, _P, _P, _P, _P, _P, _P, _P],
    ),
    "k2w8_rope_qknorm_f16": (
        ctypes.c_int, [_P, ctypes.POINTER(RopeQknormCfg), _I64, _P, _P, _P, _P, _P, _P, _P, _P]),
    "k2w8_v_transpose": (ctypes.c_int, [_P, ctypes.POINTER(VTransposeCfg), _I64, _P, _P]),
    "k2w8_attention_f16": (
        ctypes.c_int, [_P, ctypes.POINTER(AttentionCfg), _I64, _I64, _P, _P, _P, _P]),
    "k2w8_attention_f16_grouped": (
        ctypes.c_int, [_P, ctypes.POINTER(AttentionCfg), _I64, _I64, _I64, _P, _P, _P, _P]),
    "k2w8_checkpoint_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]),
    "k2w8_checkpoint_close": (None, [_P]),
    "k2w8_checkpoint_block_count": (_I64, [_P]),
    "k2w8_checkpoint_tensor": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(TensorInfo)]),
    "k2w8_plan_for_checkpoint": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_void_p)]),
    "k2w8_plan_free": (None, [_P]),
    "k2w8_plan_total_bytes": (_I64, [_P]),
    "k2w8_plan_layers": (_I64, [_P]),
    "k2w8_plan_span_count": (_I64, [_P]),
    "k2w8_plan_span_name": (ctypes.c_char_p, [_P, _I64]),
    "k2w8_plan_span": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(SpanInfo)]),
    "k2w8_plan_upload": (ctypes.c_int, [_P, _P, _P, _P, _I64]),
    "k2w8_block_pre_attention": (
        ctypes.c_int, [_P, ctypes.POINTER(BlockCfg), _I64, ctypes.POINTER(BlockWeights),
                       ctypes.POINTER(BlockBuffers)]),
    "k2w8_block_attention": (
        ctypes.c_int, [_P, ctypes.POINTER(BlockCfg), _I64, ctypes.POINTER(BlockWeights),
                       ctypes.POINTER(BlockBuffers)]),
    "k2w8_block_post_attention": (
        ctypes.c_int, [_P, ctypes.POINTER(BlockCfg), _I64, ctypes.POINTER(BlockWeights),
                       ctypes.POINTER(BlockBuffers)]),
    "k2w8_blocks_record": (
        ctypes.c_int, [_P, ctypes.POINTER(BlockCfg), _I64, ctypes.POINTER(BlockWeights),
                       ctypes.POINTER(BlockBuffers), ctypes.POINTER(ctypes.c_void_p)]),
    "k2w8_graph_launch": (ctypes.c_int, [_P, _P]),
    "k2w8_graph_free": (None, [_P]),
    "k2w8_blocks_profile": (
        ctypes.c_int, [_P, ctypes.POINTER(BlockCfg), _I64, ctypes.POINTER(BlockWeights),
                       ctypes.POINTER(BlockBuffers), ctypes.POINTER(ctypes.c_double), _I64]),
    "k2w8_block_stage_count": (_I64, []),
    "k2w8_block_stage_label": (ctypes.c_char_p, [_I64]),
    "k2w8_shape_gemm_pitch": (_I64, [_I64]),
    "k2w8_shape_capacity": (_I64, [_I64]),
    "k2w8_shape_gemm_grid_rows": (_I64, [_I64]),
    "k2w8_shape_gemm_schedule_rows": (ctypes.c_int, [_I64]),
    "k2w8_probe_mfma_i8": (ctypes.c_int, [_P, _I64, _I64, ctypes.c_int32, ctypes.c_uint32, _P]),
    "k2w8_validate_gemm_cfg": (ctypes.c_int, [ctypes.POINTER(GemmCfg)]),
    "k2w8_validate_prepare_norm_cfg": (ctypes.c_int, [ctypes.POINTER(PrepareNormCfg)]),
    "k2w8_validate_prepare_plain_cfg": (ctypes.c_int, [ctypes.POINTER(PreparePlainCfg)]),
    "k2w8_validate_prepare_gated_cfg": (ctypes.c_int, [ctypes.POINTER(PrepareGatedCfg)]),
    "k2w8_shape_gemm_rows": (_I64, []),
    "k2w8_shape_gemm_m_group": (_I64, []),
    "k2w8_shape_tokens_min": (_I64, []),
    "k2w8_shape_tokens_max": (_I64, []),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library (loaded once). Raises ``Runtime`` if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(library_path):
            raise Runtime(
                f"{library_path} is not built; run `make -C krea2-hrx_amd` "
                "(or __graft_entry__.build())"
            )
        # torch first: the HIP runtime it loads is the one this library binds to.
        import torch  # noqa: F401

        handle = ctypes.CDLL(library_path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(code: int) -> None:
    """Raise the error class matching a C ABI return code."""
    if code == K2W8_OK:
        return
    message = lib().k2w8_last_error().decode(errors="replace")
    if code == K2W8_INVALID_ARGUMENT:
        raise InvalidArgument(message)
    if code == K2W8_INTERNAL:
        raise Internal(message)
    raise Runtime(message)
