"""Python host side of the MI355X W8A8 transformer-product path.

Mirrors the reference's op surface for this path (zacharydenton/krea2-hrx):
one call per kernel with the reference's positional buffer bindings
(`kernels/*.loom` ``launch(...)`` signatures), its configuration keys
(`config.decl`), its launch-shape rules (`src/kernels/shape.rs`) and its
three-way error split (`src/error.rs:11-29`). Every call goes through the C ABI
of ``libkrea2_w8a8.so`` (``include/krea2_w8a8.h``); there is no fallback.
Tensors are torch device tensors used only as memory: the kernels read and write
them through their data pointers on torch's current HIP stream.
"""

from __future__ import annotations

from . import shape  # noqa: F401  (re-exported)
from ._lib import Internal, InvalidArgument, Krea2Error, Runtime, lib, library_path  # noqa: F401
from .ops import (  # noqa: F401
    GemmConfig,
    Quantized,
    attention_f16,
    gemm_i8,
    gemm_i8_acc,
    gemm_i8_bias,
    gemm_i8_resid,
    gemm_i8_resid_256x256,
    gemm_i8_swiglu,
    gemm_choose,
    gemm_set_workspace,
    gemm_workspace_bytes,
    linear_gated_resid_i8,
    linear_norm_i8,
    linear_norm_swiglu_i8,
    linear_plain_i8,
    linear_plain_resid_i8,
    probe_mfma_i8,
    lora_transport,
    sigmoid_f32,
    prepare_gated_i8,
    prepare_norm_i8,
    prepare_plain_i8,
    rope_qknorm_f16,
    v_transpose,
)

__all__ = [
    "GemmConfig",
    "Internal",
    "InvalidArgument",
    "Krea2Error",
    "Quantized",
    "Runtime",
    "attention_f16",
    "gemm_i8",
    "gemm_i8_acc",
    "gemm_i8_bias",
    "gemm_i8_resid",
    "gemm_i8_resid_256x256",
    "gemm_i8_swiglu",
    "gemm_choose",
    "gemm_set_workspace",
    "gemm_workspace_bytes",
    "lib",
    "linear_gated_resid_i8",
    "linear_norm_i8",
    "linear_norm_swiglu_i8",
    "linear_plain_i8",
    "linear_plain_resid_i8",
    "probe_mfma_i8",
    "library_path",
    "lora_transport",
    "sigmoid_f32",
    "prepare_gated_i8",
    "prepare_norm_i8",
    "prepare_plain_i8",
    "rope_qknorm_f16",
    "v_transpose",
    "shape",
]
