"""One call per reference kernel, with the reference's bindings and configuration.

Binding order follows the Loom ``launch(...)`` signatures:
  prepare_norm(h, norm_scale, mod_scale, mod_shift, q, q_scale)   kernels/prepare_norm_i8.loom:22
  prepare_plain(h, q, q_scale)                                    kernels/prepare_plain_i8.loom:19
  prepare_gated(attn, gate, q, q_scale)                           kernels/prepare_gated_i8.loom:22
  gemm_i8*(a, w, scale, a_scale, c[, gate])                       kernels/gemm_i8_256.loom:36,
                                                                  kernels/gemm_i8_resid_256.loom:36
  rope_qknorm(qkv, q_scale, k_scale, cos, sin, q_out, k_out, v_out) kernels/rope_qknorm_f16.loom:24
  v_transpose(x, out)                                             kernels/native/v_transpose.loom:21
  attention(q, k, v, out)                                         kernels/attention_gqa_lds_f16_wmma.loom:35
Configuration keys are the ``config.decl`` names. The runtime scalar (``tokens``
or ``m``) defaults to the leading dimension of the first operand.

Buffer extents are checked here, before the C ABI, because the ABI takes plain
pointers; a short buffer is an ``InvalidArgument``, as in the reference.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from ._lib import (
    AttentionCfg,
    GemmCfg,
    GemmChoice,
    InvalidArgument,
    PrepareGatedCfg,
    PrepareNormCfg,
    PreparePlainCfg,
    QuantizedCfg,
    RopeQknormCfg,
    VTransposeCfg,
    check,
    lib,
)


def _stream(stream) -> ctypes.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _buf(t: torch.Tensor, name: str, dtype, min_elems: int) -> ctypes.c_void_p:
    if not isinstance(t, torch.Tensor):
        raise InvalidArgument(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise InvalidArgument(f"{name} must be device memory, got {t.device}")
    if dtype is not None and t.dtype != dtype:
        raise InvalidArgument(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise InvalidArgument(f"{name} must be contiguous")
    if t.numel() < min_elems:
        raise InvalidArgument(f"{name} holds {t.numel()} elements, needs {min_elems}")
    return ctypes.c_void_p(t.data_ptr())


def _tokens(t: torch.Tensor, tokens):
    return int(t.shape[0]) if tokens is None else int(tokens)


def prepare_norm_i8(h, norm_scale, mod_scale, mod_shift, q, q_scale, *, width, out_stride, eps,
                    tokens=None, stream=None):
    """Modulated RMSNorm, Hadamard rotation and per-token int8 quantisation.

    ``h`` bf16 [tokens][width]; ``norm_scale``/``mod_scale``/``mod_shift`` f32 [width];
    ``q`` int8 [tokens][out_stride]; ``q_scale`` f32 [tokens].
    """
    n = _tokens(h, tokens)
    cfg = PrepareNormCfg(width, out_stride, eps)
    args = (
        _buf(h, "h", torch.bfloat16, n * width),
        _buf(norm_scale, "norm_scale", torch.float32, width),
        _buf(mod_scale, "mod_scale", torch.float32, width),
        _buf(mod_shift, "mod_shift", torch.float32, width),
        _buf(q, "q", torch.int8, (n - 1) * out_stride + width),
        _buf(q_scale, "q_scale", torch.float32, n),
    )
    check(lib().k2w8_prepare_norm_i8(_stream(stream), ctypes.byref(cfg), n, *args))


def prepare_plain_i8(h, q, q_scale, *, width, out_stride, tokens=None, stream=None):
    """Hadamard rotation (f16 stages) and per-token int8 quantisation of f16 rows."""
    n = _tokens(h, tokens)
    cfg = PreparePlainCfg(width, out_stride)
    args = (
        _buf(h, "h", torch.float16, n * width),
        _buf(q, "q", torch.int8, (n - 1) * out_stride + width),
        _buf(q_scale, "q_scale", torch.float32, n),
    )
    check(lib().k2w8_prepare_plain_i8(_stream(stream), ctypes.byref(cfg), n, *args))


def prepare_gated_i8(attn, gate, q, q_scale, *, width, out_stride, gate_stride, tokens=None,
                     stream=None):
    """attn x sigmoid(gate) (bf16 rounding points), rotation, per-token int8 quantisation."""
    n = _tokens(attn, tokens)
    cfg = PrepareGatedCfg(width, out_stride, gate_stride)
    args = (
        _buf(attn, "attn", torch.float16, n * width),
        _buf(gate, "gate", torch.float16, (n - 1) * gate_stride + width),
        _buf(q, "q", torch.int8, (n - 1) * out_stride + width),
        _buf(q_scale, "q_scale", torch.float32, n),
    )
    check(lib().k2w8_prepare_gated_i8(_stream(stream), ctypes.byref(cfg), n, *args))


@dataclass(frozen=True)
class GemmConfig:
    """The GEMM family's ``config.decl`` set (kernels/gemm_i8_256.loom:14-22)."""

    k_size: int
    n_size: int
    k_stride: int
    m_group: int = 4
    schedule_rows: int = 0

    def c(self) -> GemmCfg:
        return GemmCfg(self.k_size, self.n_size, self.k_stride, self.m_group, self.schedule_rows)


def _gemm_operands(cfg: GemmConfig, m: int, a, w, scale, a_scale):
    return (
        _buf(a, "a", torch.int8, (m - 1) * cfg.k_stride + cfg.k_size),
        _buf(w, "w", torch.int8, (cfg.n_size - 1) * cfg.k_stride + cfg.k_size),
        _buf(scale, "scale", torch.float32, cfg.n_size),
        _buf(a_scale, "a_scale", torch.float32, m),
    )


def gemm_i8(a, w, scale, a_scale, c, *, cfg: GemmConfig, m=None, stream=None):
    """c f16 [m][n] = f16(bf16((f32(a.w^T) * scale[n]) * a_scale[m]))."""
    m = _tokens(a, m)
    ops = _gemm_operands(cfg, m, a, w, scale, a_scale)
    out = _buf(c, "c", torch.float16, m * cfg.n_size)
    k = cfg.c()
    check(lib().k2w8_gemm_i8(_stream(stream), ctypes.byref(k), m, *ops, out))


def gemm_i8_resid(a, w, scale, a_scale, c, gate, *, cfg: GemmConfig, m=None, stream=None):
    """In place on bf16 ``c`` [m][n]: c = bf16(c + bf16(gate[n] * bf16(dequantised acc)))."""
    m = _tokens(a, m)
    ops = _gemm_operands(cfg, m, a, w, scale, a_scale)
    out = _buf(c, "c", torch.bfloat16, m * cfg.n_size)
    g = _buf(gate, "gate", torch.float32, cfg.n_size)
    k = cfg.c()
    check(lib().k2w8_gemm_i8_resid(_stream(stream), ctypes.byref(k), m, *ops, out, g))


def gemm_i8_resid_256x256(a, w, scale, a_scale, c, gate, *, cfg: GemmConfig, m=None, stream=None):
    """The down projection's residual GEMM (same results as ``gemm_i8_resid``)."""
    m = _tokens(a, m)
    ops = _gemm_operands(cfg, m, a, w, scale, a_scale)
    out = _buf(c, "c", torch.bfloat16, m * cfg.n_size)
    g = _buf(gate, "gate", torch.float32, cfg.n_size)
    k = cfg.c()
    check(lib().k2w8_gemm_i8_resid_256x256(_stream(stream), ctypes.byref(k), m, *ops, out, g))


def gemm_i8_swiglu(a, w, scale, a_scale, c, *, cfg: GemmConfig, m=None, stream=None):
    """c f16 [m][n/2] = silu(gate) * up over 16-row interleaved gate|up weight rows."""
    m = _tokens(a, m)
    ops = _gemm_operands(cfg, m, a, w, scale, a_scale)
    out = _buf(c, "c", torch.float16, m * (cfg.n_size // 2))
    k = cfg.c()
    check(lib().k2w8_gemm_i8_swiglu(_stream(stream), ctypes.byref(k), m, *ops, out))


def gemm_i8_bias(a, w, scale, a_scale, bias, c, *, cfg: GemmConfig, m=None, stream=None):
    """Plain GEMM with an f16 bias before the bf16 boundary (no reference counterpart)."""
    m = _tokens(a, m)
    ops = _gemm_operands(cfg, m, a, w, scale, a_scale)
    b = _buf(bias, "bias", torch.float16, cfg.n_size)
    out = _buf(c, "c", torch.float16, m * cfg.n_size)
    k = cfg.c()
    check(lib().k2w8_gemm_i8_bias(_stream(stream), ctypes.byref(k), m, *ops, b, out))


def gemm_i8_acc(a, w, acc, *, cfg: GemmConfig, m=None, stream=None):
    """acc int32 [m][n] = exact integer a.w^T, no epilogue (no reference counterpart)."""
    m = _tokens(a, m)
    pa = _buf(a, "a", torch.int8, (m - 1) * cfg.k_stride + cfg.k_size)
    pw = _buf(w, "w", torch.int8, (cfg.n_size - 1) * cfg.k_stride + cfg.k_size)
    out = _buf(acc, "acc", torch.int32, m * cfg.n_size)
    k = cfg.c()
    check(lib().k2w8_gemm_i8_acc(_stream(stream), ctypes.byref(k), m, pa, pw, out))


def linear_norm_i8(h, norm_scale, mod_scale, mod_shift, q, q_scale, w, scale, c, *,
                   cfg: "GemmConfig", eps, tokens=None, stream=None):
    """prepare_norm_i8 of ``h`` into ``q``/``q_scale``, then gemm_i8 of ``q`` with ``w``
    into ``c``, as one call (one persistent launch for the wide-tile shapes). The
    prepare's width and out_stride are the GEMM config's k_size and k_stride."""
    n = _tokens(h, tokens)
    width, out_stride = cfg.k_size, cfg.k_stride
    pc = PrepareNormCfg(width, out_stride, eps)
    args = (
        _buf(h, "h", torch.bfloat16, n * width),
        _buf(norm_scale, "norm_scale", torch.float32, width),
        _buf(mod_scale, "mod_scale", torch.float32, width),
        _buf(mod_shift, "mod_shift", torch.float32, width),
        _buf(q, "q", torch.int8, (n - 1) * out_stride + width),
        _buf(q_scale, "q_scale", torch.float32, n),
        _buf(w, "w", torch.int8, (cfg.n_size - 1) * cfg.k_stride + cfg.k_size),
        _buf(scale, "scale", torch.float32, cfg.n_size),
        _buf(c, "c", torch.float16, n * cfg.n_size),
    )
    k = cfg.c()
    check(lib().k2w8_linear_norm_i8(_stream(stream), ctypes.byref(pc), ctypes.byref(k), n, *args))


def linear_plain_i8(h, q, q_scale, w, scale, c, *, cfg: "GemmConfig", tokens=None, stream=None):
    """prepare_plain_i8 of f16 ``h`` into ``q``/``q_scale``, then gemm_i8 into ``c``, as
    one call (one persistent launch for the wide-tile shapes)."""
    n = _tokens(h, tokens)
    width, out_stride = cfg.k_size, cfg.k_stride
    pc = PreparePlainCfg(width, out_stride)
    args = (
        _buf(h, "h", torch.float16, n * width),
        _buf(q, "q", torch.int8, (n - 1) * out_stride + width),
        _buf(q_scale, "q_scale", torch.float32, n),
        _buf(w, "w", torch.int8, (cfg.n_size - 1) * cfg.k_stride + cfg.k_size),
        _buf(scale, "scale", torch.float32, cfg.n_size),
        _buf(c, "c", torch.float16, n * cfg.n_size),
    )
    k = cfg.c()
    check(lib().k2w8_linear_plain_i8(_stream(stream), ctypes.byref(pc), ctypes.byref(k), n, *args))


def linear_gated_resid_i8(attn, gate_in, q, q_scale, w, scale, x, gate, *, cfg: "GemmConfig",
                          gate_stride, tokens=None, stream=None):
    """prepare_gated_i8 of ``attn`` x sigmoid(``gate_in``) into ``q``/``q_scale``, then
    gemm_i8_resid of ``q`` with ``w`` into the bf16 residual ``x`` (per-channel ``gate``),
    as one call: the block's attention output projection."""
    n = _tokens(attn, tokens)
    width, out_stride = cfg.k_size, cfg.k_stride
    pc = PrepareGatedCfg(width, out_stride, gate_stride)
    args = (
        _buf(attn, "attn", torch.float16, n * width),
        _buf(gate_in, "gate_in", torch.float16, (n - 1) * gate_stride + width),
        _buf(q, "q", torch.int8, (n - 1) * out_stride + width),
        _buf(q_scale, "q_scale", torch.float32, n),
        _buf(w, "w", torch.int8, (cfg.n_size - 1) * cfg.k_stride + cfg.k_size),
        _buf(scale, "scale", torch.float32, cfg.n_size),
        _buf(x, "x", torch.bfloat16, n * cfg.n_size),
        _buf(gate, "gate", torch.float32, cfg.n_size),
    )
    k = cfg.c()
    check(lib().k2w8_linear_gated_resid_i8(_stream(stream), ctypes.byref(pc), ctypes.byref(k), n, *args))


def linear_norm_swiglu_i8(h, norm_scale, mod_scale, mod_shift, q, q_scale, w, scale, c, *,
                          cfg: "GemmConfig", eps, tokens=None, stream=None):
    """prepare_norm_i8 of ``h`` into ``q``/``q_scale``, then gemm_i8_swiglu into ``c``
    (f16 [tokens][n/2]), as one call: the block's gate|up projection."""
    n = _tokens(h, tokens)
    width, out_stride = cfg.k_size, cfg.k_stride
    pc = PrepareNormCfg(width, out_stride, eps)
    args = (
        _buf(h, "h", torch.bfloat16, n * width),
        _buf(norm_scale, "norm_scale", torch.float32, width),
        _buf(mod_scale, "mod_scale", torch.float32, width),
        _buf(mod_shift, "mod_shift", torch.float32, width),
        _buf(q, "q", torch.int8, (n - 1) * out_stride + width),
        _buf(q_scale, "q_scale", torch.float32, n),
        _buf(w, "w", torch.int8, (cfg.n_size - 1) * cfg.k_stride + cfg.k_size),
        _buf(scale, "scale", torch.float32, cfg.n_size),
        _buf(c, "c", torch.float16, n * (cfg.n_size // 2)),
    )
    k = cfg.c()
    check(lib().k2w8_linear_norm_swiglu_i8(_stream(stream), ctypes.byref(pc), ctypes.byref(k), n, *args))


def linear_plain_resid_i8(h, q, q_scale, w, scale, x, gate, *, cfg: "GemmConfig", tokens=None,
                          stream=None):
    """prepare_plain_i8 of f16 ``h`` into ``q``/``q_scale``, then gemm_i8_resid into the
    bf16 residual ``x`` (per-channel ``gate``), as one call: the block's down projection."""
    n = _tokens(h, tokens)
    width, out_stride = cfg.k_size, cfg.k_stride
    pc = PreparePlainCfg(width, out_stride)
    args = (
        _buf(h, "h", torch.float16, n * width),
        _buf(q, "q", torch.int8, (n - 1) * out_stride + width),
        _buf(q_scale, "q_scale", torch.float32, n),
        _buf(w, "w", torch.int8, (cfg.n_size - 1) * cfg.k_stride + cfg.k_size),
        _buf(scale, "scale", torch.float32, cfg.n_size),
        _buf(x, "x", torch.bfloat16, n * cfg.n_size),
        _buf(gate, "gate", torch.float32, cfg.n_size),
    )
    k = cfg.c()
    check(lib().k2w8_linear_plain_resid_i8(_stream(stream), ctypes.byref(pc), ctypes.byref(k), n, *args))


def gemm_set_workspace(workspace, *, stream=None):
    """Hand the GEMMs on ``stream`` (default: torch's current stream) a caller-owned
    split-K workspace (a device tensor; its bytes are used, its dtype is not), or remove
    the registration with ``None``. The caller keeps the tensor alive while it is
    registered and while enqueued work may use it."""
    if workspace is None:
        check(lib().k2w8_gemm_set_workspace(_stream(stream), None, 0))
        return
    if not workspace.is_cuda or not workspace.is_contiguous():
        raise InvalidArgument("workspace must be a contiguous device tensor")
    nbytes = workspace.numel() * workspace.element_size()
    check(lib().k2w8_gemm_set_workspace(_stream(stream), ctypes.c_void_p(workspace.data_ptr()),
                                        nbytes))


def gemm_workspace_bytes() -> int:
    """Size of the split-K workspace the library allocates per stream."""
    return int(lib().k2w8_gemm_workspace_bytes())


def lora_transport(x, out, *, reverse: int, count=None, stream=None):
    """The 16-bit format change of kernels/native/lora_transport.loom: ``reverse`` 1 turns
    bf16 ``x`` into f16 ``out``, 2 turns f16 into bf16 (round to nearest even)."""
    src, dst = (torch.bfloat16, torch.float16) if reverse == 1 else (torch.float16, torch.bfloat16)
    n = int(x.numel()) if count is None else int(count)
    px = _buf(x, "x", src, n)
    po = _buf(out, "out", dst, n)
    check(lib().k2w8_lora_transport(_stream(stream), int(reverse), n, px, po))


def sigmoid_f32(x, out, *, count=None, stream=None):
    """The device sigmoid 1 / (1 + exp(-x)) of the gated prepare and the SwiGLU epilogue,
    elementwise over f32 ``x`` into ``out`` (a check of the kernels' numerics)."""
    n = int(x.numel()) if count is None else int(count)
    px = _buf(x, "x", torch.float32, n)
    po = _buf(out, "out", torch.float32, n)
    check(lib().k2w8_sigmoid_f32(_stream(stream), n, px, po))


def rope_qknorm_f16(qkv, q_scale, k_scale, cos, sin, q_out, k_out, v_out, *, row_stride,
                    q_heads, kv_heads, k_offset, eps, tokens=None, stream=None):
    """Per-head RMSNorm (multiplier 1 + scale) and rotary embedding of q and k, v copied.

    ``qkv`` f16 [tokens][row_stride]; ``q_scale``/``k_scale`` f32 [128]; ``cos``/``sin``
    f32 [tokens][128]; ``q_out`` f16 [tokens][q_heads*128]; ``k_out``/``v_out`` f16
    [tokens][kv_heads*128].
    """
    n = _tokens(qkv, tokens)
    cfg = RopeQknormCfg(row_stride, q_heads, kv_heads, k_offset, eps)
    args = (
        _buf(qkv, "qkv", torch.float16, n * row_stride),
        _buf(q_scale, "q_scale", torch.float32, 128),
        _buf(k_scale, "k_scale", torch.float32, 128),
        _buf(cos, "cos", torch.float32, n * 128),
        _buf(sin, "sin", torch.float32, n * 128),
        _buf(q_out, "q_out", torch.float16, n * q_heads * 128),
        _buf(k_out, "k_out", torch.float16, n * kv_heads * 128),
        _buf(v_out, "v_out", torch.float16, n * kv_heads * 128),
    )
    check(lib().k2w8_rope_qknorm_f16(_stream(stream), ctypes.byref(cfg), n, *args))


def v_transpose(x, out, *, width, row_capacity, rows=None, stream=None):
    """f16 ``x`` [rows][width] -> ``out`` [width][row_capacity]; columns past ``rows``
    are left as they are."""
    n = _tokens(x, rows)
    cfg = VTransposeCfg(width, row_capacity)
    args = (
        _buf(x, "x", torch.float16, n * width),
        _buf(out, "out", torch.float16, width * row_capacity),
    )
    check(lib().k2w8_v_transpose(_stream(stream), ctypes.byref(cfg), n, *args))


def attention_f16(q, k, v, out, *, q_stride, kv_stride, out_stride, tokens, token_capacity, scale,
                  kv_heads, token_count=None, group=4, stream=None):
    """Grouped-query attention over ``tokens`` keys, ``group`` query heads per key-value
    head (4 as in the reference kernel; 1 and 2 are an extension).

    ``q`` f16 [token_capacity][q_stride]; ``k`` f16 [token_capacity][kv_stride]; ``v`` is
    V^T, f16 [kv_stride][token_capacity]; ``out`` f16 [token_count][out_stride].
    """
    n = int(tokens) if token_count is None else int(token_count)
    cfg = AttentionCfg(q_stride, kv_stride, out_stride, tokens, token_capacity, scale)
    args = (
        _buf(q, "q", torch.float16, token_capacity * q_stride),
        _buf(k, "k", torch.float16, token_capacity * kv_stride),
        _buf(v, "v", torch.float16, kv_stride * token_capacity),
        _buf(out, "out", torch.float16, n * out_stride),
    )
    if group == 4:
        check(lib().k2w8_attention_f16(_stream(stream), ctypes.byref(cfg), n, int(kv_heads), *args))
    else:
        check(lib().k2w8_attention_f16_grouped(_stream(stream), ctypes.byref(cfg), n, int(kv_heads),
                                               int(group), *args))


@dataclass(frozen=True)
class Quantized:
    """A ConvRot projection on the device (src/training/quantized.rs:8-49): int8 weight
    rows at ``pitch`` = ``shape.gemm_pitch(inputs)`` and their f32 scales."""

    weight: torch.Tensor  # int8 [outputs][pitch]
    scales: torch.Tensor  # f32 [outputs]
    inputs: int
    outputs: int

    @property
    def pitch(self) -> int:
        return int(lib().k2w8_shape_gemm_pitch(self.inputs))

    @staticmethod
    def load(weight_rows: torch.Tensor, scales: torch.Tensor) -> "Quantized":
        """Upload int8 [outputs][inputs] rows and f32 [outputs] scales at the GEMM pitch
        (:17-49): the padding past each row stays zero."""
        outputs, inputs = int(weight_rows.shape[0]), int(weight_rows.shape[1])
        pitch = int(lib().k2w8_shape_gemm_pitch(inputs))
        w = torch.zeros((outputs, pitch), dtype=torch.int8, device="cuda")
        w[:, :inputs].copy_(weight_rows)
        s = scales.to(device="cuda", dtype=torch.float32).contiguous()
        return Quantized(w, s, inputs, outputs)

    def forward(self, x: torch.Tensor, stream=None) -> torch.Tensor:
        """bf16 [rows][inputs] -> bf16 [rows][outputs] (:51-112), workspaces from torch."""
        if x.dim() != 2 or int(x.shape[1]) != self.inputs:
            raise InvalidArgument("ConvRot projection dimensions")
        rows = int(x.shape[0])
        transport = torch.empty(rows * self.inputs, dtype=torch.float16, device="cuda")
        quantized = torch.empty((rows, self.pitch), dtype=torch.int8, device="cuda")
        q_scales = torch.empty(rows, dtype=torch.float32, device="cuda")
        out_f16 = torch.empty((rows, self.outputs), dtype=torch.float16, device="cuda")
        out = torch.empty((rows, self.outputs), dtype=torch.bfloat16, device="cuda")
        cfg = QuantizedCfg(self.inputs, self.outputs, self.pitch)
        args = (
            _buf(x, "x", torch.bfloat16, rows * self.inputs),
            _buf(self.weight, "weight", torch.int8, (self.outputs - 1) * self.pitch + self.inputs),
            _buf(self.scales, "scales", torch.float32, self.outputs),
            _buf(transport, "transport", torch.float16, rows * self.inputs),
            _buf(quantized, "quantized", torch.int8, (rows - 1) * self.pitch + self.inputs),
            _buf(q_scales, "q_scales", torch.float32, rows),
            _buf(out_f16, "out_f16", torch.float16, rows * self.outputs),
            _buf(out, "out", torch.bfloat16, rows * self.outputs),
        )
        check(lib().k2w8_quantized_forward(_stream(stream), ctypes.byref(cfg), rows, *args))
        return out


_EPILOGUES = {"plain": 0, "resid": 1, "swiglu": 2, "bias": 3, "acc": 4}
_KERNELS = {-1: "refused", 0: "few-token", 1: "tile", 2: "tile+tail", 3: "split-k"}


def gemm_choose(m, *, cfg: GemmConfig, epilogue="plain", cus=256, workspace_bytes=None,
                workspace_required=False) -> dict:
    """Which kernel the GEMM entry points run for ``m`` tokens with ``cfg`` on a device of
    ``cus`` compute units (no launch): ``kernel`` (few-token, tile, tile+tail, split-k,
    or refused), the workgroup ``tile`` (m, n), its LDS ``stages``, ``n_big``
    (tile+tail) and ``splits`` / ``split_steps`` (split-k).

    ``workspace_bytes`` defaults to the library's own per-stream workspace, which an
    eager call has; a call captured into a graph without a registered or installed
    workspace has none (pass 0 for it). ``workspace_required`` describes a call whose
    workspace is fixed (``gemm_i8_noalloc``'s static scratch): a shape it refuses is
    reported as ``refused``."""
    if workspace_bytes is None:
        workspace_bytes = int(lib().k2w8_gemm_workspace_bytes())
    out = GemmChoice()
    k = cfg.c()
    check(lib().k2w8_gemm_choose(_EPILOGUES[epilogue], m, ctypes.byref(k), cus, workspace_bytes,
                                 1 if workspace_required else 0, ctypes.byref(out)))
    res = {"kernel": _KERNELS[out.kernel]}
    if out.kernel > 0:
        res.update(tile=(out.tile_m, out.tile_n), stages=out.stages)
    if out.kernel == 2:
        res["n_big"] = out.n_big
    if out.kernel == 3:
        res.update(splits=out.splits, split_steps=out.split_steps)
    return res


def probe_mfma_i8(out, *, blocks, iters, random=True, seed=1, stream=None):
    """The MFMA-only INT8 rate probe (a measurement aid, not part of the path):
    ``blocks`` workgroups of four waves run ``iters`` steps of eight back-to-back
    v_mfma_i32_32x32x32_i8 per wave (2^21 * blocks * iters ops) on register operands,
    pseudo-random bytes or bytes of 1. ``out`` int32 [blocks * 256]."""
    o = _buf(out, "out", torch.int32, blocks * 256)
    check(lib().k2w8_probe_mfma_i8(_stream(stream), blocks, iters, 1 if random else 0, seed, o))
