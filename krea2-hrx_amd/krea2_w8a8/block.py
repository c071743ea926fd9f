"""The W8A8 stages of the reference's transformer block, over a session's fixed buffers:
``krea2::session::Session`` (src/session/mod.rs) restricted to this path. The kernels,
the stage order and the graph recording are the library's (k2w8_block.cpp); this class
owns the workspaces (allocated once, at the session's token count, as the reference's
session does) and hands their addresses to the C ABI."""

from __future__ import annotations

import ctypes

import torch

from ._lib import BlockBuffers, BlockCfg, BlockWeights, check, lib


def _p(t: torch.Tensor) -> int:
    return t.data_ptr()


class BlockSession:
    """``layers`` blocks at ``tokens`` rows. ``weights[i]`` holds block i's operands as
    device tensors: qkvg_q/qkvg_s, wo_q/wo_s, gu_q/gu_s, down_q/down_s (int8 rows at the
    GEMM pitch, f32 scales), the prenorm/postnorm f32 vectors and, for the attention
    step, the qnorm/knorm f32 [128] vectors.

    With ``attention`` the session also owns the attention step's workspaces (q, k, v,
    V^T with zero headroom; cos/sin, which the caller fills) and every block runs the
    whole sequence of src/session/mod.rs:671-840; without it the caller runs its own
    attention between ``pre_attention`` and ``post_attention``."""

    def __init__(self, weights, *, tokens, hidden, inter, qkvg, gate_offset, eps=1e-5,
                 attention=False, stream: torch.cuda.Stream | None = None):
        self.layers = len(weights)
        self.cfg = BlockCfg(tokens, hidden, inter, qkvg, gate_offset, eps)
        self.stream = stream or torch.cuda.Stream()  # a created stream: graphs record from it
        pitch = max(int(lib().k2w8_shape_gemm_pitch(hidden)), int(lib().k2w8_shape_gemm_pitch(inter)))
        dev = "cuda"
        self.x = torch.zeros((tokens, hidden), dtype=torch.bfloat16, device=dev)
        self.a_q = torch.zeros((tokens, pitch), dtype=torch.int8, device=dev)
        self.a_s = torch.zeros(tokens, dtype=torch.float32, device=dev)
        self.fused = torch.zeros((tokens, qkvg), dtype=torch.float16, device=dev)
        self.attn_gu = torch.zeros(tokens * max(hidden, inter), dtype=torch.float16, device=dev)
        self.mods = torch.zeros((self.layers, 6, hidden), dtype=torch.float32, device=dev)
        self.attention = attention
        att = [0] * 6
        if attention:
            cap = int(lib().k2w8_shape_capacity(tokens))
            kv = (gate_offset - hidden) // 2
            self.q = torch.zeros((cap, hidden), dtype=torch.float16, device=dev)
            self.k = torch.zeros((cap, kv), dtype=torch.float16, device=dev)
            self.v = torch.zeros((cap, kv), dtype=torch.float16, device=dev)
            self.vt = torch.zeros((kv, cap), dtype=torch.float16, device=dev)
            self.cos = torch.ones((tokens, 128), dtype=torch.float32, device=dev)
            self.sin = torch.zeros((tokens, 128), dtype=torch.float32, device=dev)
            att = [_p(t) for t in (self.q, self.k, self.v, self.vt, self.cos, self.sin)]
        self._weights = weights  # keep the operands alive
        keys = [f for f, _ in BlockWeights._fields_]
        self._w = (BlockWeights * self.layers)(
            *[BlockWeights(*[_p(w[k]) if k in w else 0 for k in keys]) for w in weights])
        self._b = BlockBuffers(_p(self.x), _p(self.a_q), _p(self.a_s), _p(self.fused),
                               _p(self.attn_gu), _p(self.mods), *att)
        self._graph = ctypes.c_void_p()

    @staticmethod
    def from_checkpoint(uploaded, **shape):
        """A session over an uploaded checkpoint (``checkpoint.Weights``)."""
        layers = uploaded.plan.layers
        weights = []
        for i in range(layers):
            p = f"blocks.{i}"
            weights.append({
                "qkvg_q": uploaded.operand(f"{p}.qkvg"), "qkvg_s": uploaded.scales(f"{p}.qkvg"),
                "wo_q": uploaded.operand(f"{p}.wo"), "wo_s": uploaded.scales(f"{p}.wo"),
                "gu_q": uploaded.operand(f"{p}.gu"), "gu_s": uploaded.scales(f"{p}.gu"),
                "down_q": uploaded.operand(f"{p}.down"), "down_s": uploaded.scales(f"{p}.down"),
                "prenorm": uploaded.vector(f"{p}.prenorm"),
                "postnorm": uploaded.vector(f"{p}.postnorm"),
                "qnorm": uploaded.vector(f"{p}.qnorm"),
                "knorm": uploaded.vector(f"{p}.knorm"),
            })
        return BlockSession(weights, **shape)

    def _s(self):
        return ctypes.c_void_p(self.stream.cuda_stream)

    def pre_attention(self, index: int) -> None:
        check(lib().k2w8_block_pre_attention(self._s(), ctypes.byref(self.cfg), index,
                                             ctypes.byref(self._w[index]), ctypes.byref(self._b)))

    def attention_step(self, index: int) -> None:
        """q/k norm + rope, V transpose and f16 attention into attn_gu (needs
        ``attention``)."""
        check(lib().k2w8_block_attention(self._s(), ctypes.byref(self.cfg), index,
                                         ctypes.byref(self._w[index]), ctypes.byref(self._b)))

    def post_attention(self, index: int) -> None:
        check(lib().k2w8_block_post_attention(self._s(), ctypes.byref(self.cfg), index,
                                              ctypes.byref(self._w[index]), ctypes.byref(self._b)))

    def run(self) -> None:
        """Every block eagerly on the session stream. Without ``attention`` the
        post-attention stages read whatever attn_gu holds."""
        for i in range(self.layers):
            self.pre_attention(i)
            if self.attention:
                self.attention_step(i)
            self.post_attention(i)

    def record(self) -> None:
        """Record the block loop once (src/session/mod.rs:596-616)."""
        if self._graph:
            return
        handle = ctypes.c_void_p()
        check(lib().k2w8_blocks_record(self._s(), ctypes.byref(self.cfg), self.layers, self._w,
                                       ctypes.byref(self._b), ctypes.byref(handle)))
        self._graph = handle

    def replay(self) -> None:
        self.record()
        check(lib().k2w8_graph_launch(self._s(), self._graph))

    def profile(self) -> dict:
        """Microseconds per stage over one eager pass (src/session/mod.rs:449-479)."""
        n = int(lib().k2w8_block_stage_count())
        out = (ctypes.c_double * n)()
        check(lib().k2w8_blocks_profile(self._s(), ctypes.byref(self.cfg), self.layers, self._w,
                                        ctypes.byref(self._b), out, n))
        stages: dict = {}
        for k in range(n):
            if out[k] < 0:  # a stage this session does not run
                continue
            label = lib().k2w8_block_stage_label(k).decode()
            stages[label] = stages.get(label, 0.0) + out[k]
        return stages

    def __del__(self):
        try:
            if self._graph:
                lib().k2w8_graph_free(self._graph)
        except Exception:
            pass
