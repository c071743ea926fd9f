"""Checkpoint upload: the reference's `krea2::checkpoint::{Checkpoint, Plan}` and
`session::Weights` (src/checkpoint/file.rs, src/checkpoint/plan.rs,
src/session/weights.rs) over the C ABI. The reader, the layout and the upload are the
library's (k2w8_checkpoint.cpp); this module only owns the handles."""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from ._lib import SpanInfo, TensorInfo, check, lib

_NUMPY = {1: np.int8, 2: np.float32, 3: np.uint16, 4: np.uint16, 5: np.uint8, 6: np.int32}
DTYPES = {0: "other", 1: "I8", 2: "F32", 3: "BF16", 4: "F16", 5: "U8", 6: "I32"}


@dataclass(frozen=True)
class Tensor:
    """One tensor of a mapped checkpoint (file.rs:12-21). ``bytes`` copies it out."""

    dtype: str
    shape: tuple
    nbytes: int
    _data: int

    def numpy(self) -> np.ndarray:
        code = [k for k, v in DTYPES.items() if v == self.dtype][0]
        raw = ctypes.string_at(self._data, self.nbytes)
        return np.frombuffer(raw, dtype=_NUMPY.get(code, np.uint8)).reshape(self.shape)


class Checkpoint:
    """A memory-mapped ``.safetensors`` file (``Checkpoint::open``, file.rs:86-106)."""

    def __init__(self, path: str):
        handle = ctypes.c_void_p()
        check(lib().k2w8_checkpoint_open(str(path).encode(), ctypes.byref(handle)))
        self._h = handle
        self.path = str(path)

    def close(self) -> None:
        if self._h:
            lib().k2w8_checkpoint_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def block_count(self) -> int:
        return int(lib().k2w8_checkpoint_block_count(self._h))

    def get(self, name: str) -> Tensor:
        info = TensorInfo()
        check(lib().k2w8_checkpoint_tensor(self._h, name.encode(), ctypes.byref(info)))
        shape = tuple(int(info.shape[i]) for i in range(info.ndim))
        return Tensor(DTYPES.get(int(info.dtype), "other"), shape, int(info.nbytes), int(info.data or 0))


@dataclass(frozen=True)
class Span:
    """One destination of a plan (plan.rs:24-41)."""

    device_offset: int
    device_bytes: int
    rows: int
    row_bytes: int
    device_row_bytes: int
    file_bytes: int
    segments: int


class Plan:
    """``Plan::for_checkpoint`` (plan.rs:88-143)."""

    def __init__(self, checkpoint: Checkpoint):
        handle = ctypes.c_void_p()
        check(lib().k2w8_plan_for_checkpoint(checkpoint._h, ctypes.byref(handle)))
        self._h = handle
        self.checkpoint = checkpoint

    def __del__(self):
        try:
            if self._h:
                lib().k2w8_plan_free(self._h)
        except Exception:
            pass

    @property
    def total_bytes(self) -> int:
        return int(lib().k2w8_plan_total_bytes(self._h))

    @property
    def layers(self) -> int:
        return int(lib().k2w8_plan_layers(self._h))

    def names(self) -> list:
        n = int(lib().k2w8_plan_span_count(self._h))
        return [lib().k2w8_plan_span_name(self._h, i).decode() for i in range(n)]

    def span(self, name: str) -> Span:
        info = SpanInfo()
        check(lib().k2w8_plan_span(self._h, name.encode(), ctypes.byref(info)))
        return Span(*(int(getattr(info, f)) for f, _ in SpanInfo._fields_))

    def upload(self, stream=None) -> "Weights":
        """``Weights::upload`` (weights.rs:48-100) into one new device allocation."""
        storage = torch.empty(max(self.total_bytes, 1), dtype=torch.uint8, device="cuda")
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream if stream is None else stream)
        check(lib().k2w8_plan_upload(s, self._h, self.checkpoint._h,
                                     ctypes.c_void_p(storage.data_ptr()), storage.numel()))
        return Weights(self, storage)


@dataclass
class Weights:
    """A resident checkpoint: one allocation, views located by span name
    (weights.rs:103-126)."""

    plan: Plan
    storage: torch.Tensor

    def operand(self, name: str) -> torch.Tensor:
        """The GEMM rows of ``name`` (e.g. ``blocks.0.gu``): int8 [rows][pitch]."""
        sp = self.plan.span(f"{name}.q")
        raw = self.storage[sp.device_offset:sp.device_offset + sp.device_bytes]
        return raw.view(sp.rows, sp.device_row_bytes).view(torch.int8)

    def scales(self, name: str) -> torch.Tensor:
        sp = self.plan.span(f"{name}.s")
        return self.storage[sp.device_offset:sp.device_offset + sp.device_bytes].view(torch.float32)

    def vector(self, name: str) -> torch.Tensor:
        sp = self.plan.span(name)
        return self.storage[sp.device_offset:sp.device_offset + sp.device_bytes].view(torch.float32)
