"""Shared helpers of the GPU parity tests: seeded inputs, host<->device moves."""

from __future__ import annotations

import numpy as np
import torch

import krea2_w8a8 as k2

DEV = "cuda"
PAD = -91  # 0xa5: bytes a prepare must not write


def dev(x: np.ndarray, dtype=None) -> torch.Tensor:
    """numpy -> device tensor; uint16 arrays travel as int16 and are reinterpreted."""
    x = np.ascontiguousarray(x)
    if x.dtype == np.uint16:
        t = torch.from_numpy(x.view(np.int16)).to(DEV)
        return t.view(dtype) if dtype is not None else t
    return torch.from_numpy(x).to(DEV)


def host(t: torch.Tensor) -> np.ndarray:
    """device tensor -> numpy; 16-bit floats come back as uint16 bit patterns."""
    t = t.detach()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def activations(rng, tokens, width, outliers=8, scale=1.0):
    """N(0,1) rows with `outliers` seeded channels scaled x20, as f32."""
    x = rng.standard_normal((tokens, width), dtype=np.float32) * np.float32(scale)
    if outliers:
        ch = rng.choice(width, size=min(outliers, width), replace=False)
        x[:, ch] *= np.float32(20.0)
    return x


def f16_bits(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def bf16_bits(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_value(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def int8_weights(rng, rows, k, pitch=None):
    pitch = pitch or k
    w = np.zeros((rows, pitch), np.int8)
    w[:, :k] = rng.integers(-127, 128, (rows, k), dtype=np.int8)
    return w


def channel_scales(rng, n):
    return rng.uniform(1e-3, 1e-2, n).astype(np.float32)


def sync():
    torch.cuda.synchronize()


__all__ = ["k2", "dev", "host", "activations", "f16_bits", "bf16_bits", "bf16_value",
           "int8_weights", "channel_scales", "sync", "PAD", "DEV"]
