"""Synthetic .safetensors checkpoints for the checkpoint-upload tests: the container
format written by hand (8-byte little-endian header length, JSON header, data), with the
reference's tensor naming (src/checkpoint/plan.rs:96-134)."""

from __future__ import annotations

import json
import struct

import numpy as np

_CODES = {np.dtype(np.int8): "I8", np.dtype(np.float32): "F32", np.dtype(np.uint16): "BF16",
          np.dtype(np.float16): "F16"}


def write_safetensors(path, tensors: dict, metadata=None) -> None:
    """tensors: name -> array (uint16 arrays are written as BF16)."""
    header, blobs, offset = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, arr in tensors.items():
        arr = np.ascontiguousarray(arr)
        raw = arr.tobytes()
        header[name] = {"dtype": _CODES[arr.dtype], "shape": list(arr.shape),
                        "data_offsets": [offset, offset + len(raw)]}
        blobs.append(raw)
        offset += len(raw)
    text = json.dumps(header).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for b in blobs:
            f.write(b)


def write_raw(path, header_text: str, payload: bytes, length=None) -> None:
    data = header_text.encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(data) if length is None else length))
        f.write(data)
        f.write(payload)


def block_tensors(rng, layers=2, hidden=256, kv=64, inter=8192, bf16_norms=False):
    """Per block: attn.wq/wk/wv/gate/wo, mlp.gate/up/down (int8 rows + f32 scales) and the
    four norm vectors."""
    t = {}

    def proj(name, rows, k):
        t[f"{name}.weight"] = rng.integers(-127, 128, (rows, k), dtype=np.int8)
        t[f"{name}.weight_scale"] = rng.uniform(1e-3, 1e-2, rows).astype(np.float32)

    for b in range(layers):
        p = f"blocks.{b}"
        proj(f"{p}.attn.wq", hidden, hidden)
        proj(f"{p}.attn.wk", kv, hidden)
        proj(f"{p}.attn.wv", kv, hidden)
        proj(f"{p}.attn.gate", hidden, hidden)
        proj(f"{p}.attn.wo", hidden, hidden)
        proj(f"{p}.mlp.gate", inter, hidden)
        proj(f"{p}.mlp.up", inter, hidden)
        proj(f"{p}.mlp.down", hidden, inter)
        for v, n in (("prenorm.scale", hidden), ("postnorm.scale", hidden),
                     ("attn.qknorm.qnorm.scale", 128), ("attn.qknorm.knorm.scale", 128)):
            x = rng.uniform(0.5, 1.5, n).astype(np.float32)
            if bf16_norms:
                x = (x.view(np.uint32) >> 16).astype(np.uint16)  # exact bf16 values
            t[f"{p}.{v}"] = x
    return t


def pitch(k: int) -> int:
    return k + 64 if k % 8192 == 0 else k


def expected_layout(t: dict, layers: int):
    """The device bytes of every span, built independently of the library:
    name -> (bytes, rows, pitch)."""
    out = {}

    def rows_at_pitch(rows):
        k = rows.shape[1]
        buf = np.zeros((rows.shape[0], pitch(k)), np.int8)
        buf[:, :k] = rows
        return buf

    for b in range(layers):
        p = f"blocks.{b}"
        parts = [f"{p}.attn.{n}" for n in ("wq", "wk", "wv", "gate")]
        out[f"{p}.qkvg.q"] = rows_at_pitch(np.concatenate([t[f"{x}.weight"] for x in parts]))
        out[f"{p}.qkvg.s"] = np.concatenate([t[f"{x}.weight_scale"] for x in parts])
        for o, x in (("wo", f"{p}.attn.wo"), ("down", f"{p}.mlp.down")):
            out[f"{p}.{o}.q"] = rows_at_pitch(t[f"{x}.weight"])
            out[f"{p}.{o}.s"] = t[f"{x}.weight_scale"]
        g, u = t[f"{p}.mlp.gate.weight"], t[f"{p}.mlp.up.weight"]
        gs, us = t[f"{p}.mlp.gate.weight_scale"], t[f"{p}.mlp.up.weight_scale"]
        groups = g.shape[0] // 16
        rows = np.stack([g.reshape(groups, 16, -1), u.reshape(groups, 16, -1)], 1)
        out[f"{p}.gu.q"] = rows_at_pitch(rows.reshape(2 * g.shape[0], -1))
        out[f"{p}.gu.s"] = np.stack([gs.reshape(groups, 16), us.reshape(groups, 16)], 1).reshape(-1)
        for o, v in (("prenorm", "prenorm.scale"), ("postnorm", "postnorm.scale"),
                     ("qnorm", "attn.qknorm.qnorm.scale"), ("knorm", "attn.qknorm.knorm.scale")):
            x = t[f"{p}.{v}"]
            if x.dtype == np.uint16:
                x = (x.astype(np.uint32) << 16).view(np.float32)
            out[f"{p}.{o}"] = x
    return out
